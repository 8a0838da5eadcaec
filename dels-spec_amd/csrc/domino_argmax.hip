// Domino correction step: f(z + s) . fc2^T (+ fc2 bias), scaled by the
// guidance alpha, plus the base logits, then the vocabulary argmax -- the
// fused kernel of the Domino runner (code/kernel/domino.py:58-173: its
// _fused_mlp_bias_argmax_kernel and _reduce_argmax_kernel in one launch; f is
// SiLU there, and any of the middle layers of DELS_MIDDLE_* here, which the
// reference runs as its unfused step, 404-431).
//
// For row m (< 16 per row group) and vocabulary index v:
//     mid[m, k] = f(p),  p = fp32(z[m, k]) + fp32(s[m, k])                (fp32, never rounded)
//                 (SiLU: p * sigmoid(p))
//     dot[m, v] = sum_k fp32(fc2[v, k]) * mid[m, k]                       (fp32 accumulate)
//     score     = fma(dot (+ bias[v]), alpha, base[m, v])
// and per row the lowest v attaining the maximum.
//
// mid stays fp32 in the reference, but the matrix cores take bf16 operands,
// so each value is split into two bf16 parts, hi = bf16(mid) and
// lo = bf16(mid - hi) (|mid - hi - lo| <= 2^-17 |mid|), and every K step runs
// two v_mfma_f32_16x16x32_bf16 on the same fc2 operand: the products are exact
// in fp32, so the dot is that of mid to within 2^-17 relative per term -- well
// inside the fp32 accumulation-order freedom the reference already has.
//
// Each workgroup builds the hi/lo operands of its 16 rows in LDS (64 * E bytes,
// E <= 2048; rows past M are zero), then its four waves stream 16-row tiles of
// fc2 (MFMA-16 block layout, one contiguous KiB per K step) through two
// register sets of up to 16 K steps, walking (tile, K chunk) units so any E
// streams with the same register budget.  The cross-workgroup argmax is the
// GEMV kernel's (argmax_wg_finish).
#include <algorithm>
#include <climits>
#include <mutex>

#include "../../include/dels.h"
#include "dels_device.h"
#include "dels_internal.h"
#include "fused_argmax_gemv.h"

namespace dels {

namespace {

constexpr int kDomKC = 16;   // K steps (of 32) per register set

// The middle layer f of the correction MLP in fp32 (DELS_MIDDLE_*; `middle` is
// uniform over the launch).  GELU is x/2 (1 + erf(x / sqrt 2)) and its tanh
// form x/2 (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), as nn.GELU defines them.
template <int MIDDLE>
__device__ __forceinline__ float domino_middle(float p) {
#pragma clang fp contract(off)
    if constexpr (MIDDLE == DELS_MIDDLE_IDENTITY) return p;
    else if constexpr (MIDDLE == DELS_MIDDLE_RELU) return p > 0.f ? p : (p == p ? 0.f : p);
    else if constexpr (MIDDLE == DELS_MIDDLE_GELU) return 0.5f * p * (1.f + erff(p * 0.70710678118654752f));
    else if constexpr (MIDDLE == DELS_MIDDLE_GELU_TANH)
        return 0.5f * p * (1.f + tanhf(0.79788456080286536f * (p + 0.044715f * (p * p * p))));
    else if constexpr (MIDDLE == DELS_MIDDLE_TANH) return tanhf(p);
    else if constexpr (MIDDLE == DELS_MIDDLE_SIGMOID) return sigmoid_f32(p);
    else return p * sigmoid_f32(p);   // DELS_MIDDLE_SILU
}

// mid = f(z + s) of the 16 rows m0 .. m0 + 15 into the hi/lo operand layout in
// LDS (see the kernel); one loop per middle layer, so none carries a branch on it.
template <int MIDDLE>
__device__ __forceinline__ void domino_fill_operands(const DominoArgs& a, int m0, int kpad, uint16_t* ops) {
#pragma clang fp contract(off)
    for (int i = threadIdx.x; i < 16 * kpad; i += 256) {
        const int row = i / kpad, k = i - row * kpad;
        const int m = m0 + row;
        float mid = 0.f;
        if (m < a.M && k < a.E) {
            const float p = bf16_bits_to_f32(a.z[(int64_t)m * a.ldz + k]) + bf16_bits_to_f32(a.s[(int64_t)m * a.lds + k]);
            mid = domino_middle<MIDDLE>(p);
        }
        const uint16_t hi = f32_to_bf16_bits(mid);
        const uint16_t lo = f32_to_bf16_bits(mid - bf16_bits_to_f32(hi));
        const int ks = k >> 5, ln = row + 16 * ((k & 31) >> 3), e = k & 7;
        ops[((ks * 2 + 0) * 64 + ln) * 8 + e] = hi;
        ops[((ks * 2 + 1) * 64 + ln) * 8 + e] = lo;
    }
}

template <typename BaseT, typename BiasT>
struct DomRegs {
    bf16x8 b[kDomKC];
    uint32_t base[4];   // as loaded (load_raw), widened at use
    uint32_t bias;
};

template <typename BaseT, typename BiasT>
__global__ __launch_bounds__(256) void domino_argmax_kernel(DominoArgs a, ArgmaxKArgs fin) {
#pragma clang fp contract(off)
    extern __shared__ __attribute__((aligned(16))) char dyn_lds[];   // [ksteps][2][64 lanes][16 bytes]
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15;
    const int kg = lane >> 4;
    const int m0 = blockIdx.y * 16;
    const int ksteps = a.E / 32;

    // mid = f(z + s) of the 16 rows, split into bf16 hi/lo A operands: K step
    // ks, part p (0 hi, 1 lo) is the KiB at ((ks * 2 + p) * 64 + lane) * 16 with
    // lane = row + 16 * (k % 32 / 8), element k % 8.  K is padded with zeros to
    // whole register sets (and rows past M are zero), so the contraction below
    // runs every step of a set unconditionally: padded steps multiply zeros.
    uint16_t* ops = reinterpret_cast<uint16_t*>(dyn_lds);
    const int kpad = ((ksteps + kDomKC - 1) / kDomKC) * kDomKC * 32;
    switch (a.middle) {   // uniform
        case DELS_MIDDLE_IDENTITY: domino_fill_operands<DELS_MIDDLE_IDENTITY>(a, m0, kpad, ops); break;
        case DELS_MIDDLE_RELU: domino_fill_operands<DELS_MIDDLE_RELU>(a, m0, kpad, ops); break;
        case DELS_MIDDLE_GELU: domino_fill_operands<DELS_MIDDLE_GELU>(a, m0, kpad, ops); break;
        case DELS_MIDDLE_GELU_TANH: domino_fill_operands<DELS_MIDDLE_GELU_TANH>(a, m0, kpad, ops); break;
        case DELS_MIDDLE_TANH: domino_fill_operands<DELS_MIDDLE_TANH>(a, m0, kpad, ops); break;
        case DELS_MIDDLE_SIGMOID: domino_fill_operands<DELS_MIDDLE_SIGMOID>(a, m0, kpad, ops); break;
        default: domino_fill_operands<DELS_MIDDLE_SILU>(a, m0, kpad, ops); break;
    }
    __syncthreads();

    float al[4], best[4];
    int bidx[4];
    const BaseT* brow[4];
    const BaseT* base = static_cast<const BaseT*>(a.base);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int m = m0 + 4 * kg + q;
        const bool mok = m < a.M;
        al[q] = a.alpha;
        brow[q] = base + (int64_t)(mok ? m : 0) * a.ldbase;
        best[q] = -__builtin_inff();
        bidx[q] = INT_MAX;
    }

    const int ntiles = (a.V + 15) >> 4;
    const int nch = (ksteps + kDomKC - 1) / kDomKC;
    const int nwaves = gridDim.x * 4;
    const int t0 = blockIdx.x * 4 + wave;
    const int cnt = t0 < ntiles ? (ntiles - 1 - t0) / nwaves + 1 : 0;
    const int units = cnt * nch;
    const BiasT* bias = static_cast<const BiasT*>(a.bias);

    auto load_unit = [&](int u, DomRegs<BaseT, BiasT>& tr) {
        const int t = t0 + (u / nch) * nwaves;
        const int c = u % nch;
        const int v = t * 16 + col;
        const int vc = v < a.V ? v : a.V - 1;
        const uint16_t* bp = a.W + ((int64_t)t * ksteps + c * kDomKC) * 512 + lane * 8;
#pragma unroll
        for (int i = 0; i < kDomKC; ++i) {
            const bool ok = c * kDomKC + i < ksteps;
            tr.b[i] = masked_bf16x8(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bp + (ok ? i : 0) * 512)),
                                    ok ? 0xffffffffu : 0u);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) tr.base[q] = load_raw(brow[q] + vc);
        if constexpr (!is_no_prior<BiasT>::value) tr.bias = load_raw(bias + vc);
        else tr.bias = 0u;
    };
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto consume = [&](const DomRegs<BaseT, BiasT>& tr, int u) {
        const int t = t0 + (u / nch) * nwaves;
        const int c = u % nch;
        const char* ap = dyn_lds + (size_t)(c * kDomKC) * 2048 + lane * 16;
#pragma unroll
        for (int i = 0; i < kDomKC; ++i) {
            const bf16x8 hi = *reinterpret_cast<const bf16x8*>(ap + i * 2048);
            const bf16x8 lo = *reinterpret_cast<const bf16x8*>(ap + i * 2048 + 1024);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, tr.b[i], acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, tr.b[i], acc, 0, 0, 0);
        }
        if (c == nch - 1) {
            const int v = t * 16 + col;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float dot = acc[q];
                if constexpr (!is_no_prior<BiasT>::value) dot = dot + widen_raw<BiasT>(tr.bias);
                const float sc = __builtin_fmaf(dot, al[q], widen_raw<BaseT>(tr.base[q]));
                const bool take = (v < a.V) & argmax_better(sc, v, best[q], bidx[q]);
                best[q] = take ? sc : best[q];
                bidx[q] = take ? v : bidx[q];
            }
            acc = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    };
    // two register sets, refills unconditional inside the loop, the tail peeled
    DomRegs<BaseT, BiasT> tr0, tr1;
    if (units > 0) load_unit(0, tr0);
    if (units > 1) load_unit(1, tr1);
    int u = 0;
    for (; u + 4 <= units; u += 2) {
        consume(tr0, u);
        load_unit(u + 2, tr0);
        consume(tr1, u + 1);
        load_unit(u + 3, tr1);
    }
    if (u < units) consume(tr0, u);
    if (u + 2 < units) load_unit(u + 2, tr0);
    if (u + 1 < units) consume(tr1, u + 1);
    if (u + 3 < units) load_unit(u + 3, tr1);
    if (u + 2 < units) consume(tr0, u + 2);
    if (u + 3 < units) consume(tr1, u + 3);

    argmax_wg_finish(fin, best, bidx, m0, s_val, s_idx, s_last, nullptr);
}

template <typename BaseT, typename BiasT>
hipError_t launch_domino_inst(const DominoArgs& a, const ArgmaxKArgs& fin, int gx, int gy, size_t lds, hipStream_t s) {
    // the operands of E = 2048 take 128 KiB of dynamic LDS: allow it once per kernel instance (the
    // attribute belongs to the function, not to a device); call_once makes concurrent first launches
    // from several host threads safe, and every caller sees the call's result
    static std::once_flag once;
    static hipError_t attr_err = hipSuccess;
    std::call_once(once, [] {
        attr_err = hipFuncSetAttribute(reinterpret_cast<const void*>(&domino_argmax_kernel<BaseT, BiasT>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)domino_lds_bytes(kDominoMaxE));
    });
    if (attr_err != hipSuccess) return attr_err;
    hipLaunchKernelGGL((domino_argmax_kernel<BaseT, BiasT>), dim3(gx, gy, 1), dim3(256), lds, s, a, fin);
    return hipGetLastError();
}

template <typename BaseT>
hipError_t launch_domino_for_base(const DominoArgs& a, const ArgmaxKArgs& fin, int gx, int gy, size_t lds,
                                  hipStream_t s) {
    if (a.bias == nullptr) return launch_domino_inst<BaseT, no_prior_t>(a, fin, gx, gy, lds, s);
    if (a.bias_dtype == 1) return launch_domino_inst<BaseT, bf16_t>(a, fin, gx, gy, lds, s);
    if (a.bias_dtype == 2) return launch_domino_inst<BaseT, f16_t>(a, fin, gx, gy, lds, s);
    return launch_domino_inst<BaseT, float>(a, fin, gx, gy, lds, s);
}

}  // namespace

size_t domino_lds_bytes(int64_t E) {
    const int64_t ksteps = (E + 31) / 32;
    return (size_t)((ksteps + kDomKC - 1) / kDomKC) * kDomKC * 2048;
}

bool domino_supported(int64_t M, int64_t E, int64_t V) {
    return M >= 1 && M <= kMaxKeyRows && E >= 32 && E <= kDominoMaxE && E % 32 == 0 && V >= 1;
}

hipError_t launch_domino_argmax(const DominoArgs& a, void* ws, hipStream_t s) {
    char* w = static_cast<char*>(ws);
    ArgmaxKArgs fin{};
    fin.M = a.M; fin.V = a.V;
    fin.out_ids = a.out_ids; fin.out_score = a.out_score; fin.ld_out = a.ld_out;
    fin.counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
    fin.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    fin.key_stride = (int64_t)a.M * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
    const int ntiles = (a.V + 15) / 16;
    const int groups = (a.M + 15) / 16;
    // two workgroups per CU where both fit the LDS (8 waves; the operands of E <= 1024 take 64 KiB each):
    // 71.2 -> 69.8 us per step at 8 rows, E = 1024; more than fit at once is slower (three: 89 us)
    const size_t lds = domino_lds_bytes(a.E);
    const int per_cu = lds <= 64 * 1024 ? 2 : 1;
    const int gx = std::max(1, std::min((ntiles + 3) / 4, (per_cu * device_cu_count() + groups - 1) / groups));
    if (a.base_dtype == 1) return launch_domino_for_base<bf16_t>(a, fin, gx, groups, lds, s);
    if (a.base_dtype == 2) return launch_domino_for_base<f16_t>(a, fin, gx, groups, lds, s);
    return launch_domino_for_base<float>(a, fin, gx, groups, lds, s);
}

}  // namespace dels

// Fused low-rank LM-head combine + vocabulary argmax on gfx950.
//
// Semantics (code/kernel/dels.py:42-138): for row m and vocabulary index v,
//     s[m, v] = fp32(rank_m . B[v]) * alpha_m + base[m, v] - beta_m * prior[v]
// (prior term only when a prior is given and beta_m != 0); the result per row
// is the lowest v attaining the maximum and that maximum.  Logits never leave
// registers.
//
// Small-M kernel (M <= 16 rows per row group): the decode regime, bound by
// streaming B[V, r] from HBM once.  Each wave64 keeps the whole rank block of
// its 16 rows in VGPRs as MFMA A-operands (r/32 x 16 bytes per lane) and walks
// 16-row vocabulary tiles: lane l loads 16 bytes of B row (v0 + l%16) at
// k-group l/16 for every 32-wide K step (non-temporal, dwordx4), one
// v_mfma_f32_16x16x32_bf16 per step gives the 16x16 (row, vocab) dot tile,
// and the fp32 combine + running argmax run on the accumulator registers.
// Lane l holds rows 4*(l/16)+q (q < 4) of vocabulary column v0 + l%16.
//
// Cross-wave/cross-workgroup reduction: 16-lane shuffles, then LDS across the
// 4 waves, then one 64-bit atomicMax per (workgroup, row) on the packed key
// (order(score) << 32 | ~index), whose unsigned maximum is the argmax with the
// lowest-index tie rule.  The last workgroup to finish (atomic counter) decodes
// the keys into ids/scores and zeroes keys and counter for the next call, so a
// call needs no separate clearing launch and can be graph-captured.
#include <algorithm>
#include <climits>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

struct ArgmaxKArgs {
    const uint16_t* rank; int64_t ldrank;
    const uint16_t* B; int64_t ldb;
    const void* base; int64_t ldbase;
    const void* prior;
    const float* alpha; int64_t alpha_stride;
    const float* beta; int64_t beta_stride;
    int M, r, V, ksteps;
    int64_t* out_ids; float* out_score; int64_t ld_out;
    unsigned long long* keys;   // [M]
    unsigned int* counter;      // [1]
};

template <int KSTEPS, typename BaseT, typename PriorT>
__global__ __launch_bounds__(256) void fused_argmax_gemv_kernel(ArgmaxKArgs a) {
#pragma clang fp contract(off)
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int kg = lane >> 4;
    const int m0 = blockIdx.y * 16;

    // Rank operand of the 16 rows, resident for the whole kernel.
    bf16x8 ra[KSTEPS];
    {
        const int mrow = m0 + col;
        const bool mok = mrow < a.M;
        const uint16_t* rp = a.rank + (int64_t)(mok ? mrow : 0) * a.ldrank + kg * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            const bool ok = mok && s < a.ksteps && (s * 32 + kg * 8) < a.r;
            ra[s] = ok ? load_bf16x8(rp + s * 32) : zero_bf16x8();
        }
    }

    // Per-lane rows m0 + 4*kg + q.
    float al[4], be[4], best[4];
    int bidx[4];
    bool use_prior[4];
    const BaseT* brow[4];
    const BaseT* base = static_cast<const BaseT*>(a.base);
    const PriorT* prior = static_cast<const PriorT*>(a.prior);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int m = m0 + 4 * kg + q;
        const bool mok = m < a.M;
        al[q] = mok ? a.alpha[(int64_t)m * a.alpha_stride] : 0.f;
        be[q] = mok ? a.beta[(int64_t)m * a.beta_stride] : 0.f;
        use_prior[q] = (prior != nullptr) && (be[q] != 0.f);
        brow[q] = base + (int64_t)(mok ? m : 0) * a.ldbase;
        best[q] = -__builtin_inff();
        bidx[q] = INT_MAX;
    }

    const int ntiles = (a.V + 15) >> 4;
    const int nwaves = gridDim.x * 4;
    for (int t = blockIdx.x * 4 + wave; t < ntiles; t += nwaves) {
        const int v = t * 16 + col;
        const bool vok = v < a.V;
        const int vc = vok ? v : a.V - 1;   // clamped row: always a valid address
        const uint16_t* bp = a.B + (int64_t)vc * a.ldb + kg * 8;
        bf16x8 bb[KSTEPS];
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            const bool ok = s < a.ksteps && (s * 32 + kg * 8) < a.r;
            bb[s] = ok ? load_bf16x8_nt(bp + s * 32) : zero_bf16x8();
        }
        float bv[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) bv[q] = load_f32(brow[q] + vc);
        const float pv = prior ? load_f32(prior + vc) : 0.f;

        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ra[s], bb[s], acc, 0, 0, 0);

#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float sc = acc[q] * al[q];
            sc = sc + bv[q];
            if (use_prior[q]) sc = sc - be[q] * pv;
            if (vok && argmax_better(sc, v, best[q], bidx[q])) {
                best[q] = sc;
                bidx[q] = v;
            }
        }
    }

    // Reduce over the 16 vocabulary columns of each row (lanes sharing kg).
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
            const float ov = __shfl_xor(best[q], off, 64);
            const int oi = __shfl_xor(bidx[q], off, 64);
            if (argmax_better(ov, oi, best[q], bidx[q])) {
                best[q] = ov;
                bidx[q] = oi;
            }
        }
    }
    if (col == 0) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            s_val[wave][4 * kg + q] = best[q];
            s_idx[wave][4 * kg + q] = bidx[q];
        }
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        const int mi = threadIdx.x;
        float bvv = s_val[0][mi];
        int bii = s_idx[0][mi];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            if (argmax_better(s_val[w][mi], s_idx[w][mi], bvv, bii)) {
                bvv = s_val[w][mi];
                bii = s_idx[w][mi];
            }
        }
        const int m = m0 + mi;
        if (m < a.M && bii != INT_MAX) atomicMax(&a.keys[m], pack_argmax(bvv, (uint32_t)bii));
    }
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned total = gridDim.x * gridDim.y;
        const unsigned prev = atomicAdd(a.counter, 1u);
        s_last = (prev == total - 1);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int m = threadIdx.x; m < a.M; m += blockDim.x) {
        const unsigned long long key = atomic_load_u64(&a.keys[m]);
        uint32_t idx = ~(uint32_t)(key & 0xffffffffull);
        float val = f32_from_order_key((uint32_t)(key >> 32));
        if (key == 0ull || idx >= (uint32_t)a.V) {   // no finite-or-inf candidate (all NaN)
            idx = 0;
            val = -__builtin_inff();
        }
        a.out_ids[(int64_t)m * a.ld_out] = (int64_t)idx;
        if (a.out_score) a.out_score[(int64_t)m * a.ld_out] = val;
        atomic_store_u64(&a.keys[m], 0ull);
    }
    if (threadIdx.x == 0) atomic_store_u32(a.counter, 0u);
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

static inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

size_t argmax_ws_bytes(int64_t M, int64_t /*r*/, int64_t /*V*/) {
    return 256 + align256((size_t)std::max<int64_t>(M, 1) * sizeof(unsigned long long));
}

bool argmax_supported(int64_t /*M*/, int64_t r, int64_t /*V*/) { return r >= 8 && r <= 512; }

template <int KSTEPS, typename BaseT, typename PriorT>
static hipError_t launch_gemv(const ArgmaxKArgs& ka, hipStream_t s) {
    auto kern = fused_argmax_gemv_kernel<KSTEPS, BaseT, PriorT>;
    static int occ = -1;   // resident workgroups per CU (per instantiation)
    if (occ < 0) {
        int n = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kern, 256, 0) != hipSuccess || n < 1) n = 1;
        occ = n;
    }
    const int ntiles = (ka.V + 15) / 16;
    const int groups = (ka.M + 15) / 16;
    const int resident = device_cu_count() * occ;
    int gx = std::max(1, std::min((ntiles + 3) / 4, resident / groups));
    dim3 grid(gx, groups, 1);
    hipLaunchKernelGGL(kern, grid, dim3(256), 0, s, ka);
    return hipGetLastError();
}

template <int KSTEPS, typename BaseT>
static hipError_t dispatch_prior(const ArgmaxKArgs& ka, int prior_dtype, hipStream_t s) {
    if (prior_dtype == 1) return launch_gemv<KSTEPS, BaseT, bf16_t>(ka, s);
    if (prior_dtype == 2) return launch_gemv<KSTEPS, BaseT, f16_t>(ka, s);
    return launch_gemv<KSTEPS, BaseT, float>(ka, s);
}

template <int KSTEPS>
static hipError_t dispatch_base(const ArgmaxKArgs& ka, int base_dtype, int prior_dtype, hipStream_t s) {
    if (base_dtype == 1) return dispatch_prior<KSTEPS, bf16_t>(ka, prior_dtype, s);
    if (base_dtype == 2) return dispatch_prior<KSTEPS, f16_t>(ka, prior_dtype, s);
    return dispatch_prior<KSTEPS, float>(ka, prior_dtype, s);
}

hipError_t launch_fused_argmax(const ArgmaxArgs& a, void* ws, hipStream_t s) {
    ArgmaxKArgs ka{};
    ka.rank = a.rank; ka.ldrank = a.ldrank;
    ka.B = a.B; ka.ldb = a.ldb;
    ka.base = a.base; ka.ldbase = a.ldbase;
    ka.prior = a.prior;
    ka.alpha = a.alpha; ka.alpha_stride = a.alpha_stride;
    ka.beta = a.beta; ka.beta_stride = a.beta_stride;
    ka.M = a.M; ka.r = a.r; ka.V = a.V;
    ka.ksteps = (a.r + 31) / 32;
    ka.out_ids = a.out_ids; ka.out_score = a.out_score; ka.ld_out = a.ld_out;
    char* w = static_cast<char*>(ws);
    ka.counter = reinterpret_cast<unsigned int*>(w);
    ka.keys = reinterpret_cast<unsigned long long*>(w + 256);
    const int pd = a.prior ? a.prior_dtype : 0;
    if (ka.ksteps <= 4) return dispatch_base<4>(ka, a.base_dtype, pd, s);
    if (ka.ksteps <= 8) return dispatch_base<8>(ka, a.base_dtype, pd, s);
    return dispatch_base<16>(ka, a.base_dtype, pd, s);
}

}  // namespace dels

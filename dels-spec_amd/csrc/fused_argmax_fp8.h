// fp8 variant of the small-M GEMV argmax: B as e4m3 in K128 blocks with a
// per-vocabulary-row fp32 scale, the rank quantised per row to e4m3 in the
// kernel, one v_mfma_scale_f32_16x16x128_f8f6f4 per 128-wide K block.
//
// Semantics (the fp8 configuration; no counterpart in the reference, whose
// weights are bf16): for row m and vocabulary index v,
//     sR[m] = absmax(rank_m) / 448,  R_q = e4m3(rank_m / sR[m])
//     dot   = fp32(R_q . B_q[v]) * sR[m] * sB[v]          (two roundings, in that order)
//     s     = dot * alpha_m + base[m, v] - beta_m * prior[v]
// then the same lowest-index argmax as the bf16 kernels.  Layout, streaming and
// the cross-workgroup reduction are those of fused_argmax_gemv_kernel.
#pragma once

#include "fp8.h"
#include "fused_argmax_gemv.h"

namespace dels {

// One 16-row vocabulary tile held by a lane: the e4m3 B operand of each K128
// block, the base logits and the prior of its column, and its row scale.
template <int KS8>
struct TileRegs8 {
    i32x8 b[KS8];
    float base[4];
    float prior;
    float bscale;
};

template <int KS8, typename BaseT, typename PriorT>
__device__ __forceinline__ void load_tile8(const ArgmaxKArgs& a, int t, int lane, const BaseT* const (&brow)[4],
                                           const PriorT* prior, TileRegs8<KS8>& tr) {
    const int v = t * 16 + (lane & 15);
    const int vc = v < a.V ? v : a.V - 1;
    const uint8_t* bp = reinterpret_cast<const uint8_t*>(a.B) + (int64_t)t * KS8 * kFp8K128Block + lane * 16;
#pragma unroll
    for (int j = 0; j < KS8; ++j) {
        const u32x4 lo = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bp + j * kFp8K128Block));
        const u32x4 hi = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bp + j * kFp8K128Block + 1024));
        tr.b[j] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) tr.base[q] = load_f32(brow[q] + vc);
    if constexpr (!is_no_prior<PriorT>::value) tr.prior = load_f32(prior + vc);
    else tr.prior = 0.f;
    tr.bscale = __builtin_nontemporal_load(a.b_scale + vc);
}

// Contract one tile against the e4m3 rank operand and fold its 16 columns into
// the lane's running argmax of rows 4*(lane/16) + q.
template <int KS8>
__device__ __forceinline__ void consume_tile8(const ArgmaxKArgs& a, const i32x8 (&rq)[KS8], const float (&rsc)[4],
                                              const TileRegs8<KS8>& tr, int tile, int col, const float (&al)[4],
                                              const float (&be)[4], const bool (&use_prior)[4], float (&best)[4],
                                              int (&bidx)[4]) {
#pragma clang fp contract(off)
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS8; ++j) acc = mfma_e4m3_16x16x128(rq[j], tr.b[j], acc);
    const int v = tile * 16 + col;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float dot = acc[q] * rsc[q];
        dot = dot * tr.bscale;
        float sc = dot * al[q];
        sc = sc + tr.base[q];
        if (use_prior[q]) sc = sc - be[q] * tr.prior;
        const bool take = v < a.V && argmax_better(sc, v, best[q], bidx[q]);
        best[q] = take ? sc : best[q];
        bidx[q] = take ? v : bidx[q];
    }
}

// Double-buffered walk over the wave's tiles t, t + nwaves, ... (as the bf16
// GEMV): the prefetch inside the loop is unconditional on the continuing path.
template <int KS8, typename BaseT, typename PriorT>
__device__ __forceinline__ void stream_tiles8(const ArgmaxKArgs& a, const i32x8 (&rq)[KS8], const float (&rsc)[4],
                                              int t, int nwaves, int ntiles, int lane,
                                              const BaseT* const (&brow)[4], const PriorT* prior,
                                              const float (&al)[4], const float (&be)[4],
                                              const bool (&use_prior)[4], float (&best)[4], int (&bidx)[4],
                                              TileRegs8<KS8>& ta, TileRegs8<KS8>& tb, bool preloaded) {
    const int col = lane & 15;
    if (t >= ntiles) return;
    if (!preloaded) {
        load_tile8<KS8>(a, t, lane, brow, prior, ta);
        if (t + nwaves < ntiles) load_tile8<KS8>(a, t + nwaves, lane, brow, prior, tb);
    }
    if (t + nwaves >= ntiles) {
        consume_tile8<KS8>(a, rq, rsc, ta, t, col, al, be, use_prior, best, bidx);
        return;
    }
    while (true) {
        consume_tile8<KS8>(a, rq, rsc, ta, t, col, al, be, use_prior, best, bidx);
        if (t + 2 * nwaves >= ntiles) {
            consume_tile8<KS8>(a, rq, rsc, tb, t + nwaves, col, al, be, use_prior, best, bidx);
            break;
        }
        load_tile8<KS8>(a, t + 2 * nwaves, lane, brow, prior, ta);
        t += nwaves;
        consume_tile8<KS8>(a, rq, rsc, tb, t, col, al, be, use_prior, best, bidx);
        if (t + 2 * nwaves >= ntiles) {
            consume_tile8<KS8>(a, rq, rsc, ta, t + nwaves, col, al, be, use_prior, best, bidx);
            break;
        }
        load_tile8<KS8>(a, t + 2 * nwaves, lane, brow, prior, tb);
        t += nwaves;
    }
}

template <int KS8, typename BaseT, typename PriorT>
__global__ __launch_bounds__(256) void fused_argmax_gemv8_kernel(ArgmaxKArgs a) {
#pragma clang fp contract(off)
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;
    const int kg = lane >> 4;
    const int m0 = blockIdx.y * 16;

    // e4m3 rank operand of the 16 rows (row m0 + col, K bytes 32*kg .. of each block).
    i32x8 rq[KS8];
    float rsc[4];
    {
        const int mrow = m0 + col;
        const bool mok = mrow < a.M;
        const float own = quantize_rank_rows<KS8>(a.rank + (int64_t)(mok ? mrow : 0) * a.ldrank + 32 * kg, mok, rq);
#pragma unroll
        for (int q = 0; q < 4; ++q) rsc[q] = __shfl(own, 4 * kg + q, 64);   // lane 4*kg+q owns row 4*kg+q
    }

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
        use_prior[q] = !is_no_prior<PriorT>::value && (be[q] != 0.f);
        brow[q] = base + (int64_t)(mok ? m : 0) * a.ldbase;
        best[q] = -__builtin_inff();
        bidx[q] = INT_MAX;
    }
    const int ntiles = (a.V + 15) >> 4;
    const int nwaves = gridDim.x * 4;
    TileRegs8<KS8> ta, tb;
    stream_tiles8<KS8>(a, rq, rsc, blockIdx.x * 4 + wave, nwaves, ntiles, lane, brow, prior, al, be, use_prior,
                       best, bidx, ta, tb, false);
    argmax_wg_finish(a, best, bidx, m0, s_val, s_idx, s_last, nullptr);
}

template <int KS8, typename BaseT, typename PriorT>
hipError_t launch_gemv8_inst(const ArgmaxKArgs& ka, hipStream_t s) {
    const int ntiles = (ka.V + 15) / 16;
    const int groups = (ka.M + 15) / 16;
    const int cus = device_cu_count();
    const int gx = std::max(1, std::min((ntiles + 3) / 4, (cus + groups - 1) / groups));
    hipLaunchKernelGGL((fused_argmax_gemv8_kernel<KS8, BaseT, PriorT>), dim3(gx, groups, 1), dim3(256), 0, s, ka);
    return hipGetLastError();
}

// Dispatch over K128 blocks (r / 128: 1, 2 or 4) and the prior type for one base dtype.
template <typename BaseT>
hipError_t launch_gemv8_for_base(const ArgmaxKArgs& ka, int prior_kind, hipStream_t s) {
    auto by_prior = [&](auto ks_tag) -> hipError_t {
        constexpr int KS8 = decltype(ks_tag)::value;
        switch (prior_kind) {
            case 0: return launch_gemv8_inst<KS8, BaseT, no_prior_t>(ka, s);
            case 1: return launch_gemv8_inst<KS8, BaseT, float>(ka, s);
            case 2: return launch_gemv8_inst<KS8, BaseT, bf16_t>(ka, s);
            default: return launch_gemv8_inst<KS8, BaseT, f16_t>(ka, s);
        }
    };
    switch (ka.r / 128) {
        case 1: return by_prior(std::integral_constant<int, 1>{});
        case 2: return by_prior(std::integral_constant<int, 2>{});
        default: return by_prior(std::integral_constant<int, 4>{});
    }
}

hipError_t launch_gemv8_f32(const ArgmaxKArgs& ka, int prior_kind, hipStream_t s);
hipError_t launch_gemv8_bf16(const ArgmaxKArgs& ka, int prior_kind, hipStream_t s);
hipError_t launch_gemv8_f16(const ArgmaxKArgs& ka, int prior_kind, hipStream_t s);

}  // namespace dels

// fp8 variant of the small-M GEMV argmax: B as e4m3 in K128 blocks with a
// per-vocabulary-row fp32 scale, the rank quantised per row to e4m3 in the
// kernel, one v_mfma_scale_f32_16x16x128_f8f6f4 per 128-wide K block.
//
// Semantics (the fp8 configuration; no counterpart in the reference, whose
// weights are bf16): for row m and vocabulary index v,
//     sR[m] = absmax(rank_m) / 448,  R_q = e4m3(rank_m / sR[m])
//     dot   = fp32(R_q . B_q[v]) * sR[m] * sB[v]          (two roundings, in that order)
//     s     = fma(-beta_m, prior[v], fma(dot, alpha_m, base[m, v]))
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
    uint32_t base[4];   // base logits and prior as loaded (load_raw), widened at use
    uint32_t prior;
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
    for (int q = 0; q < 4; ++q) tr.base[q] = load_raw(brow[q] + vc);
    if constexpr (!is_no_prior<PriorT>::value) tr.prior = load_raw(prior + vc);
    else tr.prior = 0u;
    tr.bscale = __builtin_nontemporal_load(a.b_scale + vc);
}

// Contract one tile against the e4m3 rank operand and fold its 16 columns into
// the lane's running argmax of rows 4*(lane/16) + q.
template <int KS8, typename BaseT, typename PriorT>
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
        float sc = __builtin_fmaf(dot, al[q], widen_raw<BaseT>(tr.base[q]));
        if (use_prior[q]) sc = __builtin_fmaf(-be[q], widen_raw<PriorT>(tr.prior), sc);
        const bool take = (v < a.V) & argmax_better(sc, v, best[q], bidx[q]);   // no short circuit: branch-free
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
        consume_tile8<KS8, BaseT, PriorT>(a, rq, rsc, ta, t, col, al, be, use_prior, best, bidx);
        return;
    }
    while (true) {
        consume_tile8<KS8, BaseT, PriorT>(a, rq, rsc, ta, t, col, al, be, use_prior, best, bidx);
        if (t + 2 * nwaves >= ntiles) {
            consume_tile8<KS8, BaseT, PriorT>(a, rq, rsc, tb, t + nwaves, col, al, be, use_prior, best, bidx);
            break;
        }
        load_tile8<KS8>(a, t + 2 * nwaves, lane, brow, prior, ta);
        __builtin_amdgcn_sched_barrier(0);   // the refill is issued before the other tile is touched
        t += nwaves;
        consume_tile8<KS8, BaseT, PriorT>(a, rq, rsc, tb, t, col, al, be, use_prior, best, bidx);
        if (t + 2 * nwaves >= ntiles) {
            consume_tile8<KS8, BaseT, PriorT>(a, rq, rsc, ta, t + nwaves, col, al, be, use_prior, best, bidx);
            break;
        }
        load_tile8<KS8>(a, t + 2 * nwaves, lane, brow, prior, tb);
        __builtin_amdgcn_sched_barrier(0);
        t += nwaves;
    }
}

// ---- LDS-ring stream -------------------------------------------------------
//
// Register-held prefetch tiles cross the loop back-edge, where the compiler may
// move them between register classes and wait for every load in flight (the
// stream then degrades to one tile at a time).  The ring variant lands every
// streamed operand -- the B blocks, the tile's base logits, prior and row
// scales -- in a per-wave LDS ring with direct-to-LDS loads the compiler does
// not track, and waits with explicit vmcnt counts: R tiles in flight, exactly.
// Needs 16-byte-aligned rows (V a multiple of 16, base rows and the prior and
// scale vectors 16-byte aligned); see ring8_eligible on the host.

template <int KS8>
struct Ring8 {
    static constexpr int kB = KS8 * kFp8K128Block;   // B blocks of the tile
    static constexpr int kBase = kB;                  // [16 rows][16 columns] of base (fp32 or 16-bit)
    static constexpr int kPrior = kBase + 1024;       // 16 prior values
    static constexpr int kScale = kPrior + 64;        // 16 row scales of B
    static constexpr int kSlot = kScale + 64;         // bytes per tile slot
    static_assert(kSlot % 128 == 0, "slot alignment");
};

template <typename T> struct elem_bytes { static constexpr int value = 2; };
template <> struct elem_bytes<float> { static constexpr int value = 4; };

template <typename PriorT>
constexpr int ring8_dmas_per_tile(int ks8) { return 2 * ks8 + 2 + (is_no_prior<PriorT>::value ? 0 : 1); }

// Put tile t's operands in flight into `slot`.  `row_off` is the lane's byte
// offset of its base row (fp32: row lane/4; 16-bit: row lane/2 for lanes < 32;
// rows beyond the batch clamped to row 0).
template <int KS8, typename BaseT, typename PriorT>
__device__ __forceinline__ void issue_tile8_lds(const ArgmaxKArgs& a, int t, int lane, uint32_t row_off, char* slot) {
    using RS = Ring8<KS8>;
    const uint8_t* bsrc = reinterpret_cast<const uint8_t*>(a.B) + (int64_t)t * KS8 * kFp8K128Block;
#pragma unroll
    for (int j = 0; j < KS8; ++j) {
        dma16(bsrc, (uint32_t)(j * kFp8K128Block + lane * 16), slot + j * kFp8K128Block);
        dma16(bsrc, (uint32_t)(j * kFp8K128Block + 1024 + lane * 16), slot + j * kFp8K128Block + 1024);
    }
    constexpr int EB = elem_bytes<BaseT>::value;
    const char* base_t = static_cast<const char*>(a.base) + (int64_t)t * 16 * EB;
    if constexpr (EB == 4) {
        dma16(base_t, row_off + (uint32_t)(lane & 3) * 16, slot + RS::kBase);
    } else {
        if (lane < 32) dma16(base_t, row_off + (uint32_t)(lane & 1) * 16, slot + RS::kBase);
    }
    if constexpr (!is_no_prior<PriorT>::value) {
        constexpr int PB = elem_bytes<PriorT>::value;
        if (lane < PB) dma16(static_cast<const char*>(a.prior) + (int64_t)t * 16 * PB, (uint32_t)lane * 16,
                             slot + RS::kPrior);
    }
    if (lane < 4) dma16(a.b_scale + (int64_t)t * 16, (uint32_t)lane * 16, slot + RS::kScale);
}

// Contract tile `tile` from its LDS slot and fold it into the running argmax.
template <int KS8, typename BaseT, typename PriorT>
__device__ __forceinline__ void consume_tile8_lds(const ArgmaxKArgs& a, const i32x8 (&rq)[KS8], const float (&rsc)[4],
                                                  const char* slot, int tile, int lane, const float (&al)[4],
                                                  const float (&be)[4], const bool (&use_prior)[4],
                                                  float (&best)[4], int (&bidx)[4]) {
#pragma clang fp contract(off)
    using RS = Ring8<KS8>;
    const int col = lane & 15, kg = lane >> 4;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS8; ++j) {
        const u32x4 lo = *reinterpret_cast<const u32x4*>(slot + j * kFp8K128Block + lane * 16);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(slot + j * kFp8K128Block + 1024 + lane * 16);
        const i32x8 b = {(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2],
                         (int)hi[3]};
        acc = mfma_e4m3_16x16x128(rq[j], b, acc);
    }
    const BaseT* bl = reinterpret_cast<const BaseT*>(slot + RS::kBase);
    float pr = 0.f;
    if constexpr (!is_no_prior<PriorT>::value) pr = lds_f32(reinterpret_cast<const PriorT*>(slot + RS::kPrior) + col);
    const float bsc = reinterpret_cast<const float*>(slot + RS::kScale)[col];
    const int v = tile * 16 + col;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float dot = acc[q] * rsc[q];
        dot = dot * bsc;
        float sc = __builtin_fmaf(dot, al[q], lds_f32(bl + (4 * kg + q) * 16 + col));
        if (use_prior[q]) sc = __builtin_fmaf(-be[q], pr, sc);
        const bool take = (v < a.V) & argmax_better(sc, v, best[q], bidx[q]);
        best[q] = take ? sc : best[q];
        bidx[q] = take ? v : bidx[q];
    }
}

// Byte offset of the lane's base row for issue_tile8_lds.
template <typename BaseT>
__device__ __forceinline__ uint32_t ring8_row_off(const ArgmaxKArgs& a, int m0, int lane) {
    constexpr int EB = elem_bytes<BaseT>::value;
    const int row = m0 + (EB == 4 ? (lane >> 2) : ((lane >> 1) & 15));
    return (uint32_t)((int64_t)(row < a.M ? row : 0) * a.ldbase * EB);
}

// The wave's tiles t0, t0 + stride, ... through an R-slot LDS ring.  The first
// `issued` (<= R) tiles may already be in flight (issued by the caller in
// order into slots 0, 1, ...).
template <int KS8, int R, typename BaseT, typename PriorT>
__device__ __forceinline__ void stream_tiles8_lds(const ArgmaxKArgs& a, const i32x8 (&rq)[KS8], const float (&rsc)[4],
                                                  int t0, int stride, int ntiles, int lane, uint32_t row_off,
                                                  char* ring, int issued, const float (&al)[4],
                                                  const float (&be)[4], const bool (&use_prior)[4],
                                                  float (&best)[4], int (&bidx)[4]) {
    using RS = Ring8<KS8>;
    constexpr int PER = ring8_dmas_per_tile<PriorT>(KS8);
    static_assert(R <= 4, "wait_dma_groups covers up to 3 pending groups");
    const int nk = t0 < ntiles ? (ntiles - 1 - t0) / stride + 1 : 0;
    const int first = nk < R ? nk : R;
    for (int i = issued; i < first; ++i) issue_tile8_lds<KS8, BaseT, PriorT>(a, t0 + i * stride, lane, row_off,
                                                                             ring + i * RS::kSlot);
    int in_flight = first;   // tiles issued so far
    for (int k = 0; k < nk; ++k) {
        wait_dma_groups<PER>(in_flight - k - 1);
        char* slot = ring + (k % R) * RS::kSlot;
        consume_tile8_lds<KS8, BaseT, PriorT>(a, rq, rsc, slot, t0 + k * stride, lane, al, be, use_prior, best,
                                              bidx);
        if (k + R < nk) {
            // every LDS read of the slot has been consumed above; refill it
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            issue_tile8_lds<KS8, BaseT, PriorT>(a, t0 + (k + R) * stride, lane, row_off, slot);
            ++in_flight;
        }
    }
}

constexpr int kGemv8Ring = 3;   // LDS ring slots per wave (GEMV; the rank rows take 16 KB of LDS too)

template <int KS8, typename BaseT, typename PriorT, bool RING>
__global__ __launch_bounds__(256) void fused_argmax_gemv8_kernel(ArgmaxKArgs a) {
#pragma clang fp contract(off)
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;
    __shared__ __attribute__((aligned(1024))) char s_ring[RING ? 4 : 1][RING ? kGemv8Ring : 1]
                                                        [RING ? Ring8<KS8>::kSlot : 16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    const int col = lane & 15;
    const int kg = lane >> 4;
    const int m0 = blockIdx.y * 16;

    __shared__ __attribute__((aligned(16))) uint8_t s_rq[16 * (KS8 * 128 + 16)];   // e4m3 rank operand rows
    __shared__ float s_rsc[16];
    float al[4], be[4], best[4];
    int bidx[4];
    bool use_prior[4];
    const int ntiles = (a.V + 15) >> 4;
    const int nwaves = gridDim.x * 4;
    const int t0 = blockIdx.x * 4 + wave;
    i32x8 rq[KS8];
    float rsc[4];
    if constexpr (RING) {
        // Every load is direct-to-LDS, in this order: alpha/beta (wave 0), this
        // wave's four rank rows, the first ring tiles.  One explicit wait then
        // covers alpha/beta and the rank while the tiles stay in flight, so the
        // rank's quantisation overlaps the first HBM burst (a compiler-counted
        // load here would make its wait cover the whole burst).
        constexpr int R = KS8 * 128;
        constexpr int PER = ring8_dmas_per_tile<PriorT>(KS8);
        __shared__ __attribute__((aligned(16))) uint16_t s_rk[16 * R];   // the 16 rank rows, bf16
        __shared__ __attribute__((aligned(16))) float s_ab[2][16];      // alpha, beta of the rows
        const int mrow = m0 + (lane & 15);
        const uint32_t ab_row = (uint32_t)(mrow < a.M ? mrow : m0);
        if (wave == 0 && lane < 16) {
            dma4(a.alpha, ab_row * (uint32_t)a.alpha_stride * 4u, &s_ab[0][0]);
            dma4(a.beta, ab_row * (uint32_t)a.beta_stride * 4u, &s_ab[1][0]);
        }
        constexpr int kLanesPerRow = R / 8;          // 16-byte pieces per rank row
        constexpr int kRowsPerLoad = 64 / kLanesPerRow;
#pragma unroll
        for (int i = 0; i < KS8; ++i) {
            const int row = 4 * wave + i * kRowsPerLoad;                 // first row of this load
            const int g = m0 + row + lane / kLanesPerRow;
            const uint32_t off = (uint32_t)((int64_t)(g < a.M ? g : m0) * a.ldrank * 2) +
                                 (uint32_t)(lane % kLanesPerRow) * 16u;
            dma16(a.rank, off, &s_rk[row * R]);
        }
        const uint32_t row_off = ring8_row_off<BaseT>(a, m0, lane);
        const int nk = t0 < ntiles ? (ntiles - 1 - t0) / nwaves + 1 : 0;
        const int first = nk < kGemv8Ring ? nk : kGemv8Ring;
        for (int i = 0; i < first; ++i)
            issue_tile8_lds<KS8, BaseT, PriorT>(a, t0 + i * nwaves, lane, row_off, &s_ring[wave][i][0]);
        wait_dma_groups<PER>(first);
        lds_barrier();
        quantize_rank_coop<R>(s_rk, R, a.M - m0, s_rq, s_rsc);
        load_rank_operand<KS8>(s_rq, s_rsc, lane, rq, rsc);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool mok = m0 + 4 * kg + q < a.M;
            al[q] = mok ? s_ab[0][4 * kg + q] : 0.f;
            be[q] = mok ? s_ab[1][4 * kg + q] : 0.f;
            use_prior[q] = !is_no_prior<PriorT>::value && (be[q] != 0.f);
            best[q] = -__builtin_inff();
            bidx[q] = INT_MAX;
        }
        stream_tiles8_lds<KS8, kGemv8Ring, BaseT, PriorT>(a, rq, rsc, t0, nwaves, ntiles, lane, row_off,
                                                          &s_ring[wave][0][0], first, al, be, use_prior, best,
                                                          bidx);
    } else {
        quantize_rank_coop<KS8 * 128>(a.rank + (int64_t)m0 * a.ldrank, a.ldrank, a.M - m0, s_rq, s_rsc);
        load_rank_operand<KS8>(s_rq, s_rsc, lane, rq, rsc);
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
        TileRegs8<KS8> ta, tb;
        stream_tiles8<KS8>(a, rq, rsc, t0, nwaves, ntiles, lane, brow, prior, al, be, use_prior, best, bidx, ta, tb,
                           false);
    }
    argmax_wg_finish(a, best, bidx, m0, s_val, s_idx, s_last, nullptr);
}

// The LDS ring needs every streamed row 16-byte aligned (see the ring notes above).
inline bool ring8_eligible(const ArgmaxKArgs& ka, int base_bytes, int prior_bytes) {
    auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    if (ka.V % 16 != 0 || !al16(ka.base) || (ka.ldbase * base_bytes) % 16 != 0 || !al16(ka.b_scale)) return false;
    if ((int64_t)ka.M * ka.ldbase * base_bytes >= ((int64_t)1 << 31)) return false;
    // rank rows and alpha/beta by direct-to-LDS loads: 16-byte rows, 32-bit offsets
    if (ka.rank != nullptr && (!al16(ka.rank) || ka.ldrank % 8 != 0 || (int64_t)ka.M * ka.ldrank * 2 >= ((int64_t)1 << 31)))
        return false;
    if ((reinterpret_cast<uintptr_t>(ka.alpha) & 3) != 0 || (reinterpret_cast<uintptr_t>(ka.beta) & 3) != 0) return false;
    if ((int64_t)ka.M * (ka.alpha_stride + ka.beta_stride) * 4 >= ((int64_t)1 << 31)) return false;
    return ka.prior == nullptr || (al16(ka.prior) && prior_bytes > 0);
}

template <int KS8, typename BaseT, typename PriorT>
hipError_t launch_gemv8_inst(const ArgmaxKArgs& ka, hipStream_t s) {
    const int ntiles = (ka.V + 15) / 16;
    const int groups = (ka.M + 15) / 16;
    const int cus = device_cu_count();
    const int gx = std::max(1, std::min((ntiles + 3) / 4, (cus + groups - 1) / groups));
    const int pb = is_no_prior<PriorT>::value ? 0 : elem_bytes<PriorT>::value;
    if (ring8_eligible(ka, elem_bytes<BaseT>::value, pb))
        hipLaunchKernelGGL((fused_argmax_gemv8_kernel<KS8, BaseT, PriorT, true>), dim3(gx, groups, 1), dim3(256), 0,
                           s, ka);
    else
        hipLaunchKernelGGL((fused_argmax_gemv8_kernel<KS8, BaseT, PriorT, false>), dim3(gx, groups, 1), dim3(256), 0,
                           s, ka);
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

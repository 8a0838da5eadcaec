// Fused low-rank LM-head combine + vocabulary argmax: the small-M GEMV kernel.
//
// Semantics (code/kernel/dels.py:42-138): for row m and vocabulary index v,
//     s[m, v] = fma(-beta_m, prior[v], fma(fp32(rank_m . B[v]), alpha_m, base[m, v]))
// (each fma rounded once; the outer one only when a prior is given and
// beta_m != 0 -- every kernel of the path combines this way); the result per row
// is the lowest v attaining the maximum, and that maximum.  Logits never leave
// registers.
//
// Decode regime (M <= 16 rows per row group), bound by streaming B [V, r] from
// HBM once.  Each wave64 keeps the rank block of its 16 rows in VGPRs as MFMA
// A-operands (r/32 x 16 bytes per lane) and walks 16-row vocabulary tiles, one
// v_mfma_f32_16x16x32_bf16 per 32-wide K step; lane l then holds rows
// 4*(l/16)+q (q < 4) of vocabulary column v0 + l%16, where the fp32 combine and
// a running argmax run on the accumulator registers.  With B in the MFMA-16
// block layout every operand load is one contiguous KiB per wave.  Tiles are
// double-buffered in two explicit register sets, and the tile loads carry no
// branches (clamped addresses, masked data), so loads stay in flight across
// the contraction of the previous tile.
//
// Cross-workgroup reduction without cache fences: 16-lane shuffles and LDS
// reduce inside the workgroup; each row's result is then folded into a 64-bit
// key (order(score) << 32 | ~index) with a device-scope atomic max -- the
// unsigned maximum is the argmax with the lowest-index tie rule -- on its own
// 128-byte line.  A workgroup bumps the arrival counter only after its key
// updates have returned, and the workgroup that completes the count swaps the
// keys (and the counter) back to zero while decoding them.  Only returning
// read-modify-write atomics cross workgroups, so no L2 write-back/invalidate
// is issued, and the workspace is left clean for the next call or graph replay.
#pragma once

#include <algorithm>
#include <climits>
#include <type_traits>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

struct ArgmaxKArgs {
    const uint16_t* rank; int64_t ldrank;
    const int64_t* rank_rows;   // non-null: row m of the rank is rank[rank_rows[m * rank_rows_stride]]
    int64_t rank_rows_stride, rank_rows_count;
    const uint16_t* B; int64_t ldb;     // [V, r] row-major, or MFMA-16 blocks
    const void* base; int64_t ldbase;
    const void* prior;
    const float* alpha; int64_t alpha_stride;
    const float* beta; int64_t beta_stride;
    int M, r, V, ksteps;
    int64_t* out_ids; float* out_score; int64_t ld_out;
    unsigned long long* keys;   // row m at keys[m * key_stride]
    int64_t key_stride;
    unsigned int* counter;
    const float* b_scale;       // fp8 B only: per-vocabulary-row scale [V]
};

// How the B operand is addressed.
enum : int {
    B_PACKED_EXACT = 0,   // MFMA-16 blocks, KSTEPS == ksteps: no masking at all
    B_PACKED_MASKED = 1,  // MFMA-16 blocks, ksteps <= KSTEPS: clamped block, masked data
    B_ROWMAJOR = 2,       // [V, r] row-major: clamped row/column, masked data
};

// Operands of one 16-row vocabulary tile held by a lane: the B MFMA operand for
// every K step, and the four base logits and the prior of its column as loaded
// (load_raw; widened at use with widen_raw).
template <int KSTEPS>
struct TileRegs {
    bf16x8 b[KSTEPS];
    uint32_t base[4];
    uint32_t prior;
};

template <int KSTEPS, int MODE, typename BaseT, typename PriorT>
__device__ __forceinline__ void load_tile(const ArgmaxKArgs& a, int t, int lane, const BaseT* const (&brow)[4],
                                          const PriorT* prior, TileRegs<KSTEPS>& tr) {
    const int col = lane & 15, kg = lane >> 4;
    const int v = t * 16 + col;
    const int vc = v < a.V ? v : a.V - 1;   // clamped column: always a valid address
    if constexpr (MODE == B_PACKED_EXACT) {
        const uint16_t* bp = a.B + ((int64_t)t * KSTEPS) * 512 + lane * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) tr.b[s] = load_bf16x8_nt(bp + s * 512);
    } else if constexpr (MODE == B_PACKED_MASKED) {
        const uint16_t* bp = a.B + ((int64_t)t * a.ksteps) * 512 + lane * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            const int sc = s < a.ksteps ? s : a.ksteps - 1;
            const uint32_t mask = s < a.ksteps ? 0xffffffffu : 0u;
            tr.b[s] = masked_bf16x8(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bp + sc * 512)), mask);
        }
    } else {
        const uint16_t* bp = a.B + (int64_t)vc * a.ldb;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            const int k = s * 32 + kg * 8;
            const bool ok = s < a.ksteps && k < a.r;
            tr.b[s] = masked_bf16x8(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bp + (ok ? k : 0))),
                                    ok ? 0xffffffffu : 0u);
        }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) tr.base[q] = load_raw(brow[q] + vc);
    if constexpr (!is_no_prior<PriorT>::value) tr.prior = load_raw(prior + vc);
    else tr.prior = 0u;
}

// End of a workgroup's share of the argmax over rows m0 .. m0+15: reduce the
// lanes' running (score, index) pairs over the 16 vocabulary columns and the
// four waves, fold each row into its 64-bit key with a device-scope atomic max,
// count the workgroup in, and let the last one decode and clear the keys, the
// counter and `also_clear` (when given).
__device__ __forceinline__ void argmax_wg_finish(const ArgmaxKArgs& a, float (&best)[4], int (&bidx)[4], int m0,
                                                 float (&s_val)[4][16], int (&s_idx)[4][16], int& s_last,
                                                 unsigned int* also_clear) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    const int col = lane & 15;
    const int kg = lane >> 4;
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

    unsigned long long seen = 0;
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
        if (m < a.M && bii != INT_MAX)
            seen = __hip_atomic_fetch_max(&a.keys[(int64_t)m * a.key_stride], pack_argmax(bvv, (uint32_t)bii),
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Using the returned value makes the atomic a returning one: the branch
    // below cannot resolve before the update has been performed.
    if (seen == ~0ull) s_last = 2;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned total = gridDim.x * gridDim.y;
        const unsigned prev = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == total - 1);
    }
    __syncthreads();
    if (s_last != 1) return;
    for (int m = threadIdx.x; m < a.M; m += blockDim.x) {
        const unsigned long long key = __hip_atomic_exchange(&a.keys[(int64_t)m * a.key_stride], 0ull,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t idx = ~(uint32_t)(key & 0xffffffffull);
        float val = f32_from_order_key((uint32_t)(key >> 32));
        if (key == 0ull || idx >= (uint32_t)a.V) {   // no candidate at all (every score NaN)
            idx = 0;
            val = -__builtin_inff();
        }
        a.out_ids[(int64_t)m * a.ld_out] = (int64_t)idx;
        if (a.out_score) a.out_score[(int64_t)m * a.ld_out] = val;
    }
    if (threadIdx.x == 0) {
        __hip_atomic_exchange(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (also_clear) __hip_atomic_exchange(also_clear, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int KSTEPS, int MODE, typename BaseT, typename PriorT>
__global__ __launch_bounds__(256) void fused_argmax_gemv_kernel(ArgmaxKArgs a) {
#pragma clang fp contract(off)
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    const int col = lane & 15;
    const int kg = lane >> 4;
    const int m0 = blockIdx.y * 16;

    // Rank operand of the 16 rows, resident for the whole kernel.
    bf16x8 ra[KSTEPS];
    {
        const int mrow = m0 + col;
        const bool mok = mrow < a.M;
        const uint16_t* rp =
            a.rank + rank_row_of(a.rank_rows, a.rank_rows_stride, a.rank_rows_count, mok ? mrow : 0) * a.ldrank;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
            const int k = s * 32 + kg * 8;
            const bool ok = mok && s < a.ksteps && k < a.r;
            ra[s] = masked_bf16x8(*reinterpret_cast<const u32x4*>(rp + (ok ? k : 0)), ok ? 0xffffffffu : 0u);
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
        use_prior[q] = !is_no_prior<PriorT>::value && (be[q] != 0.f);
        brow[q] = base + (int64_t)(mok ? m : 0) * a.ldbase;
        best[q] = -__builtin_inff();
        bidx[q] = INT_MAX;
    }

    // Wave-strided walk over 16-row vocabulary tiles, double-buffered: the next
    // tile's loads are issued before the current tile is contracted.
    const int ntiles = (a.V + 15) >> 4;
    const int nwaves = gridDim.x * 4;
    int t = blockIdx.x * 4 + wave;
    auto consume = [&](const TileRegs<KSTEPS>& tr, int tile) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ra[s], tr.b[s], acc, 0, 0, 0);
        const int v = tile * 16 + col;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            float sc = __builtin_fmaf(acc[q], al[q], widen_raw<BaseT>(tr.base[q]));
            if (use_prior[q]) sc = __builtin_fmaf(-be[q], widen_raw<PriorT>(tr.prior), sc);
            const bool take = (v < a.V) & argmax_better(sc, v, best[q], bidx[q]);   // no short circuit: branch-free
            best[q] = take ? sc : best[q];
            bidx[q] = take ? v : bidx[q];
        }
    };
    // Tiles of this wave: t + k * nwaves, k < cnt, through a ring of ND tile
    // register sets (ND - 1 tiles in flight while one is contracted, ND right
    // after its refill).  The loop runs only while the refills exist, so its
    // loads are unconditional and every path into the loop top carries the
    // same outstanding loads: the compiler's wait before each contraction
    // covers only the oldest set.  The last 2 * ND - 1 tiles or fewer are
    // peeled.  ND = 2 measured best: for 8 K steps (r = 256) 18.0 us against
    // 20.0 with 3 sets, 26.8 with 6 and 21.2 for the earlier load-then-consume
    // loop; for 16 K steps 2 and 3 sets are within 1 %.
    constexpr int ND = 2;
    const int cnt = t < ntiles ? (ntiles - 1 - t) / nwaves + 1 : 0;
    TileRegs<KSTEPS> tr[ND];
#pragma unroll
    for (int u = 0; u < ND; ++u)
        if (u < cnt) load_tile<KSTEPS, MODE>(a, t + u * nwaves, lane, brow, prior, tr[u]);
    int k = 0;
    for (; k + 2 * ND <= cnt; k += ND) {
#pragma unroll
        for (int u = 0; u < ND; ++u) {
            consume(tr[u], t + (k + u) * nwaves);
            load_tile<KSTEPS, MODE>(a, t + (k + u + ND) * nwaves, lane, brow, prior, tr[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < ND; ++u) {
        if (k + u < cnt) consume(tr[u], t + (k + u) * nwaves);
        if (k + u + ND < cnt) load_tile<KSTEPS, MODE>(a, t + (k + u + ND) * nwaves, lane, brow, prior, tr[u]);
    }
#pragma unroll
    for (int u = 0; u < ND; ++u)
        if (k + u + ND < cnt) consume(tr[u], t + (k + u + ND) * nwaves);

    argmax_wg_finish(a, best, bidx, m0, s_val, s_idx, s_last, nullptr);
}

// Launch of one instantiation on about one workgroup per CU in total (the
// streaming loop saturates HBM there; every extra workgroup adds one more
// round of cross-workgroup atomics).
template <int KSTEPS, int MODE, typename BaseT, typename PriorT>
hipError_t launch_gemv_inst(const ArgmaxKArgs& ka, hipStream_t s) {
    const int ntiles = (ka.V + 15) / 16;
    const int groups = (ka.M + 15) / 16;
    const int cus = device_cu_count();
    const int gx = std::max(1, std::min((ntiles + 3) / 4, (cus + groups - 1) / groups));
    hipLaunchKernelGGL((fused_argmax_gemv_kernel<KSTEPS, MODE, BaseT, PriorT>), dim3(gx, groups, 1), dim3(256), 0,
                       s, ka);
    return hipGetLastError();
}

// Dispatch over B mode / K steps / prior type for one base dtype.
template <typename BaseT>
hipError_t launch_gemv_for_base(const ArgmaxKArgs& ka, bool packed, int prior_kind, hipStream_t s) {
    auto by_prior = [&](auto ks_tag, auto mode_tag) -> hipError_t {
        constexpr int KS = decltype(ks_tag)::value;
        constexpr int MODE = decltype(mode_tag)::value;
        switch (prior_kind) {
            case 0: return launch_gemv_inst<KS, MODE, BaseT, no_prior_t>(ka, s);
            case 1: return launch_gemv_inst<KS, MODE, BaseT, float>(ka, s);
            case 2: return launch_gemv_inst<KS, MODE, BaseT, bf16_t>(ka, s);
            default: return launch_gemv_inst<KS, MODE, BaseT, f16_t>(ka, s);
        }
    };
    using I2 = std::integral_constant<int, 2>;
    using I4 = std::integral_constant<int, 4>;
    using I8 = std::integral_constant<int, 8>;
    using I16 = std::integral_constant<int, 16>;
    using PE = std::integral_constant<int, B_PACKED_EXACT>;
    using PM = std::integral_constant<int, B_PACKED_MASKED>;
    using RM = std::integral_constant<int, B_ROWMAJOR>;
    if (packed) {
        switch (ka.ksteps) {
            case 2: return by_prior(I2{}, PE{});
            case 4: return by_prior(I4{}, PE{});
            case 8: return by_prior(I8{}, PE{});
            case 16: return by_prior(I16{}, PE{});
            default: return by_prior(I16{}, PM{});
        }
    }
    if (ka.ksteps <= 4) return by_prior(I4{}, RM{});
    if (ka.ksteps <= 8) return by_prior(I8{}, RM{});
    return by_prior(I16{}, RM{});
}

hipError_t launch_gemv_f32(const ArgmaxKArgs& ka, bool packed, int prior_kind, hipStream_t s);
hipError_t launch_gemv_bf16(const ArgmaxKArgs& ka, bool packed, int prior_kind, hipStream_t s);
hipError_t launch_gemv_f16(const ArgmaxKArgs& ka, bool packed, int prior_kind, hipStream_t s);

}  // namespace dels

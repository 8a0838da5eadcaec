// Fused low-rank LM-head combine + vocabulary argmax: the batched (MFMA-tiled)
// kernel for many draft rows (batch x block verification, M >= 64).
//
// Semantics as the GEMV kernel (code/kernel/dels.py:42-138):
//     s[m, v] = fma(-beta_m, prior[v], fma(fp32(rank_m . B[v]), alpha_m, base[m, v]))
// and per row the lowest v attaining max_v s[m, v].
//
// Here the contraction rank[M, r] x B[V, r]^T is a real dense GEMM, computed
// transposed with v_mfma_f32_32x32x16_bf16 (on gfx950 the 32x32 bf16 MFMA
// issues at close to twice the rate of the 16x16x32 one): the A operand is a
// 32-vocabulary x 16-K slab of B, the B operand a 16-K x 32-row slab of rank,
// so lane l ends up with row l%32 and the sixteen vocabulary columns
// 8*g + 4*(l/32) + q (g, q < 4) of the tile.  One row per lane: the running
// argmax stays in the lane over the whole vocabulary chunk, visiting its
// candidates in increasing index order (so a strict ">" keeps the lowest index
// of a tie), and the base logits it needs are four runs of four consecutive
// elements of one row.
//
// Workgroup: kWaves = 8 waves, 2 per SIMD.  Wave w keeps the rank operand of
// its kRowBlocks = 1 block of 32 rows in VGPRs for the whole kernel (r/16 K
// steps x 16 bytes per lane); a workgroup covers 256 rows and a contiguous
// chunk of 32-column vocabulary tiles, one tile per pipeline stage.  (The code
// also runs 4 waves of two 32-row blocks each, one wave per SIMD, so that
// every B operand read from LDS feeds two MFMAs: measured 20 % slower, a
// single wave per SIMD cannot cover its own LDS and DMA issue.)  A stage's B
// tile is two consecutive 16-row block rows of the MFMA-16 layout -- one
// contiguous run of HBM -- and is copied HBM -> LDS with direct-to-LDS loads
// (global_load_lds_dwordx4, no VGPR staging) that gather it into
// K-step-major MFMA-32 operand order, together with each wave's base-logit
// tile (laid out so that the epilogue reads it lane-contiguously) and the
// prior slice.  NBUF stage buffers (as many as fit in 160 KiB of LDS, up to 4)
// keep NBUF-1 stages of loads in flight; each wave waits for its own loads of
// the stage with an explicit vmcnt count (every wave issues the same number
// of loads per stage) and a barrier then publishes the stage to all waves.
// The buffers are distinct LDS objects named statically in an NBUF-way
// unrolled loop, so the compiler can tell the reads of one buffer from the
// loads in flight into the others and adds no waits of its own.
//
// The combine + argmax of stage st-1 (the epilogue) runs between the MFMAs of
// stage st: its accumulators and base/prior values are held in registers
// (the latter read from the stage buffer during st-1's own contraction), so
// the matrix core does not idle while a wave combines, and a stage buffer is
// free for new loads as soon as its contraction is done.
//
// Workgroups sharing a vocabulary chunk (the row groups) have linear ids that
// differ by a multiple of 8, so they run on the same XCD and the second read of
// each B tile is served by that XCD's L2.
//
// Cross-workgroup reduction (tiled_argmax_finish): each workgroup merges one
// 64-bit key per row (order(score) << 32 | ~index, 0 = no candidate) into the
// row's key with a device-scope atomic maximum -- the unsigned maximum is the
// argmax with the lowest-index tie rule --, and the last workgroup to arrive
// decodes the keys and returns keys and arrival counter to zero.
#pragma once

#include <algorithm>
#include <climits>
#include <type_traits>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

struct TiledKArgs {
    const uint16_t* rank; int64_t ldrank;
    const int64_t* rank_rows;   // non-null: row m of the rank is rank[rank_rows[m * rank_rows_stride]]
    int64_t rank_rows_stride, rank_rows_count;
    const uint16_t* B;          // MFMA-16 blocks, r a multiple of 32 (e4m3 kernel: K128 blocks)
    const float* b_scale;       // e4m3 kernel only: per-row scale of B
    const uint8_t* rank_q;      // e4m3 kernel only: the rank quantised per row [M][ldrank bytes]
    const float* rank_scale;    // e4m3 kernel only: its per-row scale [M]
    const void* base; int64_t ldbase;
    const void* prior;          // nullptr when there is no prior
    const float* alpha; int64_t alpha_stride;
    const float* beta; int64_t beta_stride;
    int M, V;
    int nblk16;                 // ceil(V / 16): 16-row block rows of the packed B
    int ntiles;                 // ceil(V / 32): 32-column vocabulary tiles
    unsigned long long* keys;   // per-row argmax keys (control area), key_stride apart
    int64_t key_stride;
    unsigned int* counter;      // workgroup arrivals (control area)
    int64_t* out_ids; float* out_score; int64_t ld_out;
};

// Cross-workgroup argmax of the tiled kernels: every workgroup merges its
// rows' keys (order(score) << 32 | ~index, 0 = no candidate) into the row keys
// with returning device-scope atomic maxima -- the unsigned maximum is the
// argmax with the lowest-index tie rule --, then counts itself in; the last
// workgroup decodes every row and returns keys and counter to zero.  (This
// replaces a second kernel that reduced per-chunk keys: its launch cost more
// than the atomics, which are spread over the workgroups' ends.)  `flag` may
// alias the stage buffers: the first barrier ends every wave's use of them.
template <int NB>
__device__ __forceinline__ void tiled_argmax_finish(const TiledKArgs& a, const int (&m)[NB],
                                                    const unsigned long long (&key)[NB], int* flag) {
    __syncthreads();
    unsigned long long seen = 0;
#pragma unroll
    for (int i = 0; i < NB; ++i)
        if (m[i] >= 0 && key[i] != 0ull)
            seen |= __hip_atomic_fetch_max(&a.keys[(int64_t)m[i] * a.key_stride], key[i], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    // Using the returned values makes the maxima returning atomics: each has
    // been performed before the barrier below (the write is overwritten).
    if (seen == ~0ull) *flag = 2;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned total = gridDim.x * gridDim.y;
        const unsigned prev = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = prev == total - 1;
    }
    __syncthreads();
    if (*flag != 1) return;
    for (int r = threadIdx.x; r < a.M; r += blockDim.x) {
        const unsigned long long k = __hip_atomic_exchange(&a.keys[(int64_t)r * a.key_stride], 0ull,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t idx = ~(uint32_t)(k & 0xffffffffull);
        float val = f32_from_order_key((uint32_t)(k >> 32));
        if (k == 0ull || idx >= (uint32_t)a.V) {   // no candidate at all (every score NaN)
            idx = 0;
            val = -__builtin_inff();
        }
        a.out_ids[(int64_t)r * a.ld_out] = (int64_t)idx;
        if (a.out_score) a.out_score[(int64_t)r * a.ld_out] = val;
    }
    if (threadIdx.x == 0) __hip_atomic_exchange(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

namespace tiled {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRowBlocks = 1;                         // 32-row MFMA blocks per wave
constexpr int kRowsPerWave = 32 * kRowBlocks;
constexpr int kRowsPerWG = kWaves * kRowsPerWave;
constexpr int kTileCols = 32;
constexpr int kLdsBytes = 160 * 1024;
constexpr int kPriorBytesPerWave = 256;
constexpr int kOperandAhead = 4;

// Stage buffer parts: B tile (two 16-row block rows of KS 1 KiB blocks), each
// wave's base tile (its rows x 32 columns) and each wave's prior slice.
template <int KS>
constexpr int b_bytes() { return 2 * KS * 1024; }
template <typename BaseT>
constexpr int base_bytes_per_wave() { return kRowsPerWave * kTileCols * (int)sizeof(BaseT); }
template <int KS, typename BaseT>
constexpr int stage_bytes() {
    return b_bytes<KS>() + kWaves * base_bytes_per_wave<BaseT>() + kWaves * kPriorBytesPerWave;
}
template <int KS, typename BaseT>
constexpr int num_buffers() {
    constexpr int n = kLdsBytes / stage_bytes<KS, BaseT>();
    return n > 4 ? 4 : n;
}
// Direct-to-LDS load instructions one wave issues per stage.
template <int KS, typename BaseT, bool PRIOR>
constexpr int loads_per_stage() {
    return (2 * KS) / kWaves + kRowBlocks * (sizeof(BaseT) == 4 ? 4 : 2) + (PRIOR ? 1 : 0);
}

// Wait until at most N of this wave's vector-memory operations are
// outstanding and all of its LDS operations are done (gfx9 s_waitcnt
// encoding: vmcnt split over bits 3:0 and 15:14, expcnt 6:4 left at 7,
// lgkmcnt 11:8 = 0), then the workgroup barrier.  The empty asm statements
// with a memory clobber keep the compiler from moving memory accesses across.
template <int N>
__device__ __forceinline__ void stage_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Value `hi` (0: low half, 1: high half) of a packed pair of 16-bit values, widened.
template <typename T>
__device__ __forceinline__ float half_at(uint32_t w, int hi) {
    if constexpr (std::is_same<T, bf16_t>::value) {
        return __uint_as_float(hi ? (w & 0xffff0000u) : (w << 16));
    } else {
        const uint16_t b = (uint16_t)(hi ? (w >> 16) : (w & 0xffffu));
        _Float16 x;
        __builtin_memcpy(&x, &b, 2);
        return (float)x;
    }
}

// -inf as a 16-bit value of type T.
template <typename T>
constexpr uint32_t half_neg_inf() { return std::is_same<T, bf16_t>::value ? 0xff80u : 0xfc00u; }

}  // namespace tiled

// EXACT: V is a multiple of the 32-column tile, so no tile needs masking.
template <int KS, typename BaseT, typename PriorT, bool EXACT>
__global__ __launch_bounds__(tiled::kThreads) void fused_argmax_tiled_kernel(TiledKArgs a) {
#pragma clang fp contract(off)
    using namespace tiled;
    constexpr int kSteps = 2 * KS;                       // 16-deep K steps
    constexpr int kB = b_bytes<KS>();
    constexpr int kBaseW = base_bytes_per_wave<BaseT>();
    constexpr int kBaseRB = kBaseW / kRowBlocks;         // base bytes of one row block
    constexpr bool kPrior = !is_no_prior<PriorT>::value;
    constexpr int NBUF = num_buffers<KS, BaseT>();
    constexpr int P = NBUF - 1;                          // stages in flight
    constexpr int E = loads_per_stage<KS, BaseT, kPrior>();
    constexpr int nb = kSteps / kWaves;                  // B blocks per wave and stage
    constexpr int nbase = sizeof(BaseT) == 4 ? 4 : 2;    // base loads per row block
    constexpr int kWB = sizeof(BaseT) == 4 ? 16 : 8;     // words of one row block's base values
    constexpr int kWP = sizeof(PriorT) == 4 ? 16 : 8;    // words of the prior values
    constexpr int kSlots = kSteps * kRowBlocks;          // MFMAs per stage
    constexpr int kCands = 16 * kRowBlocks;              // epilogue candidates per stage
    constexpr int kAhead = kOperandAhead;                // B operand reads in flight per wave
    static_assert(NBUF >= 2, "stage does not fit twice in LDS");
    static_assert((2 * KS) % kWaves == 0, "B blocks per stage must split over the waves");
    static_assert(E <= 31, "vmcnt holds the loads of two stages");

    struct __attribute__((aligned(1024))) Stage {
        char b[kB];
        char base[kWaves][kBaseW];
        char prior[kWaves][kPriorBytesPerWave];
    };
    struct NoStage {};
    __shared__ Stage lds0, lds1;
    __shared__ std::conditional_t<(NBUF > 2), Stage, NoStage> lds2;
    __shared__ std::conditional_t<(NBUF > 3), Stage, NoStage> lds3;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar control
    const int rl = lane & 31;       // row of this lane within a 32-row block
    const int h = lane >> 5;        // K half of the operands / vocabulary quad of the results
    const int mw = blockIdx.y * kRowsPerWG + wave * kRowsPerWave;   // first row of this wave
    const bool wave_active = mw < a.M;

    // Vocabulary chunk of this workgroup: 32-column tiles [T0, T0 + nst), one per
    // stage.  (A round-robin assignment of tiles measured slower: the base rows
    // are then read in pieces no workgroup continues.)
    const int T0 = (int)(((int64_t)blockIdx.x * a.ntiles) / gridDim.x);
    const int nst = (int)(((int64_t)(blockIdx.x + 1) * a.ntiles) / gridDim.x) - T0;
    auto tile_of = [&](int st) { return T0 + st; };

    // Rank operand of the wave's rows, resident for the whole kernel; rows past
    // M repeat row M-1 (their results are not written).
    bf16x8 ra[kRowBlocks][kSteps];
    float al[kRowBlocks], nbeta[kRowBlocks], best[kRowBlocks];
    int bidx[kRowBlocks];
    // prior bits kept (the row uses the prior term) or cleared: fp32/f16 mask, the
    // high half of a 16-bit pair, and the v_perm_b32 selector of the low half
    uint32_t pmask[kRowBlocks], pmask_hi[kRowBlocks], psel_lo[kRowBlocks];
    uint32_t row_off[kRowBlocks];   // byte offset of the lane's base row (M * ldbase * size < 2^31)
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb) {
        const int mrow = min(mw + 32 * rb + rl, a.M - 1);
        const uint16_t* rp =
            a.rank + rank_row_of(a.rank_rows, a.rank_rows_stride, a.rank_rows_count, mrow) * a.ldrank + h * 8;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) ra[rb][s] = load_bf16x8(rp + s * 16);
        al[rb] = a.alpha[(int64_t)mrow * a.alpha_stride];
        const float be = a.beta[(int64_t)mrow * a.beta_stride];
        // beta == 0 skips the prior term: fma(0, +0, sc) == sc, whatever the prior holds
        const bool use_prior = kPrior && be != 0.f;
        nbeta[rb] = use_prior ? -be : 0.f;
        pmask[rb] = use_prior ? 0xffffffffu : 0u;
        pmask_hi[rb] = use_prior ? 0xffff0000u : 0u;
        psel_lo[rb] = use_prior ? 0x01000c0cu : 0x0c0c0c0cu;   // bytes 1,0 -> 3,2; zeros below
        best[rb] = -__builtin_inff();
        bidx[rb] = INT_MAX;
        row_off[rb] = (uint32_t)mrow * (uint32_t)a.ldbase * (uint32_t)sizeof(BaseT);
    }
    // Wait for the rank (and alpha/beta) loads here, before any direct-to-LDS
    // load is issued.  The compiler's wait insertion does not see those asm
    // loads and joins the state before the stage loop into every iteration:
    // with these loads still pending there it would wait for them -- that is,
    // for every stage load in flight -- before each MFMA of every stage.
    __builtin_amdgcn_s_waitcnt(0x0070 | (0xf << 8));   // vmcnt(0); expcnt and lgkmcnt left free

    const char* Bg = reinterpret_cast<const char*>(a.B);
    const char* baseg = static_cast<const char*>(a.base);
    const char* priorg = static_cast<const char*>(a.prior);

    // Direct-to-LDS loads of stage `st` into buffer S: exactly E instructions
    // per wave.  Addresses past the data are clamped to valid memory; their
    // results are masked in the epilogue.
    // The B tile is stored K-step-major: LDS block s (1 KiB) holds the A
    // operand of 16-deep step s in lane order, gathered by the loads from the
    // two 16-row block rows of the packed layout (lane L: row L%32 of the tile,
    // K 16s + 8*(L/32) .. +7), so every operand read is one contiguous,
    // bank-conflict-free KiB.
    // Per-lane part of the B gather offset: row l%16 of block row (l/16)%2, K group l/32.
    const uint32_t b_lane = ((lane & 15) + 16 * h) * 16;
    const uint32_t b_hi = ((lane >> 4) & 1) ? (uint32_t)KS * 1024 : 0u;
    // Load `piece` (0 <= piece < E) of stage `st` into buffer S: pieces 0..nb-1
    // are B blocks, then the base-logit loads of each row block, then the prior
    // slice.  `piece` is a constant wherever this is called (unrolled loops), so
    // the chain of tests folds away.
    auto issue_piece = [&](Stage& S, int st, int piece) {
        const int T = tile_of(st);
        const int vs = T * kTileCols;
        if (piece < nb) {
            // block rows 2T and 2T+1 (the second clamped to the last one, masked later)
            const int rb0 = min(2 * T, a.nblk16 - 1);
            const bool two = 2 * T + 1 < a.nblk16;
            const char* bt = Bg + (int64_t)rb0 * KS * 1024;
            const int step = wave * nb + piece;                  // K step of this load
            dma16(bt, b_lane + (two ? b_hi : 0u) + (step >> 1) * 1024 + (step & 1) * 512, S.b + step * 1024);
        } else if (piece < nb + kRowBlocks * nbase) {
            const int rb = (piece - nb) / nbase, g = (piece - nb) % nbase;
            char* dst = S.base[wave] + rb * kBaseRB + g * 1024;
            if constexpr (sizeof(BaseT) == 4) {
                // load g: lane L -> row L%32, 4-column chunk 2g + L/32
                const int v = min(vs + 4 * (2 * g + h), a.V - 4);
                dma16(baseg, row_off[rb] + (uint32_t)v * 4u, dst);
            } else {
                // load g: lane L -> row L%32, 8-column chunk 2g + L/32
                const int v = min(vs + 8 * (2 * g + h), a.V - 8);
                dma16(baseg, row_off[rb] + (uint32_t)v * 2u, dst);
            }
        } else if (kPrior && piece == nb + kRowBlocks * nbase) {
            if constexpr (sizeof(PriorT) == 4) {
                const int v = min(vs + (lane & 31), a.V - 1);
                dma4(priorg, (uint32_t)v * 4u, S.prior[wave]);
            } else {
                const int v = min(vs + 2 * (lane & 15), a.V - 2);
                dma4(priorg, (uint32_t)v * 2u, S.prior[wave]);
            }
        }
    };
    auto issue_stage = [&](Stage& S, int st) {
#pragma unroll
        for (int piece = 0; piece < E; ++piece) issue_piece(S, st, piece);
    };

    // Epilogue operands of one stage in registers: per row block the base
    // values of the lane's 16 columns 8g + 4h + q (candidate j = 4g + q; fp32
    // words, or 16-bit pairs with j in word j/2), and the prior values of the
    // same columns.  Columns past V carry a -inf base, which never wins.
    struct EpiRegs {
        uint32_t b[kRowBlocks][kWB];
        uint32_t p[kWP];
    };
    constexpr uint32_t kNegInf = sizeof(BaseT) == 4 ? 0xff800000u : half_neg_inf<BaseT>();
    // Group g (candidates 4g .. 4g+3) of row block rb of stage st from S; the
    // prior group with the last row block (the last reader of the old values).
    auto load_epi_group = [&](const Stage& S, int st, int rb, int g, EpiRegs& e) {
        const int vs = tile_of(st) * kTileCols;
        const int v = vs + 8 * g + 4 * h;   // column of candidate 4g
        const bool partial = !EXACT && vs + kTileCols > a.V;   // only the last tile of the vocabulary
        if constexpr (sizeof(BaseT) == 4) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(S.base[wave] + rb * kBaseRB + g * 1024 + lane * 16);
#pragma unroll
            for (int q = 0; q < 4; ++q) e.b[rb][4 * g + q] = (partial && v + q >= a.V) ? kNegInf : w[q];
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(S.base[wave] + rb * kBaseRB + (g >> 1) * 1024 +
                                                            (rl + 32 * (g & 1)) * 16 + h * 8);
            uint32_t w0 = w.x, w1 = w.y;
            if (partial) {
                w0 = v < a.V ? w0 : ((w0 & 0xffff0000u) | kNegInf);
                w0 = v + 1 < a.V ? w0 : ((w0 & 0xffffu) | (kNegInf << 16));
                w1 = v + 2 < a.V ? w1 : ((w1 & 0xffff0000u) | kNegInf);
                w1 = v + 3 < a.V ? w1 : ((w1 & 0xffffu) | (kNegInf << 16));
            }
            e.b[rb][2 * g] = w0;
            e.b[rb][2 * g + 1] = w1;
        }
        if constexpr (kPrior) {
            if (rb == kRowBlocks - 1) {
                const char* pp = S.prior[wave] + (8 * g + 4 * h) * (int)sizeof(PriorT);
                if constexpr (sizeof(PriorT) == 4) {
                    const u32x4 w = *reinterpret_cast<const u32x4*>(pp);
#pragma unroll
                    for (int q = 0; q < 4; ++q) e.p[4 * g + q] = w[q];
                } else {
                    const uint2 w = *reinterpret_cast<const uint2*>(pp);
                    e.p[2 * g] = w.x;
                    e.p[2 * g + 1] = w.y;
                }
            }
        }
    };
    auto word_to_base = [&](uint32_t w, int j) -> float {
        if constexpr (sizeof(BaseT) == 4) return __uint_as_float(w);
        else return half_at<BaseT>(w, j & 1);
    };
    // Prior value of candidate j, as +0 for rows without the prior term.
    auto masked_prior = [&](uint32_t w, int j, int rb) -> float {
        if constexpr (sizeof(PriorT) == 4) {
            return __uint_as_float(w & pmask[rb]);
        } else if constexpr (std::is_same<PriorT, bf16_t>::value) {
            return __uint_as_float((j & 1) ? (w & pmask_hi[rb]) : __builtin_amdgcn_perm(w, w, psel_lo[rb]));
        } else {
            return __uint_as_float(__float_as_uint(half_at<PriorT>(w, j & 1)) & pmask[rb]);
        }
    };
    // Candidate j of row block rb of stage stp.
    // The empty volatile asm statements pin the candidate's work to its place
    // between the MFMAs: pure arithmetic is otherwise free to be gathered
    // after the last MFMA of the stage, which is where the compiler puts it.
    // They pin values just extracted, so that no register is copied for them.
    auto epi_one = [&](const f32x16 (&accp)[kRowBlocks], const EpiRegs& e, int sidx, int rb, int j) {
        float av = accp[rb][j];
        float bv = word_to_base(e.b[rb][sizeof(BaseT) == 4 ? j : (j >> 1)], j);
        asm volatile("" : "+v"(av), "+v"(bv));
        float sc = __builtin_fmaf(av, al[rb], bv);
        if constexpr (kPrior) {
            float pv = masked_prior(e.p[sizeof(PriorT) == 4 ? j : (j >> 1)], j, rb);
            asm volatile("" : "+v"(pv));
            sc = __builtin_fmaf(nbeta[rb], pv, sc);
        }
        // candidates arrive in increasing index order: strict ">" keeps the lowest index
        const bool take = sc > best[rb];
        best[rb] = take ? sc : best[rb];
        bidx[rb] = take ? sidx + j : bidx[rb];
        asm volatile("" : "+v"(best[rb]), "+v"(bidx[rb]));
    };

    // Contraction of stage st from S (one accumulation chain per row block,
    // operands read kAhead steps ahead), with three kinds of work spread between
    // its MFMAs: the epilogue of the previous stage (accp, ep, stp), the reads
    // of stage st's epilogue operands into ep_next (group by group, each after
    // the same group of ep is done), and the loads of stage st_next into next.
    auto contract = [&](const Stage& S, int st, Stage& next, int st_next, f32x16 (&acc)[kRowBlocks],
                        const f32x16 (&accp)[kRowBlocks], const EpiRegs& ep, int stp, EpiRegs& ep_next) {
#pragma unroll
        for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[rb][i] = 0.f;
        const char* ap = S.b + lane * 16;
        auto opnd = [&](int s) { return *reinterpret_cast<const bf16x8*>(ap + s * 1024); };
        const bool issue = st_next >= 0;
        // operand ring: the read of step s + kAhead is issued before the MFMAs of step s
        bf16x8 opq[kAhead];
#pragma unroll
        for (int i = 0; i < kAhead; ++i) opq[i] = opnd(i < kSteps ? i : 0);
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const bf16x8 a0 = opq[s % kAhead];
            if (s + kAhead < kSteps) opq[s % kAhead] = opnd(s + kAhead);
#pragma unroll
            for (int rb = 0; rb < kRowBlocks; ++rb) {
                const int slot = s * kRowBlocks + rb;
                __builtin_amdgcn_sched_barrier(0);
                acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, ra[rb][s], acc[rb], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
                // candidates c in [slot * kCands / kSlots, (slot + 1) * kCands / kSlots): row block c / 16, j = c % 16
#pragma unroll
                for (int c = slot * kCands / kSlots; c < (slot + 1) * kCands / kSlots; ++c) {
                    epi_one(accp, ep, stp * 16, c >> 4, c & 15);
                    if ((c & 3) == 3) load_epi_group(S, st, c >> 4, (c & 15) >> 2, ep_next);
                }
#pragma unroll
                for (int piece = 0; piece < E; ++piece)
                    if (slot == piece * kSlots / E && issue) issue_piece(next, st_next, piece);
            }
        }
    };

    // Pipeline: stages 0..P-1 are issued up front; at stage st each wave waits
    // for its own loads of st (the younger stages may stay in flight), the
    // barrier publishes st, the freed buffer of st-1 takes stage st+P, and st
    // is contracted while st-1 is combined.
    auto buf = [&](int i) -> Stage& {
        if constexpr (NBUF > 3) { if (i == 3) return lds3; }
        if constexpr (NBUF > 2) { if (i == 2) return lds2; }
        return i == 1 ? lds1 : lds0;
    };
    f32x16 acc_prev[kRowBlocks];
    EpiRegs ep_prev, ep_cur;
    int st_prev = 0;
    // no stage before stage 0: a -inf base makes its epilogue a no-op
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc_prev[rb][i] = 0.f;
#pragma unroll
        for (int i = 0; i < kWB; ++i) ep_prev.b[rb][i] = sizeof(BaseT) == 4 ? kNegInf : kNegInf * 0x10001u;
    }
#pragma unroll
    for (int i = 0; i < kWP; ++i) ep_prev.p[i] = 0u;

#pragma unroll
    for (int i = 0; i < P; ++i)
        if (i < nst) issue_stage(buf(i), i);
    for (int st0 = 0; st0 < nst; st0 += NBUF) {
#pragma unroll
        for (int u = 0; u < NBUF; ++u) {
            const int st = st0 + u;
            if (st < nst) {
                const int younger = min(P - 1, nst - 1 - st);
                if constexpr (P >= 3) {
                    if (younger >= 2) stage_barrier<2 * E>();
                    else if (younger == 1) stage_barrier<E>();
                    else stage_barrier<0>();
                } else if constexpr (P == 2) {
                    if (younger >= 1) stage_barrier<E>();
                    else stage_barrier<0>();
                } else {
                    stage_barrier<0>();
                }
                const int st_next = st + P < nst ? st + P : -1;
                if (wave_active) {
                    f32x16 acc[kRowBlocks];
                    contract(buf(u), st, buf((u + P) % NBUF), st_next, acc, acc_prev, ep_prev, st_prev, ep_cur);
#pragma unroll
                    for (int rb = 0; rb < kRowBlocks; ++rb) acc_prev[rb] = acc[rb];
                    ep_prev = ep_cur;
                    st_prev = st;
                } else if (st_next >= 0) {
                    issue_stage(buf((u + P) % NBUF), st_next);
                }
            }
        }
    }
    if (wave_active && nst > 0) {
        // the epilogue of the last stage
#pragma unroll
        for (int c = 0; c < kCands; ++c) epi_one(acc_prev, ep_prev, st_prev * 16, c >> 4, c & 15);
    }

    // Decode the candidate slot st*16 + j into the vocabulary index, then merge
    // the two vocabulary quads of each row (lanes l and l^32).
    int fin_m[kRowBlocks];
    unsigned long long fin_key[kRowBlocks];
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb) {
        float bv = best[rb];
        int bi = bidx[rb];
        if (bi != INT_MAX) {
            const int st = bi >> 4, c = bi & 15;
            bi = tile_of(st) * kTileCols + 8 * (c >> 2) + 4 * h + (c & 3);
        }
        const float ov = __shfl_xor(bv, 32, 64);
        const int oi = __shfl_xor(bi, 32, 64);
        if (argmax_better(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
        const int m = mw + 32 * rb + rl;
        fin_m[rb] = (h == 0 && m < a.M) ? m : -1;
        fin_key[rb] = bi == INT_MAX ? 0ull : pack_argmax(bv, (uint32_t)bi);
    }
    tiled_argmax_finish(a, fin_m, fin_key, reinterpret_cast<int*>(&lds0));
}

// Grid of the tiled kernel: row groups of 256 rows times vocabulary chunks,
// about one workgroup per CU, chunk count a multiple of 8 (XCD pairing).
inline void tiled_grid(int M, int V, int cus, int* gx, int* gy) {
    const int groups = (M + tiled::kRowsPerWG - 1) / tiled::kRowsPerWG;
    const int ntiles = (V + tiled::kTileCols - 1) / tiled::kTileCols;
    int x = std::max(1, cus / groups);
    if (x >= 8) x -= x % 8;
    x = std::max(1, std::min(x, ntiles));
    *gx = x;
    *gy = groups;
}

template <int KS, typename BaseT, typename PriorT>
hipError_t launch_tiled_inst(const TiledKArgs& ka, int gx, int gy, hipStream_t s) {
    if (ka.V % tiled::kTileCols == 0)
        hipLaunchKernelGGL((fused_argmax_tiled_kernel<KS, BaseT, PriorT, true>), dim3(gx, gy, 1),
                           dim3(tiled::kThreads), 0, s, ka);
    else
        hipLaunchKernelGGL((fused_argmax_tiled_kernel<KS, BaseT, PriorT, false>), dim3(gx, gy, 1),
                           dim3(tiled::kThreads), 0, s, ka);
    return hipGetLastError();
}

template <typename BaseT>
hipError_t launch_tiled_for_base(const TiledKArgs& ka, int ksteps, int prior_kind, int gx, int gy, hipStream_t s) {
    auto by_prior = [&](auto ks_tag) -> hipError_t {
        constexpr int KS = decltype(ks_tag)::value;
        switch (prior_kind) {
            case 0: return launch_tiled_inst<KS, BaseT, no_prior_t>(ka, gx, gy, s);
            case 1: return launch_tiled_inst<KS, BaseT, float>(ka, gx, gy, s);
            case 2: return launch_tiled_inst<KS, BaseT, bf16_t>(ka, gx, gy, s);
            default: return launch_tiled_inst<KS, BaseT, f16_t>(ka, gx, gy, s);
        }
    };
    switch (ksteps) {
        case 8: return by_prior(std::integral_constant<int, 8>{});
        case 16: return by_prior(std::integral_constant<int, 16>{});
        default: return by_prior(std::integral_constant<int, 4>{});
    }
}

hipError_t launch_tiled_f32(const TiledKArgs& ka, int ksteps, int prior_kind, int gx, int gy, hipStream_t s);
hipError_t launch_tiled_bf16(const TiledKArgs& ka, int ksteps, int prior_kind, int gx, int gy, hipStream_t s);
hipError_t launch_tiled_f16(const TiledKArgs& ka, int ksteps, int prior_kind, int gx, int gy, hipStream_t s);

}  // namespace dels

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
// 32-vocabulary x 16-K slab of B, the B operand a 16-K x 32-row slab of rank.
// The 32 vocabulary rows of a tile enter the MFMA permuted (operand row
// m = 8a + 4h + q holds tile column 16h + 4a + q), so lane l ends up with row
// l%32 and the sixteen consecutive columns 16h .. 16h+15 (h = l/32).  One row
// per lane: the running argmax stays in the lane over the whole vocabulary
// chunk, visiting its candidates in increasing index order (a strict ">"
// keeps the lowest index of a tie).
//
// Workgroup: kWaves = 8 waves, 2 per SIMD.  Wave w keeps the rank operand of
// its 32 rows in VGPRs for the whole kernel (r/16 K steps x 16 bytes per
// lane); a workgroup covers 256 rows and a contiguous chunk of 32-column
// vocabulary tiles, one tile per pipeline stage.  Every byte the CUs take in
// counts: on MI355X a CU holds about 72 line requests in flight, so at the
// several hundred cycles a request takes under load the L2 -> CU ingress of the
// whole chip is near 6 TB/s, HBM hit or L2 hit alike.  256 rows per workgroup
// is the most the register file holds, so B enters twice at M = 512 (once per
// row group); everything else enters once, in whole 128-byte lines:
//  * B: a stage's tile (two consecutive 16-row block rows of the MFMA-16
//    layout, one contiguous run of HBM) is copied HBM -> LDS with direct-to-LDS
//    loads (global_load_lds_dwordx4, no VGPR staging) gathered into
//    K-step-major operand order: every operand read is one bank-conflict-free
//    KiB.  Two B buffers: the next stage's tile loads while one is contracted.
//  * base logits: in chunks of one whole 128-byte line per row (64 columns of
//    16-bit logits, 32 of fp32: two stages or one), eight rows per load, into
//    two chunk buffers -- the chunk after next loads while one is read.  A
//    row's 16-byte pieces are XOR-swizzled by the row so that the epilogue's
//    reads of 32 consecutive rows spread over the banks.  (A 32-column stage
//    of 16-bit logits would take half a line per row: twice the requests.)
//  * prior: each wave's copy of the stage's slice with the B tile.
// Each wave waits for its own loads with an explicit vmcnt count before the
// stage barrier (every wave issues the same loads, unconditionally, repeating
// the last tile past the chunk); with 16-bit logits the chunk loads issued
// last stay in flight through the barrier of the next (odd) stage.  The
// buffers are distinct LDS objects named statically in a four-stage unrolled
// loop, so the compiler can tell the reads of one buffer from the loads in
// flight into another and adds no waits of its own; with the schedule pinned
// (sched_barrier around each MFMA) a barrier per stage costs under 1 %.
//
// The combine + argmax of stage st-1 (the epilogue) runs between the MFMAs of
// stage st: its accumulators and base/prior values are held in registers
// (the latter read from LDS during st-1's own contraction), so the matrix core
// does not idle while a wave combines.
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
constexpr int kRowsPerWave = 32;
constexpr int kRowsPerWG = kWaves * kRowsPerWave;
constexpr int kTileCols = 32;
constexpr int kLineBytes = 128;                       // one base chunk row: a whole cache line
constexpr int kPriorBytesPerWave = 256;
constexpr int kOperandAhead = 4;

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

// Stages (32-column tiles) per base chunk: a chunk is one 128-byte line of
// every row, 64 columns of 16-bit logits or 32 of fp32.
template <typename BaseT>
constexpr int stages_per_chunk() { return kLineBytes / ((int)sizeof(BaseT) * kTileCols); }

// Vocabulary rows of a tile enter the 32x32 MFMAs permuted: operand row m (the
// lane's row l%32 of the A operand) holds tile column 16*((m>>2)&1) + 4*(m>>3) +
// (m&3), so that output lane l holds the consecutive columns 16h .. 16h+15.
// That column is row perm_row(m) of 16-row block row 2T + perm_block(m).
__device__ __forceinline__ int perm_block(int m) { return (m >> 2) & 1; }
__device__ __forceinline__ int perm_row(int m) { return 4 * (m >> 3) + (m & 3); }

// A base chunk in LDS: one 128-byte line per row, its 16-byte pieces rotated by
// the row, so that 32 consecutive rows read at one column spread over the banks.
__device__ __forceinline__ int line_swizzle(int r) { return (r >> 1) & 7; }
// Byte `byte` of row r's line.
__device__ __forceinline__ const char* line_at(const char* q, int r, int byte) {
    return q + r * kLineBytes + (((byte >> 4) ^ line_swizzle(r)) << 4) + (byte & 15);
}
// Direct-to-LDS load i (of kRowsPerWG / 8) of the chunk whose first column is
// col0: rows 8i .. 8i+7 of the workgroup (first row m_wg), each a whole line;
// lane L fetches piece (L%8) ^ swizzle of row 8i + L/8.  Rows past M repeat row
// M-1; columns past V are clamped into the row (their candidates are masked).
template <typename BaseT>
__device__ __forceinline__ void dma_base_lines(const TiledKArgs& a, int m_wg, int col0, int i, char* q) {
    constexpr int kPieceElems = 16 / (int)sizeof(BaseT);
    const int lane = threadIdx.x & 63;
    const int r = 8 * i + (lane >> 3);
    const int p = (lane & 7) ^ line_swizzle(r);
    const int col = min(col0 + p * kPieceElems, a.V - kPieceElems);
    const int m = min(m_wg + r, a.M - 1);
    dma16(a.base, (uint32_t)m * (uint32_t)a.ldbase * (uint32_t)sizeof(BaseT) + (uint32_t)col * (uint32_t)sizeof(BaseT),
          q + i * 1024);
}

}  // namespace tiled

// EXACT: V is a multiple of the 32-column tile, so no tile needs masking.
template <int KS, typename BaseT, typename PriorT, bool EXACT>
__global__ __launch_bounds__(tiled::kThreads) void fused_argmax_tiled_kernel(TiledKArgs a) {
#pragma clang fp contract(off)
    using namespace tiled;
    constexpr int kSteps = 2 * KS;                                   // 16-deep K steps
    constexpr bool kPrior = !is_no_prior<PriorT>::value;
    constexpr int SPC = stages_per_chunk<BaseT>();                   // 2 (16-bit base) or 1 (fp32)
    constexpr int kBPieces = kSteps / kWaves;                        // B blocks one wave loads per stage
    constexpr int kQPieces = kRowsPerWG * kLineBytes / 1024 / kWaves; // base chunk loads per wave (4)
    constexpr int kWB = sizeof(BaseT) == 4 ? 16 : 8;                 // words of a lane's 16 base values
    constexpr int kWP = sizeof(PriorT) == 4 ? 16 : 8;                // words of its 16 prior values
    constexpr int kAhead = kOperandAhead;                            // B operand reads in flight per wave
    static_assert(kSteps % kWaves == 0, "B blocks per stage must split over the waves");
    static_assert(SPC == 1 || SPC == 2, "a base chunk spans one or two stages");

    struct __attribute__((aligned(1024))) BBuf {
        char b[kSteps * 1024];                      // the stage's B tile, K-step-major operand order
        char prior[kWaves][kPriorBytesPerWave];     // each wave's copy of the stage's prior slice
    };
    struct __attribute__((aligned(1024))) QBuf {
        char q[kRowsPerWG * kLineBytes];            // one 128-byte line of base logits per row
    };
    __shared__ BBuf bb0, bb1;
    __shared__ QBuf qb0, qb1;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar control
    const int rl = lane & 31;       // row of this lane within the wave's 32 rows
    const int h = lane >> 5;        // K half of the operands / column half of the results
    const int m_wg = blockIdx.y * kRowsPerWG;
    const int mw = m_wg + wave * kRowsPerWave;                      // first row of this wave
    const bool wave_active = mw < a.M;

    // Vocabulary chunk of this workgroup: tiles [T0, T0 + nst), starting on a base
    // chunk boundary, so every base line it reads is whole.
    const int nunits = (a.ntiles + SPC - 1) / SPC;
    const int u0 = (int)(((int64_t)blockIdx.x * nunits) / gridDim.x);
    const int u1 = (int)(((int64_t)(blockIdx.x + 1) * nunits) / gridDim.x);
    const int T0 = u0 * SPC;
    const int nst = max(0, min(a.ntiles, u1 * SPC) - T0);
    const int last_chunk = max(nst - 1, 0) / SPC;
    // loads past the chunk (the unconditional ones of the last stages) repeat its last tile
    auto tile_of = [&](int st) { return min(T0 + min(st, max(nst - 1, 0)), a.ntiles - 1); };

    // Rank operand of the wave's rows, resident for the whole kernel; rows past
    // M repeat row M-1 (their results are not written).
    bf16x8 ra[kSteps];
    const int mrow = min(mw + rl, a.M - 1);
    {
        const uint16_t* rp =
            a.rank + rank_row_of(a.rank_rows, a.rank_rows_stride, a.rank_rows_count, mrow) * a.ldrank + h * 8;
#pragma unroll
        for (int s = 0; s < kSteps; ++s) ra[s] = load_bf16x8(rp + s * 16);
    }
    const float al = a.alpha[(int64_t)mrow * a.alpha_stride];
    const float be = a.beta[(int64_t)mrow * a.beta_stride];
    // beta == 0 skips the prior term: fma(0, +0, sc) == sc, whatever the prior holds;
    // prior bits kept or cleared: fp32/f16 mask, the high half of a 16-bit pair,
    // and the v_perm_b32 selector of the low half
    const bool use_prior = kPrior && be != 0.f;
    const float nbeta = use_prior ? -be : 0.f;
    const uint32_t pmask = use_prior ? 0xffffffffu : 0u;
    const uint32_t pmask_hi = use_prior ? 0xffff0000u : 0u;
    const uint32_t psel_lo = use_prior ? 0x01000c0cu : 0x0c0c0c0cu;   // bytes 1,0 -> 3,2; zeros below
    float best = -__builtin_inff();
    int bidx = INT_MAX;
    // Wait for the rank (and alpha/beta) loads here, before any direct-to-LDS
    // load is issued: the compiler's wait insertion does not see those asm
    // loads, and with tracked loads pending at the loop it would wait for
    // every stage load in flight before each MFMA.
    __builtin_amdgcn_s_waitcnt(0x0070 | (0xf << 8));   // vmcnt(0); expcnt and lgkmcnt left free

    const char* Bg = reinterpret_cast<const char*>(a.B);
    const char* priorg = static_cast<const char*>(a.prior);

    // B tile of stage st: the 32 vocabulary rows enter the MFMA permuted -- operand
    // row m = lane%32 holds tile column 16*((m>>2)&1) + 4*(m>>3) + (m&3) -- so that
    // lane l ends with the 16 consecutive columns 16h .. 16h+15 of its row.  LDS
    // block s (1 KiB) is the A operand of K step s in lane order (lane L: column
    // pi(L%32), K 16s + 8h .. +7), gathered from block row 2T + ((m>>2)&1).
    const int hh = perm_block(rl);
    const uint32_t b_lane = (uint32_t)((perm_row(rl) + 16 * h) * 16);
    auto issue_b = [&](BBuf& S, int st, int piece) {
        const int blk = min(2 * tile_of(st) + hh, a.nblk16 - 1);
        const int s = wave * kBPieces + piece;                      // K step of this load
        dma16(Bg, (uint32_t)blk * (uint32_t)(KS * 1024) + b_lane + (uint32_t)((s >> 1) * 1024 + (s & 1) * 512),
              S.b + s * 1024);
    };
    auto issue_prior = [&](BBuf& S, int st) {
        const int vs = tile_of(st) * kTileCols;
        if constexpr (sizeof(PriorT) == 4) {
            const int v = min(vs + (lane & 31), a.V - 1);
            dma4(priorg, (uint32_t)v * 4u, S.prior[wave]);
        } else {
            const int v = min(vs + 2 * (lane & 15), a.V - 2);
            dma4(priorg, (uint32_t)v * 2u, S.prior[wave]);
        }
    };
    // Base chunk c (clamped to the workgroup's last): whole lines of the rows.
    auto issue_q = [&](QBuf& Q, int c, int piece) {
        dma_base_lines<BaseT>(a, m_wg, (T0 + min(c, last_chunk) * SPC) * kTileCols, wave * kQPieces + piece, Q.q);
    };

    // Epilogue operands of one stage in registers: the base values of the lane's
    // candidates j = 0..15 (columns 16h + j; fp32 words, or 16-bit pairs with j in
    // word j/2) and their prior values.  Columns past V carry a -inf base.
    struct EpiRegs {
        uint32_t b[kWB];
        uint32_t p[kWP];
    };
    constexpr uint32_t kNegInf = sizeof(BaseT) == 4 ? 0xff800000u : half_neg_inf<BaseT>();
    // Group g (candidates 4g .. 4g+3) of stage st: base from the chunk line of the
    // lane's row, prior from the wave's slice.
    const int qrow = wave * kRowsPerWave + rl;
    auto load_epi_group = [&](const QBuf& Q, const BBuf& S, int st, int g, EpiRegs& e) {
        const int vs = tile_of(st) * kTileCols;
        const int v = vs + 16 * h + 4 * g;                           // column of candidate 4g
        const bool partial = !EXACT && vs + kTileCols > a.V;          // only the last tile of the vocabulary
        const char* src = line_at(Q.q, qrow, ((st % SPC) * kTileCols + 16 * h + 4 * g) * (int)sizeof(BaseT));
        if constexpr (sizeof(BaseT) == 4) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(src);
#pragma unroll
            for (int q = 0; q < 4; ++q) e.b[4 * g + q] = (partial && v + q >= a.V) ? kNegInf : w[q];
        } else {
            const uint2 w = *reinterpret_cast<const uint2*>(src);
            uint32_t w0 = w.x, w1 = w.y;
            if (partial) {
                w0 = v < a.V ? w0 : ((w0 & 0xffff0000u) | kNegInf);
                w0 = v + 1 < a.V ? w0 : ((w0 & 0xffffu) | (kNegInf << 16));
                w1 = v + 2 < a.V ? w1 : ((w1 & 0xffff0000u) | kNegInf);
                w1 = v + 3 < a.V ? w1 : ((w1 & 0xffffu) | (kNegInf << 16));
            }
            e.b[2 * g] = w0;
            e.b[2 * g + 1] = w1;
        }
        if constexpr (kPrior) {
            const char* pp = S.prior[wave] + (16 * h + 4 * g) * (int)sizeof(PriorT);
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
    };
    auto word_to_base = [&](uint32_t w, int j) -> float {
        if constexpr (sizeof(BaseT) == 4) return __uint_as_float(w);
        else return half_at<BaseT>(w, j & 1);
    };
    // Prior value of candidate j, as +0 for rows without the prior term.
    auto masked_prior = [&](uint32_t w, int j) -> float {
        if constexpr (sizeof(PriorT) == 4) {
            return __uint_as_float(w & pmask);
        } else if constexpr (std::is_same<PriorT, bf16_t>::value) {
            return __uint_as_float((j & 1) ? (w & pmask_hi) : __builtin_amdgcn_perm(w, w, psel_lo));
        } else {
            return __uint_as_float(__float_as_uint(half_at<PriorT>(w, j & 1)) & pmask);
        }
    };
    // Candidate j of the previous stage (first column cb).  The empty volatile asm
    // statements pin the candidate's work between the MFMAs: pure arithmetic is
    // otherwise gathered after the last MFMA of the stage.
    auto epi_one = [&](const f32x16& accp, const EpiRegs& e, int cb, int j) {
        float av = accp[j];
        float bv = word_to_base(e.b[sizeof(BaseT) == 4 ? j : (j >> 1)], j);
        asm volatile("" : "+v"(av), "+v"(bv));
        float sc = __builtin_fmaf(av, al, bv);
        if constexpr (kPrior) {
            float pv = masked_prior(e.p[sizeof(PriorT) == 4 ? j : (j >> 1)], j);
            asm volatile("" : "+v"(pv));
            sc = __builtin_fmaf(nbeta, pv, sc);
        }
        // candidates arrive in increasing column order: strict ">" keeps the lowest index
        const bool take = sc > best;
        best = take ? sc : best;
        bidx = take ? cb + j : bidx;
        asm volatile("" : "+v"(best), "+v"(bidx));
    };

    // Loads of stage st (issued during stage st - 1): B(st) and the prior slice
    // into S, and -- when st opens a base chunk's second-to-next stage -- base chunk
    // c into Q.  The chunk loads come last, so that a wait for B(st) can leave them
    // in flight.
    constexpr int kEB = kBPieces + (kPrior ? 1 : 0);
    auto issue_piece = [&](BBuf& S, int st_next, QBuf& Q, int c_next, int piece) {
        if (piece < kBPieces) issue_b(S, st_next, piece);
        else if (kPrior && piece == kBPieces) issue_prior(S, st_next);
        else issue_q(Q, c_next, piece - kEB);
    };

    // Contraction of stage st from S (one accumulation chain, operands read kAhead
    // steps ahead) with, spread between its MFMAs: the epilogue of the previous
    // stage (accp, ep, cbp), the reads of stage st's epilogue operands into epn
    // (group by group, each after the same group of ep is done), and the loads of
    // the next stage (E pieces: B and prior of st + 1, then base chunk c_next if
    // ISSUE_Q).
    auto contract = [&](auto issue_q_tag, const BBuf& S, const QBuf& Q, int st, BBuf& Sn, QBuf& Qn, int c_next,
                        f32x16& acc, const f32x16& accp, const EpiRegs& ep, int cbp, EpiRegs& epn) {
        constexpr bool ISSUE_Q = decltype(issue_q_tag)::value;
        constexpr int E = kEB + (ISSUE_Q ? kQPieces : 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[i] = 0.f;
        const char* ap = S.b + lane * 16;
        auto opnd = [&](int s) { return *reinterpret_cast<const bf16x8*>(ap + s * 1024); };
        bf16x8 opq[kAhead];
#pragma unroll
        for (int i = 0; i < kAhead; ++i) opq[i] = opnd(i < kSteps ? i : 0);
#pragma unroll
        for (int s = 0; s < kSteps; ++s) {
            const bf16x8 a0 = opq[s % kAhead];
            if (s + kAhead < kSteps) opq[s % kAhead] = opnd(s + kAhead);
            __builtin_amdgcn_sched_barrier(0);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, ra[s], acc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int c = s * 16 / kSteps; c < (s + 1) * 16 / kSteps; ++c) {
                epi_one(accp, ep, cbp, c);
                if ((c & 3) == 3) load_epi_group(Q, S, st, c >> 2, epn);
            }
#pragma unroll
            for (int piece = 0; piece < E; ++piece)
                if (s == piece * kSteps / E) issue_piece(Sn, st + 1, Qn, c_next, piece);
        }
    };
    auto issue_all = [&](auto issue_q_tag, BBuf& Sn, int st_next, QBuf& Qn, int c_next) {
        constexpr bool ISSUE_Q = decltype(issue_q_tag)::value;
        constexpr int E = kEB + (ISSUE_Q ? kQPieces : 0);
#pragma unroll
        for (int piece = 0; piece < E; ++piece) issue_piece(Sn, st_next, Qn, c_next, piece);
    };

    // Pipeline.  Prologue: B(0), prior(0) and base chunk 0.  At stage st every
    // wave waits for its own loads of B(st) -- the base chunk issued during the
    // previous stage may stay in flight (SPC = 2, st odd) -- the barrier publishes
    // st and frees the buffers of st - 1, and while st is contracted the loads of
    // B(st + 1) (and of base chunk st/SPC + 1 when st opens a chunk) are issued.
    // Loads past the chunk repeat its last tile into freed buffers, so every stage
    // issues the same loads and every wait count is fixed.  Four stages per loop
    // iteration name the buffers statically: B buffer st % 2, chunk buffer
    // (st / SPC) % 2.
    f32x16 acc_prev;
    EpiRegs ep_prev, ep_cur;
    int cb_prev = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc_prev[i] = 0.f;
#pragma unroll
    for (int i = 0; i < kWB; ++i) ep_prev.b[i] = sizeof(BaseT) == 4 ? kNegInf : kNegInf * 0x10001u;   // no-op epilogue
#pragma unroll
    for (int i = 0; i < kWP; ++i) ep_prev.p[i] = 0u;

    issue_all(std::true_type{}, bb0, 0, qb0, 0);
    for (int st0 = 0; st0 < nst; st0 += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int st = st0 + u;
            if (st >= nst) break;
            // the wait at the start of st: the chunk loads issued during st - 1 may stay in flight
            const bool q_in_flight = SPC == 2 && (u & 1) == 1;
            if (q_in_flight) stage_barrier<kQPieces>();
            else stage_barrier<0>();
            BBuf& S = (u & 1) ? bb1 : bb0;
            BBuf& Sn = (u & 1) ? bb0 : bb1;
            const int cbuf = SPC == 2 ? ((u >> 1) & 1) : (u & 1);
            const QBuf& Q = cbuf ? qb1 : qb0;
            QBuf& Qn = cbuf ? qb0 : qb1;
            const int c_next = st / SPC + 1;
            const bool opens = (st % SPC) == 0;                   // the next chunk's loads go out here
            if (wave_active) {
                f32x16 acc;
                if (opens) contract(std::true_type{}, S, Q, st, Sn, Qn, c_next, acc, acc_prev, ep_prev, cb_prev, ep_cur);
                else contract(std::false_type{}, S, Q, st, Sn, Qn, c_next, acc, acc_prev, ep_prev, cb_prev, ep_cur);
                acc_prev = acc;
                ep_prev = ep_cur;
                cb_prev = tile_of(st) * kTileCols + 16 * h;
            } else if (opens) {
                issue_all(std::true_type{}, Sn, st + 1, Qn, c_next);
            } else {
                issue_all(std::false_type{}, Sn, st + 1, Qn, c_next);
            }
        }
    }
    if (wave_active && nst > 0) {
        // the epilogue of the last stage
#pragma unroll
        for (int c = 0; c < 16; ++c) epi_one(acc_prev, ep_prev, cb_prev, c);
    }
    // no direct-to-LDS load may land after this point: the finish reuses the buffers
    __builtin_amdgcn_s_waitcnt(0x0070 | (0xf << 8));

    // merge the two column halves of each row (lanes l, l^32)
    {
        const float ov = __shfl_xor(best, 32, 64);
        const int oi = __shfl_xor(bidx, 32, 64);
        if (argmax_better(ov, oi, best, bidx)) {
            best = ov;
            bidx = oi;
        }
    }
    const int m = mw + rl;
    int fin_m[1] = {(h == 0 && m < a.M) ? m : -1};
    unsigned long long fin_key[1] = {bidx == INT_MAX ? 0ull : pack_argmax(best, (uint32_t)bidx)};
    tiled_argmax_finish(a, fin_m, fin_key, reinterpret_cast<int*>(&bb0));
}


// Grid of the tiled kernel: row groups of 256 rows times vocabulary chunks,
// about one workgroup per CU, chunk count a multiple of 8 (XCD pairing).
inline void tiled_grid(int M, int V, int cus, int* gx, int* gy) {
    const int groups = (M + tiled::kRowsPerWG - 1) / tiled::kRowsPerWG;
    const int ntiles = (V + tiled::kTileCols - 1) / tiled::kTileCols;
    int x = std::max(1, cus / groups);
    if (x >= 8) x -= x % 8;
    // at least one pair of tiles per chunk (a whole 128-byte line of 16-bit base logits)
    x = std::max(1, std::min(x, (ntiles + 1) / 2));
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

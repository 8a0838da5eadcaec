// The DeLS rollout as one launch with the low-rank head's B resident on chip.
//
// The rollout (code/kernel/dels.py:425-467: prefix GRU, then per step rank
// projection -> fused combine + argmax -> GRU on the chosen id, none after the
// last step) reads the same B [V, r] every step; per-step launches stream it
// from HBM each time (77.8 MB at V = 151936, r = 256: ~11 us of every ~24 us
// step).  Here one workgroup per CU holds its share of B for the whole
// rollout -- 4 vocabulary tiles of 16 rows per wave in VGPRs (the MFMA
// operand of every K step, 128 registers), up to 6 more per workgroup in LDS
// -- so a step moves only its base rows and a few tagged words:
//   * GRU: every workgroup owns G / nwg units (4 at G = 1024 on 256 CUs) and
//     keeps their W_hh rows in LDS as one 16-row MFMA operand per K step
//     (3 gates x units <= 16 rows); gh = h . W_hh^T + b_hh is summed per wave
//     over its K steps, then over the eight waves in a fixed order, rounded to
//     bf16 after the bias (as F.linear in bf16), and the gates combine with
//     the gathered input-table row (gru_unit);
//   * the new state goes out as words {tag, two bf16} (an agent-scope store
//     per word); every workgroup reads all of them into LDS (bounded
//     re-reads of words whose tag is not this step's);
//   * rank: workgroups 0 .. r/16 - 1 each own one 16-column tile of the rank
//     and keep its 16 rows of A in LDS; rank = bf16(act(bf16(h . A^T + b)))
//     goes out as words {tag, two bf16}, read by every workgroup;
//   * argmax: every wave contracts its resident tiles against the rank
//     (v_mfma_f32_16x16x32_bf16, lane l holding rows 4(l/16)+q of column
//     l%16), combines s = fma(-beta, prior, fma(dot, alpha, base)) as every
//     kernel of the path does, and keeps a running (score, index) per lane;
//     the workgroup publishes each row's best as one slot word (order(score)
//     in the high half, ~index above two flag bits in the low half, so the
//     larger word is the argmax with ties to the lower index) and every
//     workgroup reads all nwg slots of each row, takes the maximum and so
//     knows the step's ids for its GRU units.  Each workgroup owns its slots
//     (no two workgroups write one address: no atomics queue on a hot word).
// Pacing the exchanges: every read issues all its loads before it examines
// any (a value consumed as soon as it is loaded would cost one memory round
// trip per word instead of one per read).
// The tag of a state or rank word is a function of the launch generation and
// the step, and the words live in a workspace region no other kernel writes,
// so a word of an earlier step or launch never passes.  Slot words alternate
// between two sets by step parity and carry bit 1 of the step; a launch first
// clears its own slots (returning exchanges, complete before the workgroup
// publishes its first state words, which every reader waits for), so a slot
// holds zero, this launch's word for the step or its word of two steps
// before.  Every wait is bounded: a wait that runs out sets a sticky error
// word, every other wait sees it and stops, the remaining ids are written as
// -1, and the launch still ends (every workgroup reaches the end, the last
// one resets the error word and advances the generation).  The workgroups
// must be resident at once (one per CU) for the waits to succeed.
#include <algorithm>
#include <climits>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

namespace {

constexpr int kRrWaves = 8;
constexpr int kRrThreads = kRrWaves * 64;
constexpr int kRrKs = kResidentRank / 32;             // K steps of 32 over r
constexpr int kRrRegTiles = 4;                        // vocabulary tiles per wave in registers
constexpr int kRrRankWGs = kResidentRank / 16;        // rank column tiles, one workgroup each
constexpr int kRrHPitch = kResidentMaxG + 8;          // bf16 per row of the state in LDS (rows 16 B apart in banks)
constexpr int kRrRPitch = kResidentRank + 8;          // bf16 per row of the rank in LDS
constexpr int kRrUnionBytes = std::max(kResidentLdsTiles * kRrKs * 1024, (kResidentMaxG / 32) * 1024);

// control area: one 128-byte line (32 words) per counter
constexpr int kRrDoneCounter = 250 * 32;
constexpr int kRrErrorWord = 251 * 32;

struct RrArgs {
    const uint16_t* w_hh; const uint16_t* b_hh;     // [3G, G] MFMA-16 blocks, [3G] or null
    const uint16_t* A; const uint16_t* rank_b;      // [r, G] MFMA-16 blocks, [r] or null
    int act;
    const uint16_t* B;                              // [V, r] MFMA-16 blocks
    const uint16_t* gi_table; int64_t ld_gi; int64_t table_rows;
    const int64_t* prefix; int64_t ld_prefix;       // row m at prefix[m * ld_prefix]
    const void* base; int64_t ld_base;              // row m, step s at base + m * ld_base + s * V (elements)
    const void* prior;
    const float* alpha; const float* beta;          // [steps]
    int M, G, V, steps, ntiles, upw;                // upw: GRU units per workgroup
    int mp_shift;                                   // log2 of M rounded up to a power of two
    int np_shift;                                   // log2(upw / 2): state words per row and workgroup
    int64_t* out_ids; float* out_scores;            // row m, step s at [m * ld_out + s]
    int64_t ld_out;
    unsigned int* counters;                         // control area
    unsigned long long* h_words;                    // per workgroup: rows x upw/2 words, on lines of its own
    unsigned long long* rank_words;                 // per rank workgroup: rows x 8 words
    unsigned long long* slots;                      // [2][nwg][16]: parity, workgroup (a line each), row
    int spin_limit;
};

constexpr int kRrSlotSet = 16 * kResidentMaxWGs;    // words per parity set

__device__ __forceinline__ uint32_t rr_tag(uint32_t gen, int step) {
    const uint32_t x = gen * 256u + (uint32_t)step + 1u;
    const uint32_t t = x * 0x2C1B3C6Du;
    return t == 0u ? 0x5bd1e995u : t;
}

__device__ __forceinline__ bool rr_failed(const RrArgs& a) {
    return __hip_atomic_load(a.counters + kRrErrorWord, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0u;
}
__device__ __forceinline__ void rr_fail(const RrArgs& a) {
    __hip_atomic_store(a.counters + kRrErrorWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Where a reader finds the words of one exchange.  Every producer writes its
// words as one block (rows x words per row, the rows rounded up to a power of
// two) starting on its own 128-byte line or lines: when one line gathers words
// of many producers, their writes and the readers' polls of it queue behind one
// another (an all-to-all of 256 x 8 words takes ~1.9 us with a line per
// producer, ~3.4 us with sixteen producers per line).  The reader numbers the
// words j < n = producers << blk and takes them in that order.
struct RrWords {
    int n;        // words the reader takes
    int blk;      // log2 of one producer's block (rows rounded up x words per row)
    int stride;   // log2 of the words from one producer's block to the next (>= blk)
    int row;      // log2 of the words per row
    int mp;       // log2 of the rows rounded up
    int M;        // rows present
    __device__ __forceinline__ uint32_t addr(int j) const {
        j = j < n ? j : n - 1;   // past the end: the last word again (loaded, never examined)
        return ((uint32_t)(j >> blk) << stride) + (uint32_t)(j & ((1 << blk) - 1));
    }
    __device__ __forceinline__ int row_of(int j) const { return (j >> row) & ((1 << mp) - 1); }
    __device__ __forceinline__ bool live(int j) const { return j < n && row_of(j) < M; }
};

// Load the words j = tid + kRrThreads * i, i < NPT -- every load issued before
// any value is examined -- then re-read the live ones that `arrived` rejects,
// at most spin_limit rounds.  False when they did not all arrive or another
// workgroup reported a failure (this thread's view).
template <int NPT, typename Arrived>
__device__ __forceinline__ bool rr_gather(const RrArgs& a, const unsigned long long* src, const RrWords& pl, int tid,
                                          unsigned long long (&w)[NPT], Arrived arrived) {
    static_assert(NPT <= 32, "one bit per word in a 32-bit mask");
#pragma unroll
    for (int i = 0; i < NPT; ++i)
        w[i] = __hip_atomic_load(src + pl.addr(tid + kRrThreads * i), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t missing = 0;
#pragma unroll
    for (int i = 0; i < NPT; ++i)
        if (pl.live(tid + kRrThreads * i)) missing |= (uint32_t)!arrived(w[i]) << i;
    int it = 0;
    while (missing != 0) {
        // poll the first missing word alone (one load per thread and round, not
        // one per missing word: the polls of every workgroup share the memory
        // system with the words being written), then re-read the rest once
        const int f = __builtin_ctz(missing);
        const unsigned long long* pf = src + pl.addr(tid + kRrThreads * f);
        for (;;) {
            if (it >= a.spin_limit) return false;
            if ((it & 63) == 63 && rr_failed(a)) return false;
            ++it;
            __builtin_amdgcn_s_sleep(2);
            if (arrived(__hip_atomic_load(pf, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))) break;
        }
#pragma unroll
        for (int i = 0; i < NPT; ++i)
            if ((missing >> i) & 1u)
                w[i] = __hip_atomic_load(src + pl.addr(tid + kRrThreads * i), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        uint32_t still = 0;
#pragma unroll
        for (int i = 0; i < NPT; ++i)
            if ((missing >> i) & 1u) still |= (uint32_t)!arrived(w[i]) << i;
        missing = still;
    }
    return true;
}

// Read the tagged words of `pl` until every live one carries `tag` (word j to
// the LDS pair slot map(j)); all threads.  Returns false (for every thread)
// when they did not all arrive.  Ends with a barrier.
template <int NPT, typename Map>
__device__ __forceinline__ bool rr_read_words(const RrArgs& a, const unsigned long long* src, const RrWords& pl,
                                              uint32_t tag, Map map) {
    // the thread index passes through an empty asm statement so that the word
    // addresses are formed here, not held in registers across the caller's loop
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    unsigned long long w[NPT];
    const bool got = rr_gather<NPT>(a, src, pl, tid, w,
                                    [&](unsigned long long x) { return (uint32_t)(x >> 32) == tag; });
    if (got) {
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
            const int j = tid + kRrThreads * i;
            if (pl.live(j)) *map(j) = (uint32_t)w[i];
        }
    }
    return !__syncthreads_or(!got);
}

// The step's slot words (one per row and workgroup, `pl` with one word per row)
// once every live one carries the step's flag bits `low2`; each row's maximum
// into s_rowmax[row] (an LDS maximum, s_rowmax zero before).  All threads;
// false for every thread when they did not all arrive.  Ends with a barrier.
template <int NPT>
__device__ __forceinline__ bool rr_slot_maxima(const RrArgs& a, const unsigned long long* src, const RrWords& pl,
                                               uint32_t low2, unsigned long long* s_rowmax) {
    int tid = threadIdx.x;
    asm volatile("" : "+v"(tid));
    unsigned long long w[NPT];
    const bool got = rr_gather<NPT>(a, src, pl, tid, w,
                                    [&](unsigned long long x) { return ((uint32_t)x & 3u) == low2; });
    // word j holds row j mod 2^mp, so lanes with equal low mp bits share a row
    const int lane = tid & 63;
    unsigned long long k = 0;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const unsigned long long v = got && pl.live(tid + kRrThreads * i) ? w[i] : 0ull;
        k = v > k ? v : k;
    }
    for (int off = 1 << pl.mp; off < 64; off <<= 1) {
        const unsigned long long o = __shfl_xor(k, off, 64);
        k = o > k ? o : k;
    }
    if (lane < pl.M && lane < (1 << pl.mp)) atomicMax(&s_rowmax[lane], k);
    return !__syncthreads_or(!got);
}

// One step of a maximum over the 16 lanes of each DPP row of 64-bit argmax keys
// (pack_argmax): every lane takes the larger of its key and that of the lane K
// below it in its row (lanes with none read key 0, the lowest).  After K = 1,
// 2, 4, 8 lane 15 of a row holds the row's best.
template <int K>
__device__ __forceinline__ void rr_row_max(unsigned long long& k) {
    constexpr int kRowShr = 0x110 + K;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)k, kRowShr, 0xf, 0xf, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(k >> 32), kRowShr, 0xf, 0xf, true);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    k = o > k ? o : k;
}

template <typename BaseT, typename PriorT>
__global__ __launch_bounds__(kRrThreads) void rollout_resident_kernel(RrArgs a) {
#pragma clang fp contract(off)
    __shared__ __attribute__((aligned(16))) uint16_t s_h[16 * kRrHPitch];        // the state, rows >= M zero
    __shared__ __attribute__((aligned(16))) char s_whh[(kResidentMaxG / 32) * 1024];   // W_hh rows of the units
    __shared__ __attribute__((aligned(16))) char s_union[kRrUnionBytes];       // A rows (rank WGs) or B tiles
    __shared__ __attribute__((aligned(16))) uint16_t s_rank[16 * kRrRPitch];
    __shared__ __attribute__((aligned(16))) float s_red[kRrWaves * 256];
    __shared__ float s_prior[(kRrWaves * kRrRegTiles + kResidentLdsTiles) * 16];
    __shared__ unsigned long long s_key[kRrWaves][16];    // each wave's best key of each row
    __shared__ float s_gh[16 * 16];
    __shared__ float s_ab[2][kResidentMaxSteps];          // alpha, beta of each step
    __shared__ float s_bias[32];                          // b_hh of the operand rows, rank bias of the tile
    __shared__ unsigned long long s_rowmax[16];           // the step's maximum slot word of each row
    __shared__ int64_t s_ids[16];
    __shared__ int s_flag;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kg = lane >> 4;
    const int w = blockIdx.x, nwg = gridDim.x;
    const int G = a.G, KB = G / 32, M = a.M, V = a.V;
    const uint32_t gen = __hip_atomic_load(a.counters + kDecodeGenWord, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const BaseT* base = static_cast<const BaseT*>(a.base);
    const PriorT* prior = static_cast<const PriorT*>(a.prior);
    const bool rank_wg = w < kRrRankWGs;

    // ---- this workgroup's vocabulary tiles [T0, T1): 32 for a rank workgroup, the
    // rest shared evenly by the others (the plan checks they fit)
    int T0, T1;
    {
        const int first = min(a.ntiles, kRrRankWGs * kRrWaves * kRrRegTiles);
        if (rank_wg) {
            T0 = min(a.ntiles, w * kRrWaves * kRrRegTiles);
            T1 = min(a.ntiles, T0 + kRrWaves * kRrRegTiles);
        } else {
            const int rest = a.ntiles - first, j = w - kRrRankWGs, n = nwg - kRrRankWGs;
            T0 = first + (int)(((int64_t)j * rest) / n);
            T1 = first + (int)(((int64_t)(j + 1) * rest) / n);
        }
    }
    const int ntl = T1 - T0;
    // register tile j of this wave: T0 + wave + 8 j; LDS tile e (e < ntl - 32): T0 + 32 + e, contracted by wave e
    const int nlds = max(0, ntl - kRrWaves * kRrRegTiles);
    const bool has_lds_tile = wave < nlds;

    const int u0 = w * a.upw;   // this workgroup's first GRU unit
    for (int i = threadIdx.x; i < 16 * kRrHPitch / 2; i += kRrThreads) reinterpret_cast<uint32_t*>(s_h)[i] = 0u;
    for (int i = threadIdx.x; i < 16 * kRrRPitch / 2; i += kRrThreads) reinterpret_cast<uint32_t*>(s_rank)[i] = 0u;
    for (int i = threadIdx.x; i < a.steps; i += kRrThreads) {
        s_ab[0][i] = a.alpha[i];
        s_ab[1][i] = a.beta[i];
    }
    if (threadIdx.x < 16) {
        const int j = threadIdx.x;
        float bh = 0.f, br = 0.f;
        if (a.b_hh && j < 3 * a.upw) {
            const int g = j / a.upw, u = u0 + (j - g * a.upw);
            bh = bf16_bits_to_f32(a.b_hh[g * G + u]);
        }
        if (rank_wg && a.rank_b) br = bf16_bits_to_f32(a.rank_b[w * 16 + j]);
        s_bias[j] = bh;
        s_bias[16 + j] = br;
        s_rowmax[j] = 0ull;
    } else if (threadIdx.x < 48) {
        // this workgroup's slots of both parity sets back to zero; waiting for the
        // old values means the exchanges are done before the barrier below, so
        // before the prefix state words that every reader waits for
        const int p = (threadIdx.x - 16) >> 4, m = threadIdx.x & 15;
        const unsigned long long old = __hip_atomic_exchange(a.slots + p * kRrSlotSet + w * 16 + m, 0ull,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(old));
    }
    __syncthreads();

    // ---- the exchanges' word blocks: the state (upw / 2 words per row and
    // workgroup, each workgroup on lines of its own), the rank (8 words per row
    // and rank workgroup), the argmax slots (one word per row and workgroup, a
    // line per workgroup)
    const int mp = a.mp_shift;
    const RrWords h_pl{nwg << (mp + a.np_shift), mp + a.np_shift, max(4, mp + a.np_shift), a.np_shift, mp, M};
    const RrWords r_pl{kRrRankWGs << (mp + 3), mp + 3, mp + 3, 3, mp, M};
    const RrWords s_pl{nwg << mp, mp, 4, 0, mp, M};

    // ---- pieces of a step ----------------------------------------------------------
    // gh of the workgroup's units from the state in s_h (zero previous state:
    // no product) into s_gh[m * 16 + j], bf16-rounded after the bias.
    auto compute_gh = [&](bool zero_state) __attribute__((always_inline)) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        if (!zero_state) {
            for (int kb = wave; kb < KB; kb += kRrWaves) {
                const bf16x8 hv = *reinterpret_cast<const bf16x8*>(&s_h[col * kRrHPitch + kb * 32 + kg * 8]);
                const bf16x8 wv = *reinterpret_cast<const bf16x8*>(s_whh + kb * 1024 + lane * 16);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hv, wv, acc, 0, 0, 0);
            }
        }
        *reinterpret_cast<f32x4*>(&s_red[wave * 256 + lane * 4]) = acc;
        __syncthreads();
        if (threadIdx.x < 256) {
            // element (row m, operand row j): lane (m/4)*16 + j, entry m%4
            const int m = threadIdx.x >> 4, j = threadIdx.x & 15;
            const int e = (((m >> 2) * 16 + j) << 2) + (m & 3);
            float v = s_red[e];
#pragma unroll
            for (int ww = 1; ww < kRrWaves; ++ww) v = v + s_red[ww * 256 + e];
            if (a.b_hh) v = v + s_bias[j];
            s_gh[m * 16 + j] = round_bf16(v);
        }
        __syncthreads();
    };
    // the workgroup's units of the next state for tokens tok[m], published as words
    auto gru_publish = [&](const int64_t* tok, int64_t tok_stride, uint32_t tag) __attribute__((always_inline)) {
        const int np = a.upw / 2;   // words per row
        if ((int)threadIdx.x < M * np) {
            const int m = threadIdx.x / np, p = threadIdx.x - m * np;
            int64_t t = tok[(int64_t)m * tok_stride];
            t = t < 0 ? 0 : (t >= a.table_rows ? a.table_rows - 1 : t);
            const uint16_t* gi = a.gi_table + t * a.ld_gi + u0 + 2 * p;
            // the six input-table values first: one memory round trip
            uint16_t gv[3][2];
#pragma unroll
            for (int g = 0; g < 3; ++g)
#pragma unroll
                for (int h = 0; h < 2; ++h) gv[g][h] = gi[g * G + h];
            uint32_t pair = 0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int i = 2 * p + h, u = u0 + i;
                const float hv = bf16_bits_to_f32(s_h[m * kRrHPitch + u]);
                const float v = gru_unit(bf16_bits_to_f32(gv[0][h]), bf16_bits_to_f32(gv[1][h]),
                                         bf16_bits_to_f32(gv[2][h]), s_gh[m * 16 + i],
                                         s_gh[m * 16 + a.upw + i], s_gh[m * 16 + 2 * a.upw + i], hv);
                pair |= (uint32_t)f32_to_bf16_bits(v) << (16 * h);
            }
            __hip_atomic_store(a.h_words + h_pl.addr((m << a.np_shift) + p + (w << h_pl.blk)),
                               ((unsigned long long)tag << 32) | pair, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    // every row's state from the words into s_h
    auto read_state = [&](uint32_t tag) __attribute__((always_inline)) -> bool {
        auto map = [&](int j) {
            const int m = h_pl.row_of(j), wp = j >> h_pl.blk, p = j & ((1 << a.np_shift) - 1);
            return reinterpret_cast<uint32_t*>(&s_h[m * kRrHPitch + wp * a.upw + 2 * p]);
        };
        // as few loads per thread as cover the words
        if (h_pl.n <= 4 * kRrThreads) return rr_read_words<4>(a, a.h_words, h_pl, tag, map);
        if (h_pl.n <= 8 * kRrThreads) return rr_read_words<8>(a, a.h_words, h_pl, tag, map);
        return rr_read_words<16>(a, a.h_words, h_pl, tag, map);
    };
    // rank workgroup: its 16 columns of the rank from s_h, published as words
    auto rank_publish = [&](uint32_t tag) __attribute__((always_inline)) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int kb = wave; kb < KB; kb += kRrWaves) {
            const bf16x8 hv = *reinterpret_cast<const bf16x8*>(&s_h[col * kRrHPitch + kb * 32 + kg * 8]);
            const bf16x8 av = *reinterpret_cast<const bf16x8*>(s_union + kb * 1024 + lane * 16);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hv, av, acc, 0, 0, 0);
        }
        *reinterpret_cast<f32x4*>(&s_red[wave * 256 + lane * 4]) = acc;
        __syncthreads();
        if (threadIdx.x < 128) {
            const int m = threadIdx.x >> 3, p = threadIdx.x & 7;
            if (m < M) {
                uint32_t pair = 0;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const int n = 2 * p + h;
                    const int e = (((m >> 2) * 16 + n) << 2) + (m & 3);
                    float v = s_red[e];
#pragma unroll
                    for (int ww = 1; ww < kRrWaves; ++ww) v = v + s_red[ww * 256 + e];
                    if (a.rank_b) v = v + s_bias[16 + n];
                    v = round_bf16(v);
                    if (a.act == 1) v = round_bf16(silu_f32(v));
                    pair |= (uint32_t)f32_to_bf16_bits(v) << (16 * h);
                }
                __hip_atomic_store(a.rank_words + r_pl.addr((w << r_pl.blk) + (m << 3) + p),
                                   ((unsigned long long)tag << 32) | pair, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
        __syncthreads();   // s_red is reused
    };
    auto read_rank = [&](uint32_t tag) __attribute__((always_inline)) -> bool {
        auto map = [&](int j) {
            const int m = r_pl.row_of(j), wr = j >> r_pl.blk, p = j & 7;
            return reinterpret_cast<uint32_t*>(&s_rank[m * kRrRPitch + wr * 16 + 2 * p]);
        };
        if (r_pl.n <= 2 * kRrThreads) return rr_read_words<2>(a, a.rank_words, r_pl, tag, map);
        return rr_read_words<4>(a, a.rank_words, r_pl, tag, map);
    };


    // ---- prefix: h_0 = GRU(gi_table[prefix], 0) --------------------------------
    bool ok = true;
    compute_gh(true);
    gru_publish(a.prefix, a.ld_prefix, rr_tag(gen, 0));

    // ---- resident operands, loaded while the prefix state travels (a read
    // waits for every load issued before it, so the state went out first):
    // the LDS operands, then this wave's register tiles of B
    if (rank_wg) {
        // A rows 16 w .. 16 w + 15: the MFMA-16 blocks of that row block, in order
        for (int i = threadIdx.x; i < KB * 64; i += kRrThreads) {
            const int kb = i >> 6, l = i & 63;
            *reinterpret_cast<u32x4*>(s_union + kb * 1024 + l * 16) =
                *reinterpret_cast<const u32x4*>(a.A + ((int64_t)w * KB + kb) * 512 + l * 8);
        }
    } else {
        for (int i = threadIdx.x; i < nlds * kRrKs * 64; i += kRrThreads) {
            const int e = i / (kRrKs * 64), rem = i - e * (kRrKs * 64), s = rem >> 6, l = rem & 63;
            const int t = T0 + kRrWaves * kRrRegTiles + e;
            *reinterpret_cast<u32x4*>(s_union + (e * kRrKs + s) * 1024 + l * 16) =
                *reinterpret_cast<const u32x4*>(a.B + ((int64_t)t * kRrKs + s) * 512 + l * 8);
        }
    }
    // W_hh rows of units u0 .. u0 + upw - 1: operand row j = g * upw + i holds row
    // g * G + u0 + i of W_hh (rows past 3 upw are zero)
    for (int i = threadIdx.x; i < KB * 64; i += kRrThreads) {
        const int kb = i >> 6, l = i & 63;
        const int j = l & 15, oct = l >> 4;
        u32x4 v = {0u, 0u, 0u, 0u};
        if (j < 3 * a.upw) {
            const int g = j / a.upw, row = g * G + u0 + (j - g * a.upw);
            v = *reinterpret_cast<const u32x4*>(a.w_hh + ((int64_t)(row >> 4) * KB + kb) * 512 + ((row & 15) + 16 * oct) * 8);
        }
        *reinterpret_cast<u32x4*>(s_whh + kb * 1024 + l * 16) = v;
    }
    // the prior of every column of the workgroup's tiles (widened)
    for (int i = threadIdx.x; i < ntl * 16; i += kRrThreads) {
        const int v = min(T0 * 16 + i, V - 1);
        if constexpr (is_no_prior<PriorT>::value) s_prior[i] = 0.f;
        else s_prior[i] = widen_raw<PriorT>(load_raw(prior + v));
    }
    // the register tiles after the LDS operands (whose stores wait for their loads)
    asm volatile("" ::: "memory");
    bf16x8 bt[kRrRegTiles][kRrKs];
#pragma unroll
    for (int j = 0; j < kRrRegTiles; ++j) {
        // a tile that is not this wave's loads the last tile (in bounds) and keeps zeros
        const int ti = wave + 8 * j;
        const int t = min(T0 + ti, a.ntiles - 1);
        const uint32_t keep = ti < ntl ? ~0u : 0u;
#pragma unroll
        for (int s = 0; s < kRrKs; ++s)
            bt[j][s] = masked_bf16x8(__builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
                                         a.B + ((int64_t)t * kRrKs + s) * 512 + lane * 8)),
                                     keep);
    }

    ok = read_state(rr_tag(gen, 0));

    int s = 0;
    for (; ok && s < a.steps; ++s) {
        const uint32_t tag = rr_tag(gen, s);
        // lane values pass through an empty asm statement each step, so that the
        // compiler forms the step's addresses here instead of holding them in
        // registers across the loop
        int lcol = col, lkg = kg;
        asm volatile("" : "+v"(lcol), "+v"(lkg));
        if (rank_wg) rank_publish(tag);
        // base values of this wave's tiles (issued before the rank wait): the
        // wave-uniform start of each tile's columns plus one per-lane offset per row
        uint32_t braw[kRrRegTiles + 1][4];
        {
            const BaseT* bs = base + (int64_t)s * V;
#pragma unroll
            for (int j = 0; j <= kRrRegTiles; ++j) {
                const int ti = j < kRrRegTiles ? wave + 8 * j : kRrWaves * kRrRegTiles + wave;
                const int tc = min(T0 + min(ti, max(ntl - 1, 0)), a.ntiles - 1);
                const int vc = min(tc * 16 + lcol, V - 1);
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int m = 4 * lkg + q;
                    braw[j][q] = load_raw(bs + (int64_t)(m < M ? m : 0) * a.ld_base + vc);
                }
            }
        }
        // keep these loads ahead of the rank wait (the compiler would otherwise
        // issue them after it, where their round trip adds to the step)
        asm volatile("" ::: "memory");
        ok = read_rank(tag);
        if (!ok) break;

        // ---- argmax over the resident tiles -------------------------------------
        // K step outermost: each rank operand is read from LDS once and feeds
        // every tile's accumulator
        const float al = s_ab[0][s], be = s_ab[1][s];
        const bool use_prior = !is_no_prior<PriorT>::value && be != 0.f;
        const bool lds_tile = !rank_wg && has_lds_tile;
        f32x4 acc[kRrRegTiles + 1];
#pragma unroll
        for (int j = 0; j <= kRrRegTiles; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        // unconditional contractions (no branches between the MFMAs): a tile that
        // is not this wave's holds zeros, or for the LDS slot of a wave without
        // one any data, and is not combined
        const int lslot = lds_tile ? wave : 0;
#pragma unroll
        for (int k = 0; k < kRrKs; ++k) {
            const bf16x8 rk = *reinterpret_cast<const bf16x8*>(&s_rank[lcol * kRrRPitch + k * 32 + lkg * 8]);
            const bf16x8 bv = *reinterpret_cast<const bf16x8*>(s_union + (lslot * kRrKs + k) * 1024 + lane * 16);
#pragma unroll
            for (int j = 0; j < kRrRegTiles; ++j)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rk, bt[j][k], acc[j], 0, 0, 0);
            acc[kRrRegTiles] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(rk, bv, acc[kRrRegTiles], 0, 0, 0);
        }
        float best[4];
        int bidx[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) { best[q] = -__builtin_inff(); bidx[q] = INT_MAX; }
        // a lane's column grows with its tile number, so a later tile takes the
        // lead only on a larger score, or on an equal one while nothing has
        // (the first -inf); written with bitwise tests, no branches
#pragma unroll
        for (int j = 0; j <= kRrRegTiles; ++j) {
            const int ti = j < kRrRegTiles ? wave + 8 * j : kRrWaves * kRrRegTiles + wave;
            const bool live = j < kRrRegTiles ? ti < ntl : lds_tile;   // wave-uniform
            const int tc = min(ti, max(ntl - 1, 0));
            const int v = (T0 + tc) * 16 + lcol;
            const bool livev = live & (v < V);
            const float pv = s_prior[tc * 16 + lcol];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float sc = __builtin_fmaf(acc[j][q], al, widen_raw<BaseT>(braw[j][q]));
                if (use_prior) sc = __builtin_fmaf(-be, pv, sc);
                const bool take = livev & ((sc > best[q]) | ((sc == best[q]) & (bidx[q] == INT_MAX)));
                best[q] = take ? sc : best[q];
                bidx[q] = take ? v : bidx[q];
            }
        }
        // over the 16 columns of each row as argmax keys (a lane without a
        // candidate holds -inf at index INT_MAX, below every real one; DPP row
        // shifts: lane 15 of a row ends with the row's best), then (below) the waves
        unsigned long long key[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            key[q] = pack_argmax(best[q], (uint32_t)bidx[q]);
            rr_row_max<1>(key[q]);
            rr_row_max<2>(key[q]);
            rr_row_max<4>(key[q]);
            rr_row_max<8>(key[q]);
        }
        if (col == 15) {
#pragma unroll
            for (int q = 0; q < 4; ++q) s_key[wave][4 * kg + q] = key[q];
        }
        __syncthreads();
        // the workgroup's best of each row into its slot word for the step
        const uint32_t low2 = 1u | ((((uint32_t)s >> 1) & 1u) << 1);
        unsigned long long* slot_set = a.slots + (s & 1) * kRrSlotSet;
        if ((int)threadIdx.x < M) {
            const int m = threadIdx.x;
            unsigned long long k = s_key[0][m];   // order(score) << 32 | ~index
#pragma unroll
            for (int ww = 1; ww < kRrWaves; ++ww) k = max(k, s_key[ww][m]);
            // no candidate (index INT_MAX) leaves the index field zero: index
            // 2^30 - 1, past every vocabulary, below every real candidate
            const unsigned long long word =
                low2 | (k & 0xffffffff00000000ull) | ((unsigned long long)((uint32_t)k & 0x3fffffffu) << 2);
            __hip_atomic_store(slot_set + w * 16 + m, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }

        // next step's gh while the slot words travel (every workgroup: placed
        // before the rank wait it would delay the rank workgroups' argmax, and
        // with it every workgroup's slot read)
        if (s + 1 < a.steps) compute_gh(false);

        // ---- the step's ids (every workgroup: its GRU units need them) ---------------
        const bool need = s + 1 < a.steps || w == 0;
        if (need) {
            if (s_pl.n <= 2 * kRrThreads) ok = rr_slot_maxima<2>(a, slot_set, s_pl, low2, s_rowmax);
            else if (s_pl.n <= 4 * kRrThreads) ok = rr_slot_maxima<4>(a, slot_set, s_pl, low2, s_rowmax);
            else ok = rr_slot_maxima<8>(a, slot_set, s_pl, low2, s_rowmax);
            if (!ok) break;
            if (threadIdx.x < 16) {
                const int m = threadIdx.x;
                int64_t id = 0;
                float val = -__builtin_inff();
                if (m < M) {
                    const unsigned long long key = s_rowmax[m];
                    s_rowmax[m] = 0ull;   // for the next step (barriers come between)
                    const uint32_t idx = ~(uint32_t)(key >> 2) & 0x3fffffffu;
                    if (idx < (uint32_t)V) {
                        id = idx;
                        val = f32_from_order_key((uint32_t)(key >> 32));
                    }
                    if (w == 0) {
                        a.out_ids[(int64_t)m * a.ld_out + s] = id;
                        if (a.out_scores) a.out_scores[(int64_t)m * a.ld_out + s] = val;
                    }
                }
                s_ids[m] = id;
            }
            __syncthreads();
        }
        if (s + 1 < a.steps) {
            gru_publish(s_ids, 1, rr_tag(gen, s + 1));
            ok = read_state(rr_tag(gen, s + 1));
        }
    }
    if (!ok) {
        if (threadIdx.x == 0) rr_fail(a);
        // the ids this launch could not produce
        if (w == 0) {
            for (int i = threadIdx.x; i < M * a.steps; i += kRrThreads) {
                const int m = i / a.steps, st = i - m * a.steps;
                if (st >= s) {
                    a.out_ids[(int64_t)m * a.ld_out + st] = -1;
                    if (a.out_scores) a.out_scores[(int64_t)m * a.ld_out + st] = -__builtin_inff();
                }
            }
        }
    }

    // ---- the last workgroup clears the control area and advances the generation
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.counters + kRrDoneCounter, 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_flag = prev == (unsigned)nwg - 1 ? 3 : 0;
    }
    __syncthreads();
    if (s_flag != 3) return;
    if (threadIdx.x == 0) {
        __hip_atomic_store(a.counters + kRrErrorWord, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.counters + kRrDoneCounter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(a.counters + kDecodeGenWord, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <typename BaseT>
hipError_t launch_rr_base(const RrArgs& a, int prior_kind, int nwg, hipStream_t s) {
    const dim3 grid(nwg), block(kRrThreads);
    switch (prior_kind) {
        case 0: hipLaunchKernelGGL((rollout_resident_kernel<BaseT, no_prior_t>), grid, block, 0, s, a); break;
        case 1: hipLaunchKernelGGL((rollout_resident_kernel<BaseT, float>), grid, block, 0, s, a); break;
        case 2: hipLaunchKernelGGL((rollout_resident_kernel<BaseT, bf16_t>), grid, block, 0, s, a); break;
        default: hipLaunchKernelGGL((rollout_resident_kernel<BaseT, f16_t>), grid, block, 0, s, a); break;
    }
    return hipGetLastError();
}

int g_resident_spin_limit = 1 << 16;   // re-reads before a wait gives up (each ~1-2 us)
int g_resident_enabled = 1;

}  // namespace

int resident_spin_limit() { return g_resident_spin_limit; }
int set_resident_spin_limit(int limit) {
    const int prev = g_resident_spin_limit;
    g_resident_spin_limit = std::max(0, limit);
    return prev;
}
int set_rollout_resident(int enable) {
    const int prev = g_resident_enabled;
    g_resident_enabled = enable != 0;
    return prev;
}
bool rollout_resident_enabled() { return g_resident_enabled != 0; }

bool rollout_resident_eligible(int64_t batch, int64_t G, int64_t r, int64_t V, int64_t steps, bool packed) {
    const int nwg = device_cu_count();
    if (!packed || batch < 1 || batch > 16 || r != kResidentRank || steps < 1 || steps > kResidentMaxSteps) return false;
    if (G < 64 || G > kResidentMaxG || (G & (G - 1)) != 0 || G % nwg != 0) return false;
    // slot rows of whole 64-word chunks, at most the slots the workspace holds
    if (nwg < 64 || nwg > kResidentMaxWGs || nwg % 64 != 0 || V >= (int64_t)1 << 30) return false;
    const int upw = (int)(G / nwg);
    if (upw % 2 != 0 || 3 * upw > 16) return false;
    const int64_t ntiles = (V + 15) / 16;
    const int64_t first = std::min<int64_t>(ntiles, (int64_t)kRrRankWGs * kRrWaves * kRrRegTiles);
    const int64_t rest = ntiles - first;
    const int64_t per = (rest + (nwg - kRrRankWGs) - 1) / (nwg - kRrRankWGs);
    return per <= kRrWaves * kRrRegTiles + kResidentLdsTiles;
}

hipError_t launch_rollout_resident(const ResidentRolloutArgs& r, void* ws, hipStream_t s) {
    char* w = static_cast<char*>(ws);
    RrArgs a{};
    a.w_hh = r.w_hh; a.b_hh = r.b_hh;
    a.A = r.A; a.rank_b = r.rank_b; a.act = r.act;
    a.B = r.B;
    a.gi_table = r.gi_table; a.ld_gi = r.ld_gi; a.table_rows = r.table_rows;
    a.prefix = r.prefix; a.ld_prefix = r.ld_prefix;
    a.base = r.base; a.ld_base = r.ld_base;
    a.prior = r.prior;
    a.alpha = r.alpha; a.beta = r.beta;
    a.M = (int)r.batch; a.G = (int)r.G; a.V = (int)r.V; a.steps = (int)r.steps;
    a.ntiles = (int)((r.V + 15) / 16);
    const int nwg = device_cu_count();
    a.upw = (int)(r.G / nwg);
    a.mp_shift = 0;
    while ((1 << a.mp_shift) < a.M) ++a.mp_shift;
    a.np_shift = 0;
    while ((2 << a.np_shift) < a.upw) ++a.np_shift;   // upw / 2 = 1 << np_shift (upw a power of two)
    a.out_ids = r.out_ids; a.out_scores = r.out_scores; a.ld_out = r.ld_out;
    a.counters = reinterpret_cast<unsigned int*>(w + kCountersOff);
    a.h_words = reinterpret_cast<unsigned long long*>(w + kResidentOff);
    a.rank_words = reinterpret_cast<unsigned long long*>(w + kResidentOff + kResidentHWordBytes);
    a.slots = reinterpret_cast<unsigned long long*>(w + kResidentOff + kResidentHWordBytes + kResidentRankWordBytes);
    a.spin_limit = resident_spin_limit();
    const int pk = r.prior == nullptr ? 0 : (r.prior_dtype == 1 ? 2 : (r.prior_dtype == 2 ? 3 : 1));
    if (r.base_dtype == 1) return launch_rr_base<bf16_t>(a, pk, nwg, s);
    if (r.base_dtype == 2) return launch_rr_base<f16_t>(a, pk, nwg, s);
    return launch_rr_base<float>(a, pk, nwg, s);
}

}  // namespace dels

// One draft step for few rows (M <= 16) in a single launch: the rank
// projection rank = bf16(act(bf16(h . A^T + bias))) (code/kernel/dels.py:437-443)
// followed by the fused combine + vocabulary argmax (code/kernel/dels.py:15-138).
//
// Two kernels back to back leave the rank projection's latency chain on the
// critical path while HBM idles.  Here the grid is 256 workgroups (one per CU,
// all resident) and the rank is handed over inside the launch:
//   1. workgroup g computes the fp32 partial of rank column tile c = g % nct
//      (16 columns, nct = r/16) over K slice z = g / nct; for z > 0 it
//      publishes the partial as 64-bit words {tag, fp32} with device-coherent
//      stores.  The z = 0 workgroup of each tile (its "combiner") collects the
//      other slices' words (re-reading those whose tag is not this launch's),
//      sums the partials in slice order, applies bias, bf16 rounding and the
//      activation, and publishes the tile as words {tag, two bf16};
//   2. every workgroup then puts the first two tiles of its argmax stream in
//      flight, reads the whole rank (re-reading untagged words, bounded) and
//      runs the GEMV-argmax stream of fused_argmax_gemv.h on the prefetched
//      tiles onwards.
// The order inside a workgroup follows from how a CU serves its loads: in
// issue order, so anything issued behind the CU's own prefetch waits for it
// (the prefetch of the whole grid takes about 5 us to drain).  The operand
// loads and the partial's store therefore go first; a combiner, whose polls
// are on the critical path, issues its prefetch only after it has published
// its tile; everybody else's rank read waits behind its own prefetch, which it
// would do anyway, since those tiles are consumed first.  Data and readiness
// travel in the same word, so there are no counters, flags or atomics besides
// the argmax keys.
//
// The tag is a function of a launch generation word in the control area that
// the last workgroup advances at the end of each launch, and it is never zero.
// The words live in a workspace region that only the decode kernels write
// (every other entry point's data starts past it), so a word holds zero (a
// fresh workspace) or the tag of an earlier launch: neither passes for the
// current one.  Tags repeat only after 2^32 - 1 launches on one workspace, so
// a word would have to go unwritten by every launch of its shape for that long
// to be mistaken.  If the re-reads run out (the grid is not
// co-resident, e.g. other work shares the device), the workgroup computes the
// whole rank itself with the same partials in the same order, so the result
// is the same bit for bit and the kernel always terminates.
//
// The fp8 variant (lowrank_decode8_kernel) runs the same phases with the rank
// projection weight A as e4m3 (K32 blocks, widened to bf16 in registers, its
// per-column scale applied before the bias) and the argmax of fused_argmax_fp8.h
// (the rank quantised per row to e4m3, B as e4m3 K128 blocks).
#pragma once

#include "fused_argmax_fp8.h"
#include "fused_argmax_gemv.h"

namespace dels {


struct DecodeKArgs {
    ArgmaxKArgs am;                      // argmax part; am.rank is unused
    const uint16_t* h; int64_t ldh;      // [M, d] bf16
    const void* A;                       // [r, d] in blocks of 16 rows x 32 K: bf16 (1 KiB) or e4m3 (512 B)
    const float* a_scale;                // e4m3 A only: per-rank-column scale [r]
    const uint16_t* bias; int act;
    int ksa;                             // d / 32
    int nct, nz, kpz;                    // rank column tiles (r/16), K slices (256/nct), K blocks per slice
    unsigned long long* partial_words;   // [nct][nz][256]: tag << 32 | fp32 partial (slices z > 0)
    unsigned long long* rank_words;      // [16][r/2]: tag << 32 | bf16 pair
    unsigned int* gen;                   // launch generation (control area; advanced once per launch)
    int spin_limit;                      // re-reads of untagged words before computing the rank locally
    // rollout step with the GRU fused in (GRU instantiations only; h above unused)
    const uint16_t* gi_table; int64_t ld_gi, table_rows;   // [rows, 3G] bf16: E . W_ih^T + b_ih
    const int64_t* tokens; int64_t tok_stride;             // the previous step's ids
    const uint16_t* w_hh;                // [3G, G] in MFMA-16 blocks
    const uint16_t* b_hh;                // [3G] or NULL
    const uint16_t* h_prev;              // [M, G] bf16, row stride G; NULL: a zero state
    uint16_t* h_out;                     // [M, G] bf16, row stride G: the new state
    unsigned long long* h_words;         // [16][G/2]: tag << 32 | two bf16 of the new state
};

// Tag of the words of the launch that read generation g: an odd multiple of
// g + 1 (a bijection on 32-bit words), with the one g that would give 0
// (g = 2^32 - 1) mapped like g = 0 -- so never the zero of a fresh workspace,
// and distinct for 2^32 - 1 launches in a row.
__device__ __forceinline__ uint32_t decode_tag(uint32_t g) {
    return (g + 1u + (g == 0xffffffffu ? 1u : 0u)) * 0x9E3779B1u;
}

// fp32 dot of rank column tile c over K blocks [kb0, kb1) for the 16 rows,
// this wave taking every 4th block from kb0 + wave (all loads issued first).
// A8: A holds e4m3 bytes, widened to bf16 at use.
template <bool A8, int J>
__device__ __forceinline__ f32x4 decode_rank_partial(const DecodeKArgs& d, const uint16_t* hsrc, int64_t ldh, int M,
                                                     int c, int kb0, int kb1, int wave, int lane) {
    const int col = lane & 15, kg = lane >> 4;
    const bool mok = col < M;
    const uint16_t* hp = hsrc + (int64_t)(mok ? col : 0) * ldh + kg * 8;
    u32x4 xv[J], wv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int kb = kb0 + wave + 4 * j;
        const int kc = kb < kb1 ? kb : min(kb0, d.ksa - 1);   // a valid block when masked
        xv[j] = *reinterpret_cast<const u32x4*>(hp + kc * 32);
        if constexpr (A8) {
            const uint8_t* ap = static_cast<const uint8_t*>(d.A) + ((int64_t)c * d.ksa + kc) * kFp8K32Block + lane * 8;
            const u32x2 q = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(ap));
            wv[j] = u32x4{q[0], q[1], 0u, 0u};
        } else {
            const uint16_t* ap = static_cast<const uint16_t*>(d.A) + (int64_t)c * d.ksa * 512 + lane * 8;
            wv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ap + (int64_t)kc * 512));
        }
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const bool ok = kb0 + wave + 4 * j < kb1;
        u32x4 w = wv[j];
        if constexpr (A8) w = widen_e4m3x8(w[0], w[1]);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(masked_bf16x8(xv[j], (ok && mok) ? ~0u : 0u),
                                                      masked_bf16x8(w, ok ? ~0u : 0u), acc, 0, 0, 0);
    }
    return acc;
}

// Sum the four waves' 16x16 accumulators into red[lane * 4 + q] in a fixed order
// ((w0 + w2) + (w1 + w3)); `red` holds 512 floats.  Ends with a barrier.
__device__ __forceinline__ void decode_wave_sum(float* red, f32x4 acc, int wave, int lane) {
    if (wave >= 2) *reinterpret_cast<f32x4*>(&red[(wave - 2) * 256 + lane * 4]) = acc;
    __syncthreads();
    if (wave < 2) acc += *reinterpret_cast<const f32x4*>(&red[wave * 256 + lane * 4]);
    __syncthreads();
    if (wave == 1) *reinterpret_cast<f32x4*>(&red[lane * 4]) = acc;
    __syncthreads();
    if (wave == 0) {
        f32x4* p = reinterpret_cast<f32x4*>(&red[lane * 4]);
        *p = acc + *p;
    }
    __syncthreads();
}

// rank = bf16(act(bf16(v * a_scale + bias))) for column n (no scale for bf16 A).
__device__ __forceinline__ uint16_t decode_rank_epilogue(const DecodeKArgs& d, float v, int n) {
#pragma clang fp contract(off)
    if (d.a_scale) v = v * d.a_scale[n];
    if (d.bias) v = v + bf16_bits_to_f32(d.bias[n]);
    v = round_bf16(v);
    if (d.act == 1) v = round_bf16(silu_f32(v));
    return f32_to_bf16_bits(v);
}

// Value of (row m, column n of the tile) in a wave-summed accumulator tile.
__device__ __forceinline__ float decode_tile_at(const float* red, int m, int n) {
    return red[(((m >> 2) * 16 + n) << 2) + (m & 3)];
}

// Partial of rank column tile c over K slice z (K blocks [z*kpz, (z+1)*kpz)),
// wave-summed into `red`.  Rounds of 4*J blocks, J the smallest of 2/4/8/16
// that covers the slice in one round where it can (no loads of masked blocks).
template <bool A8, int J>
__device__ __forceinline__ f32x4 decode_slice_acc(const DecodeKArgs& d, const uint16_t* hsrc, int64_t ldh, int M,
                                                  int c, int k0, int k1, int wave, int lane) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int kb0 = k0; kb0 < k1; kb0 += 4 * J)
        acc += decode_rank_partial<A8, J>(d, hsrc, ldh, M, c, kb0, min(k1, kb0 + 4 * J), wave, lane);
    return acc;
}
// hsrc/ldh: the rows of h (global memory, or the fused GRU's new state in LDS).
template <bool A8>
__device__ __forceinline__ void decode_slice_partial(const DecodeKArgs& d, const uint16_t* hsrc, int64_t ldh, int M,
                                                     int c, int z, float* red, int wave, int lane) {
    const int k0 = z * d.kpz, k1 = min(d.ksa, k0 + d.kpz);
    f32x4 acc;
    if (d.kpz <= 8) acc = decode_slice_acc<A8, 2>(d, hsrc, ldh, M, c, k0, k1, wave, lane);
    else if (d.kpz <= 16) acc = decode_slice_acc<A8, 4>(d, hsrc, ldh, M, c, k0, k1, wave, lane);
    else if (d.kpz <= 32) acc = decode_slice_acc<A8, 8>(d, hsrc, ldh, M, c, k0, k1, wave, lane);
    else acc = decode_slice_acc<A8, 16>(d, hsrc, ldh, M, c, k0, k1, wave, lane);
    decode_wave_sum(red, acc, wave, lane);
}

// ---- the fused GRU (rollout steps) ---------------------------------------------
// In GRU mode a launch first advances the local head,
//     h = GRU(gi_table[tokens], h_prev)    (code/kernel/dels.py:359-373, 202-211),
// and then runs the draft step on h.  Workgroups nr .. nr + G/16 - 1 (nr =
// nct * nz: the first workgroups without rank work) each compute 16 units of h
// -- gh = h_prev . W_hh^T (+ b_hh) for the units' three gate rows, 96 KiB of
// W_hh at G = 1024 -- write them to h_out for the next step and publish them as
// words {tag, two bf16} in h_words.  A rank workgroup reads the units of its K
// slice from those words into LDS; a workgroup whose words do not arrive
// computes the units it needs itself, with the same partial sums in the same
// order, so the result does not depend on who computed it.
constexpr int kGruUnits = 16;      // units of h per GRU workgroup
constexpr int kGruMaxG = 2048;     // largest hidden size of the fused GRU: LDS holds [16][G] bf16 of h

// Units u0 .. u0+15 of the new state for rows m < M (zero for rows past M)
// into hblk[16][16] (bf16 bits, row-major).  gh sums each wave's K blocks
// (wave, wave + 4, ...) in fp32, then the four waves in a fixed order, and is
// rounded to bf16 after the bias, as F.linear in bf16.  gred: 3 x 4 x 256
// floats of LDS.  All threads; ends with a barrier.
__device__ __forceinline__ void gru_block(const DecodeKArgs& d, int M, int G, int u0, float* gred, uint16_t* hblk) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, kg = lane >> 4;
    const int KB = G / 32;
    const int KBl = d.h_prev ? KB : 0;   // a zero previous state (a first step): gh = b_hh
    const bool mok = col < M;
    const uint16_t* hp = d.h_prev ? d.h_prev + (int64_t)(mok ? col : 0) * G + kg * 8 : nullptr;
    const uint16_t* wp[3];
#pragma unroll
    for (int g = 0; g < 3; ++g) wp[g] = d.w_hh + (int64_t)((g * G + u0) / 16) * KB * 512 + lane * 8;
    f32x4 acc[3];
#pragma unroll
    for (int g = 0; g < 3; ++g) acc[g] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int kb0 = wave; kb0 < KBl; kb0 += 4 * 8) {
        u32x4 xv[8], wv[3][8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int kb = kb0 + 4 * j;
            const int kc = kb < KB ? kb : wave;   // a valid block when masked
            xv[j] = *reinterpret_cast<const u32x4*>(hp + kc * 32);
            // plain (cached) loads: every step of a rollout reads the same
            // W_hh (6 MB at G = 1024), unlike the streamed B (14-step rollout
            // 358 -> 347 us against non-temporal loads)
#pragma unroll
            for (int g = 0; g < 3; ++g) wv[g][j] = *reinterpret_cast<const u32x4*>(wp[g] + (int64_t)kc * 512);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const bool ok = kb0 + 4 * j < KB;
#pragma unroll
            for (int g = 0; g < 3; ++g)
                acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(masked_bf16x8(xv[j], (ok && mok) ? ~0u : 0u),
                                                                 masked_bf16x8(wv[g][j], ok ? ~0u : 0u), acc[g], 0,
                                                                 0, 0);
        }
    }
#pragma unroll
    for (int g = 0; g < 3; ++g) *reinterpret_cast<f32x4*>(&gred[(g * 4 + wave) * 256 + lane * 4]) = acc[g];
    __syncthreads();
    // thread t: row m = t / 16, unit n = t % 16 (element m % 4 of lane (m / 4) * 16 + n)
    const int m = threadIdx.x >> 4, n = threadIdx.x & 15;
    const int e = (((m >> 2) * 16 + n) << 2) + (m & 3);
    uint16_t out = 0;
    if (m < M) {
        const int j = u0 + n;
        float gh[3];
#pragma unroll
        for (int g = 0; g < 3; ++g) {
            gh[g] = (gred[(g * 4 + 0) * 256 + e] + gred[(g * 4 + 1) * 256 + e]) +
                    (gred[(g * 4 + 2) * 256 + e] + gred[(g * 4 + 3) * 256 + e]);
            if (d.b_hh) gh[g] = gh[g] + bf16_bits_to_f32(d.b_hh[g * G + j]);
            gh[g] = round_bf16(gh[g]);
        }
        int64_t tok = d.tokens[(int64_t)m * d.tok_stride];
        tok = tok < 0 ? 0 : (tok >= d.table_rows ? d.table_rows - 1 : tok);
        const uint16_t* gi = d.gi_table + tok * d.ld_gi;
        const float hv = d.h_prev ? bf16_bits_to_f32(d.h_prev[(int64_t)m * G + j]) : 0.f;
        out = f32_to_bf16_bits(gru_unit(bf16_bits_to_f32(gi[j]), bf16_bits_to_f32(gi[G + j]),
                                        bf16_bits_to_f32(gi[2 * G + j]), gh[0], gh[1], gh[2], hv));
    }
    hblk[m * 16 + n] = out;
    __syncthreads();
}

// A GRU workgroup's share: its 16 units to h_out and to the tagged words.
__device__ __forceinline__ void gru_publish(const DecodeKArgs& d, int M, int G, uint32_t tag, float* gred,
                                            uint16_t* hblk) {
    const int u0 = ((int)blockIdx.x - d.nct * d.nz) * kGruUnits;
    gru_block(d, M, G, u0, gred, hblk);
    if (threadIdx.x < 128) {
        const int m = threadIdx.x >> 3, p = threadIdx.x & 7;
        if (m < M) {
            const uint32_t pair = (uint32_t)hblk[m * 16 + 2 * p] | ((uint32_t)hblk[m * 16 + 2 * p + 1] << 16);
            *reinterpret_cast<uint32_t*>(d.h_out + (int64_t)m * G + u0 + 2 * p) = pair;
            __hip_atomic_store(d.h_words + (int64_t)m * (G / 2) + u0 / 2 + p, ((unsigned long long)tag << 32) | pair,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Units [ub, ue) (multiples of 16) of the new state into s_h[16][G] (rows past
// M are not written): from the tagged words, re-read (bounded) until each
// carries `tag`; if some never do, every block of the range is computed here.
// All threads; ends with a barrier.
template <int NW>
__device__ __forceinline__ void gru_fill(const DecodeKArgs& d, int M, int G, int ub, int ue, uint32_t tag,
                                      uint16_t* s_h, float* gred, uint16_t* hblk) {
    static_assert(NW <= 32, "one bit per word in a 32-bit mask");
    const int np = (ue - ub) / 2, nw = M * np;
    bool ok = d.spin_limit > 0;
    for (int w0 = threadIdx.x; ok && w0 < nw; w0 += 256 * NW) {
        unsigned long long w[NW];
        uint32_t missing = 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const int idx = w0 + 256 * i;
            if (idx < nw) {
                const int m = idx / np, p = idx - m * np;
                w[i] = __hip_atomic_load(d.h_words + (int64_t)m * (G / 2) + ub / 2 + p, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
                missing |= (uint32_t)((uint32_t)(w[i] >> 32) != tag) << i;
            }
        }
        // re-read the whole group: every load in flight at once
        for (int it = 0; missing != 0 && it < d.spin_limit; ++it) {
            __builtin_amdgcn_s_sleep(2);
            missing = 0;
#pragma unroll
            for (int i = 0; i < NW; ++i) {
                const int idx = w0 + 256 * i;
                if (idx < nw) {
                    const int m = idx / np, p = idx - m * np;
                    w[i] = __hip_atomic_load(d.h_words + (int64_t)m * (G / 2) + ub / 2 + p, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
                }
            }
#pragma unroll
            for (int i = 0; i < NW; ++i)
                if (w0 + 256 * i < nw) missing |= (uint32_t)((uint32_t)(w[i] >> 32) != tag) << i;
        }
        ok = missing == 0;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            const int idx = w0 + 256 * i;
            if (ok && idx < nw) {
                const int m = idx / np, p = idx - m * np;
                *reinterpret_cast<uint32_t*>(s_h + m * G + ub + 2 * p) = (uint32_t)w[i];
            }
        }
    }
    if (!__syncthreads_or(!ok)) return;
    for (int u0 = ub; u0 < ue; u0 += kGruUnits) {   // the words did not come: compute the range here
        gru_block(d, M, G, u0, gred, hblk);
        s_h[(threadIdx.x >> 4) * G + u0 + (threadIdx.x & 15)] = hblk[threadIdx.x];
    }
    __syncthreads();
}

// A rank workgroup's partial in GRU mode when its slice is one round of J
// blocks per wave (decode_slice_partial with that J, the same sums): the slice
// of A goes in flight before the wait for the new state's words (NW in flight
// per thread; 4 or 16 measured slower, as were longer sleeps between
// re-reads).  Ends with a barrier.
template <int J, int NW>
__device__ __forceinline__ void gru_rank_partial(const DecodeKArgs& d, int M, int c, int k0, int k1, uint32_t tag,
                                                 uint16_t* s_h, float* gred, uint16_t* hblk, float* red, int wave,
                                                 int lane) {
    const int G = d.ksa * 32;
    u32x4 wv[J];
    const uint16_t* ap = static_cast<const uint16_t*>(d.A) + (int64_t)c * d.ksa * 512 + lane * 8;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int kb = k0 + wave + 4 * j;
        const int kc = kb < k1 ? kb : min(k0, d.ksa - 1);
        wv[j] = *reinterpret_cast<const u32x4*>(ap + (int64_t)kc * 512);   // cached: every step reads this A
    }
    gru_fill<NW>(d, M, G, k0 * 32, k1 * 32, tag, s_h, gred, hblk);
    const int col = lane & 15, kg = lane >> 4;
    const bool mok = col < M;
    const uint16_t* hp = s_h + (mok ? col : 0) * G + kg * 8;
    f32x4 part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int kb = k0 + wave + 4 * j;
        const bool ok = kb < k1;
        const int kc = ok ? kb : min(k0, d.ksa - 1);
        const u32x4 xv = *reinterpret_cast<const u32x4*>(hp + kc * 32);
        part = __builtin_amdgcn_mfma_f32_16x16x32_bf16(masked_bf16x8(xv, (ok && mok) ? ~0u : 0u),
                                                       masked_bf16x8(wv[j], ok ? ~0u : 0u), part, 0, 0, 0);
    }
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    acc += part;
    decode_wave_sum(red, acc, wave, lane);
}

// Phase 1 (see the top of the file).  Ends with a barrier; `red` is free after it.
// GRU mode: h is the fused GRU's new state, read into s_h (LDS) for this K slice.
template <bool A8, bool GRU = false>
__device__ __forceinline__ void decode_rank_phase(const DecodeKArgs& d, int M, int r, float* red, uint32_t tag,
                                                  uint16_t* s_h = nullptr, float* gred = nullptr,
                                                  uint16_t* hblk = nullptr) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    if ((int)blockIdx.x >= d.nct * d.nz) return;   // no rank work: straight to the argmax stream
    const int c = (int)blockIdx.x % d.nct;
    const int z = (int)blockIdx.x / d.nct;
    if constexpr (GRU) {
        const int G = d.ksa * 32;
        const int k0 = z * d.kpz, k1 = min(d.ksa, k0 + d.kpz);
        if (!A8 && d.kpz > 8 && d.kpz <= 16) {   // every fused-GRU plan up to G = 2048
            gru_rank_partial<4, 8>(d, M, c, k0, k1, tag, s_h, gred, hblk, red, wave, lane);
        } else {
            gru_fill<8>(d, M, G, k0 * 32, k1 * 32, tag, s_h, gred, hblk);
            decode_slice_partial<A8>(d, s_h, G, M, c, z, red, wave, lane);
        }
    } else {
        decode_slice_partial<A8>(d, d.h, d.ldh, M, c, z, red, wave, lane);
    }
    unsigned long long* pw = d.partial_words + (int64_t)c * d.nz * 256 + threadIdx.x;
    if (z > 0) {
        __hip_atomic_store(pw + z * 256, ((unsigned long long)tag << 32) | __float_as_uint(red[threadIdx.x]),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __syncthreads();
        return;
    }
    // the combiner: slices 1 .. nz-1 in order, eight words in flight per thread
    float v = red[threadIdx.x];
    bool ok = d.spin_limit > 0;
    for (int z0 = 1; ok && z0 < d.nz; z0 += 8) {
        unsigned long long w[8];
        uint32_t missing = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (z0 + i < d.nz) {
                w[i] = __hip_atomic_load(pw + (z0 + i) * 256, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                missing |= (uint32_t)((uint32_t)(w[i] >> 32) != tag) << i;
            }
        }
        // re-read the whole group: every load in flight at once (a test right
        // after each load would wait for it before the next is issued)
        for (int it = 0; missing != 0 && it < d.spin_limit; ++it) {
            __builtin_amdgcn_s_sleep(2);
            missing = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (z0 + i < d.nz) w[i] = __hip_atomic_load(pw + (z0 + i) * 256, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < 8; ++i)
                if (z0 + i < d.nz) missing |= (uint32_t)((uint32_t)(w[i] >> 32) != tag) << i;
        }
        ok = missing == 0;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (ok && z0 + i < d.nz) v = v + __uint_as_float((uint32_t)w[i]);
    }
    if (__syncthreads_or(!ok)) return;   // the consumers will time out and compute the rank themselves
    red[threadIdx.x] = v;
    __syncthreads();
    if (threadIdx.x < 128) {
        const int m = threadIdx.x >> 3, n = (threadIdx.x & 7) * 2;
        const uint32_t lo = decode_rank_epilogue(d, decode_tile_at(red, m, n), c * 16 + n);
        const uint32_t hi = decode_rank_epilogue(d, decode_tile_at(red, m, n + 1), c * 16 + n + 1);
        __hip_atomic_store(d.rank_words + (int64_t)m * (r / 2) + c * 8 + (threadIdx.x & 7),
                           ((unsigned long long)tag << 32) | (lo | (hi << 16)), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
}

// Phase 2: bring the rank ([16][R] bf16) into LDS.  Each thread reads its R/32
// words with device-coherent loads and re-reads (at most spin_limit times) the
// ones whose tag is not `tag`; if any word is still missing the workgroup
// computes the whole rank itself (the same partials summed in the same order
// as phase 1).  Ends with a barrier.
template <int R, bool A8, bool GRU = false>
__device__ __forceinline__ void decode_rank_into_lds(const DecodeKArgs& d, int M, float* red, uint32_t tag,
                                                     uint16_t* s_rank, uint16_t* s_h = nullptr,
                                                     float* gred = nullptr, uint16_t* hblk = nullptr) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    constexpr int kPer = R / 32;   // words per thread
    static_assert(kPer <= 32, "one bit per word in a 32-bit mask");
    unsigned long long w[kPer];
    uint32_t missing = (1u << (kPer - 1) << 1) - 1u;
    if (d.spin_limit > 0) {
        // Wait until one word of every tile carries the tag -- eight bytes per
        // lane, so waiting adds little traffic -- then read all the words.
        {
            const unsigned long long* pr = d.rank_words + (lane % d.nct) * 8;
            for (int it = 0; it < d.spin_limit; ++it) {
                const unsigned long long pw = __hip_atomic_load(pr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (__builtin_amdgcn_ballot_w64((uint32_t)(pw >> 32) != tag) == 0) break;
                __builtin_amdgcn_s_sleep(2);
            }
        }
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            w[i] = __hip_atomic_load(d.rank_words + threadIdx.x + 256 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        missing = 0;
#pragma unroll
        for (int i = 0; i < kPer; ++i) missing |= (uint32_t)((uint32_t)(w[i] >> 32) != tag) << i;
        for (int it = 0; missing != 0 && it < d.spin_limit; ++it) {   // all words in flight at once
            __builtin_amdgcn_s_sleep(2);
            missing = 0;
#pragma unroll
            for (int i = 0; i < kPer; ++i)
                w[i] = __hip_atomic_load(d.rank_words + threadIdx.x + 256 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
            for (int i = 0; i < kPer; ++i) missing |= (uint32_t)((uint32_t)(w[i] >> 32) != tag) << i;
        }
    }
    if (!__syncthreads_or(missing != 0)) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(s_rank);
#pragma unroll
        for (int i = 0; i < kPer; ++i) dst[threadIdx.x + 256 * i] = (uint32_t)w[i];
    } else {
#pragma clang fp contract(off)
        const uint16_t* hsrc = d.h;
        int64_t ldh = d.ldh;
        if constexpr (GRU) {   // the whole new state, from the words or computed here
            gru_fill<8>(d, M, d.ksa * 32, 0, d.ksa * 32, tag, s_h, gred, hblk);
            hsrc = s_h;
            ldh = d.ksa * 32;
        }
        for (int cc = 0; cc < d.nct; ++cc) {
            float v = 0.f;
            for (int z = 0; z < d.nz; ++z) {
                decode_slice_partial<A8>(d, hsrc, ldh, M, cc, z, red, wave, lane);
                v = z == 0 ? red[threadIdx.x] : v + red[threadIdx.x];
                __syncthreads();   // red is rewritten by the next partial
            }
            red[threadIdx.x] = v;
            __syncthreads();
            {
                const int m = threadIdx.x >> 4, n = threadIdx.x & 15;
                s_rank[m * R + cc * 16 + n] = decode_rank_epilogue(d, decode_tile_at(red, m, n), cc * 16 + n);
            }
            __syncthreads();   // red is rewritten by the next tile
        }
    }
    __syncthreads();
}

// Slot of this workgroup in the wave-strided tile walk.  The first slots get
// one tile more when the tiles do not divide evenly; they go to the
// workgroups without rank work, which start streaming first.
__device__ __forceinline__ int decode_first_tile(const DecodeKArgs& d) {
    return ((int)blockIdx.x + (int)gridDim.x - d.nct * d.nz) % (int)gridDim.x;
}

// Per-lane argmax state of rows 4*(lane/16) + q (M <= 16: one row group).
template <typename BaseT, typename PriorT>
__device__ __forceinline__ void decode_rows(const ArgmaxKArgs& a, int kg, float (&al)[4], float (&be)[4],
                                            bool (&use_prior)[4], const BaseT* (&brow)[4], float (&best)[4],
                                            int (&bidx)[4]) {
    const BaseT* base = static_cast<const BaseT*>(a.base);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int m = 4 * kg + q;
        const bool mok = m < a.M;
        al[q] = mok ? a.alpha[(int64_t)m * a.alpha_stride] : 0.f;
        be[q] = mok ? a.beta[(int64_t)m * a.beta_stride] : 0.f;
        use_prior[q] = !is_no_prior<PriorT>::value && (be[q] != 0.f);
        brow[q] = base + (int64_t)(mok ? m : 0) * a.ldbase;
        best[q] = -__builtin_inff();
        bidx[q] = INT_MAX;
    }
}

// GRU: a rollout step with the local head's GRU fused in (see gru_block).
template <int KSTEPS, typename BaseT, typename PriorT, bool GRU>
__global__ __launch_bounds__(256) void lowrank_decode_kernel(DecodeKArgs d) {
#pragma clang fp contract(off)
    const ArgmaxKArgs& a = d.am;
    constexpr int r = KSTEPS * 32;
    __shared__ float red[512];
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;
    __shared__ __attribute__((aligned(16))) uint16_t s_rank[16 * r];   // the rank, [16][r] bf16
    struct GruLds {
        uint16_t h[16 * kGruMaxG];   // the new state [16][G]
        float gred[3 * 4 * 256];
        uint16_t hblk[16 * 16];
    };
    struct NoGruLds {
        uint16_t h[1];
        float gred[1];
        uint16_t hblk[1];
    };
    __shared__ __attribute__((aligned(16))) std::conditional_t<GRU, GruLds, NoGruLds> gl;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    const int col = lane & 15;
    const int kg = lane >> 4;

    const uint32_t tag = decode_tag(__hip_atomic_load(d.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    if constexpr (GRU) {
        const int nr = d.nct * d.nz;
        if ((int)blockIdx.x >= nr && (int)blockIdx.x < nr + d.ksa * 32 / kGruUnits) {
            gru_publish(d, a.M, d.ksa * 32, tag, gl.gred, gl.hblk);
        } else if ((int)blockIdx.x >= nr) {
            // The other workgroups start their B prefetch 3 us late (the 100 MHz
            // real-time clock), so that the GRU's W_hh and the rank's A loads
            // reach HBM ahead of it: the rank is on every workgroup's critical
            // path, and the prefetch still lands before it (14-step rollout at
            // G = 1024: 366 -> 360 us, flat from 2 to 6 us; a decode step
            // without the GRU is slower with any delay).
            const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
            while (__builtin_amdgcn_s_memrealtime() - t0 < 300ull) __builtin_amdgcn_s_sleep(8);
        }
    }
    decode_rank_phase<false, GRU>(d, a.M, r, red, tag, gl.h, gl.gred, gl.hblk);

    const int nwaves = gridDim.x * 4;
    int t = decode_first_tile(d) * 4 + wave;
    float al[4], be[4], best[4];
    int bidx[4];
    bool use_prior[4];
    const BaseT* brow[4];
    const PriorT* prior = static_cast<const PriorT*>(a.prior);
    decode_rows<BaseT, PriorT>(a, kg, al, be, use_prior, brow, best, bidx);
    // The first two tiles of the argmax stream go in flight while the rank is finished.
    const int ntiles = (a.V + 15) >> 4;
    // Tiles of this wave: t + k * nwaves, k < cnt, through a ring of ND tile
    // register sets.  The first ND go in flight before the rank is read, so
    // HBM stays busy while the rank is finished: with four sets (64 MB over
    // the grid at r = 512) the step takes 31.5 us, with two 33.4 us; at
    // r = 256 four sets beat two (a 14-step rollout 406 -> 389 us) and six
    // lose (439 us).  The
    // loop runs only while the refills exist, so its loads are unconditional
    // and every path into the loop top carries the same outstanding loads:
    // the compiler's wait before each contraction covers only the oldest set
    // (with a conditional refill inside the loop it waited for all of them).
    constexpr int ND = KSTEPS >= 8 ? 4 : 2;
    const int cnt = t < ntiles ? (ntiles - 1 - t) / nwaves + 1 : 0;
    TileRegs<KSTEPS> tr[ND];
#pragma unroll
    for (int u = 0; u < ND; ++u)
        if (u < cnt) load_tile<KSTEPS, B_PACKED_EXACT>(a, t + u * nwaves, lane, brow, prior, tr[u]);

    decode_rank_into_lds<r, false, GRU>(d, a.M, red, tag, s_rank, gl.h, gl.gred, gl.hblk);
    bf16x8 ra[KSTEPS];
    {
        const bool mok = col < a.M;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s)
            ra[s] = masked_bf16x8(*reinterpret_cast<const u32x4*>(&s_rank[col * r + s * 32 + kg * 8]),
                                  mok ? ~0u : 0u);
    }

    // ---- 4. the argmax stream (as fused_argmax_gemv_kernel) -------------------
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
    int k = 0;
    for (; k + 2 * ND <= cnt; k += ND) {
#pragma unroll
        for (int u = 0; u < ND; ++u) {
            consume(tr[u], t + (k + u) * nwaves);
            load_tile<KSTEPS, B_PACKED_EXACT>(a, t + (k + u + ND) * nwaves, lane, brow, prior, tr[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < ND; ++u) {
        if (k + u < cnt) consume(tr[u], t + (k + u) * nwaves);
        if (k + u + ND < cnt) load_tile<KSTEPS, B_PACKED_EXACT>(a, t + (k + u + ND) * nwaves, lane, brow, prior, tr[u]);
    }
#pragma unroll
    for (int u = 0; u < ND; ++u)
        if (k + u + ND < cnt) consume(tr[u], t + (k + u + ND) * nwaves);

    // ---- cross-workgroup argmax; the last workgroup advances the generation ----
    argmax_wg_finish(a, best, bidx, 0, s_val, s_idx, s_last, nullptr);
    if (s_last == 1 && threadIdx.x == 0) __hip_atomic_fetch_add(d.gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// fp8 variant: A e4m3 (K32 blocks) with per-column scales in the rank
// projection; rank quantised per row to e4m3; B e4m3 (K128 blocks) with
// per-row scales in the argmax.  KS8 = r / 128.

template <int KS8, typename BaseT, typename PriorT>
__global__ __launch_bounds__(256) void lowrank_decode8_kernel(DecodeKArgs d) {
#pragma clang fp contract(off)
    const ArgmaxKArgs& a = d.am;
    constexpr int r = KS8 * 128;
    __shared__ float red[512];
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;
    __shared__ __attribute__((aligned(16))) uint16_t s_rank[16 * r];   // the rank, [16][r] bf16

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    const int col = lane & 15;
    const int kg = lane >> 4;

    const uint32_t tag = decode_tag(__hip_atomic_load(d.gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    decode_rank_phase<true>(d, a.M, r, red, tag);

    const int nwaves = gridDim.x * 4;
    const int t = decode_first_tile(d) * 4 + wave;
    float al[4], be[4], best[4];
    int bidx[4];
    bool use_prior[4];
    const BaseT* brow[4];
    const PriorT* prior = static_cast<const PriorT*>(a.prior);
    decode_rows<BaseT, PriorT>(a, kg, al, be, use_prior, brow, best, bidx);
    const int ntiles = (a.V + 15) >> 4;
    // Tiles of this wave: t + k * nwaves, k < cnt, through a ring of ND8 tile
    // register sets (the structure of the bf16 decode step): all ND8 go in
    // flight before the rank read, and the loop's refills are unconditional,
    // so the compiler's waits cover only the oldest set.  Six sets (48 MB over
    // the grid at r = 512) measured best: 23.1 us against 24.6 with four, 24.8
    // with eight, and 27.4 for a per-wave LDS ring of three tiles (the LDS
    // cannot hold more next to the rank).
    constexpr int ND8 = 6;
    const int cnt = t < ntiles ? (ntiles - 1 - t) / nwaves + 1 : 0;
    TileRegs8<KS8> tr[ND8];
#pragma unroll
    for (int u = 0; u < ND8; ++u)
        if (u < cnt) load_tile8<KS8>(a, t + u * nwaves, lane, brow, prior, tr[u]);
    decode_rank_into_lds<r, true>(d, a.M, red, tag, s_rank);
    __shared__ __attribute__((aligned(16))) uint8_t s_rq[16 * (r + 16)];
    __shared__ float s_rsc[16];
    quantize_rank_coop<r>(s_rank, r, a.M, s_rq, s_rsc);
    i32x8 rq[KS8];
    float rsc[4];
    load_rank_operand<KS8>(s_rq, s_rsc, lane, rq, rsc);
    int k = 0;
    for (; k + 2 * ND8 <= cnt; k += ND8) {
#pragma unroll
        for (int u = 0; u < ND8; ++u) {
            consume_tile8<KS8, BaseT, PriorT>(a, rq, rsc, tr[u], t + (k + u) * nwaves, col, al, be, use_prior, best, bidx);
            load_tile8<KS8>(a, t + (k + u + ND8) * nwaves, lane, brow, prior, tr[u]);
        }
    }
#pragma unroll
    for (int u = 0; u < ND8; ++u) {
        if (k + u < cnt) consume_tile8<KS8, BaseT, PriorT>(a, rq, rsc, tr[u], t + (k + u) * nwaves, col, al, be, use_prior, best, bidx);
        if (k + u + ND8 < cnt) load_tile8<KS8>(a, t + (k + u + ND8) * nwaves, lane, brow, prior, tr[u]);
    }
#pragma unroll
    for (int u = 0; u < ND8; ++u)
        if (k + u + ND8 < cnt)
            consume_tile8<KS8, BaseT, PriorT>(a, rq, rsc, tr[u], t + (k + u + ND8) * nwaves, col, al, be, use_prior, best, bidx);
    argmax_wg_finish(a, best, bidx, 0, s_val, s_idx, s_last, nullptr);
    if (s_last == 1 && threadIdx.x == 0) __hip_atomic_fetch_add(d.gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Dispatch over K steps of B (r / 32) and the prior type for one base dtype.
template <typename BaseT>
hipError_t launch_decode_for_base(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s, bool gru) {
    auto go = [&](auto ks_tag, auto prior_tag) -> hipError_t {
        constexpr int KS = decltype(ks_tag)::value;
        using PT = decltype(prior_tag);
        if (gru)
            hipLaunchKernelGGL((lowrank_decode_kernel<KS, BaseT, PT, true>), dim3(kDecodeWGs), dim3(256), 0, s, ka);
        else
            hipLaunchKernelGGL((lowrank_decode_kernel<KS, BaseT, PT, false>), dim3(kDecodeWGs), dim3(256), 0, s, ka);
        return hipGetLastError();
    };
    auto by_prior = [&](auto ks_tag) -> hipError_t {
        switch (prior_kind) {
            case 0: return go(ks_tag, no_prior_t{});
            case 1: return go(ks_tag, float{});
            case 2: return go(ks_tag, bf16_t{});
            default: return go(ks_tag, f16_t{});
        }
    };
    switch (ksteps) {
        case 2: return by_prior(std::integral_constant<int, 2>{});
        case 4: return by_prior(std::integral_constant<int, 4>{});
        case 8: return by_prior(std::integral_constant<int, 8>{});
        default: return by_prior(std::integral_constant<int, 16>{});
    }
}

// fp8: dispatch over K128 blocks of B (r / 128) and the prior type.
template <typename BaseT>
hipError_t launch_decode8_for_base(const DecodeKArgs& ka, int prior_kind, hipStream_t s) {
    auto go = [&](auto ks_tag, auto prior_tag) -> hipError_t {
        constexpr int KS8 = decltype(ks_tag)::value;
        using PT = decltype(prior_tag);
        hipLaunchKernelGGL((lowrank_decode8_kernel<KS8, BaseT, PT>), dim3(kDecodeWGs), dim3(256), 0, s, ka);
        return hipGetLastError();
    };
    auto by_prior = [&](auto ks_tag) -> hipError_t {
        switch (prior_kind) {
            case 0: return go(ks_tag, no_prior_t{});
            case 1: return go(ks_tag, float{});
            case 2: return go(ks_tag, bf16_t{});
            default: return go(ks_tag, f16_t{});
        }
    };
    switch (ka.am.r / 128) {
        case 1: return by_prior(std::integral_constant<int, 1>{});
        case 2: return by_prior(std::integral_constant<int, 2>{});
        default: return by_prior(std::integral_constant<int, 4>{});
    }
}

hipError_t launch_decode_f32(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s, bool gru);
hipError_t launch_decode_bf16(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s, bool gru);
hipError_t launch_decode_f16(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s, bool gru);
hipError_t launch_decode8_f32(const DecodeKArgs& ka, int prior_kind, hipStream_t s);
hipError_t launch_decode8_bf16(const DecodeKArgs& ka, int prior_kind, hipStream_t s);
hipError_t launch_decode8_f16(const DecodeKArgs& ka, int prior_kind, hipStream_t s);

}  // namespace dels

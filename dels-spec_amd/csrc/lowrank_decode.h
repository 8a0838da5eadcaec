// One draft step for few rows (M <= 16) in a single launch: the rank
// projection rank = bf16(act(bf16(h . A^T + bias))) (code/kernel/dels.py:437-443)
// followed by the fused combine + vocabulary argmax (code/kernel/dels.py:15-138).
//
// Two kernels back to back leave the rank projection's latency chain (operand
// round trip, split-K reduction) on the critical path, ~7 us of a ~37 us step,
// while HBM idles.  Here the grid is 256 workgroups (one per CU, all resident)
// and the rank projection is split over all of them:
//   1. workgroup g computes the fp32 partial of rank column tile c = g % nct
//      (16 columns) over K slice z = g / nct, sums its four waves in LDS and
//      publishes the 16x16 partial with device-coherent stores;
//   2. the workgroup that completes a tile's arrival count (a returning atomic)
//      sums the tile's nz partials in split order -- deterministic --, applies
//      bias, bf16 rounding and the activation, publishes the bf16 tile and bumps
//      a global tile count;
//   3. every workgroup puts the first two tiles of its argmax stream in flight,
//      waits (bounded) for the tile count to reach nct, loads the full rank
//      with device-coherent loads and runs the GEMV-argmax stream of
//      fused_argmax_gemv.h on the prefetched tiles onwards.
// Only returning atomics and agent-scope loads/stores cross workgroups; no
// cache fences.  If the wait times out (the grid is not co-resident, e.g. other
// work shares the device), the workgroup computes the whole rank itself -- slow
// but correct -- so the kernel always terminates.  The last workgroup of the
// argmax reduction returns every counter to zero.
//
// The fp8 variant (lowrank_decode8_kernel) runs the same phases with the rank
// projection weight A as e4m3 (K32 blocks, widened to bf16 in registers, its
// per-column scale applied before the bias) and the argmax of fused_argmax_fp8.h
// (the rank quantised per row to e4m3, B as e4m3 K128 blocks).
#pragma once

#include "fused_argmax_fp8.h"
#include "fused_argmax_gemv.h"

namespace dels {

constexpr int kDecodeWGs = 256;          // grid of the fused decode step
constexpr int kDecodeMaxJ = 8;           // K steps per wave in the split rank projection

struct DecodeKArgs {
    ArgmaxKArgs am;                      // argmax part; am.rank is unused (rank_buf)
    const uint16_t* h; int64_t ldh;      // [M, d] bf16
    const void* A;                       // [r, d] in blocks of 16 rows x 32 K: bf16 (1 KiB) or e4m3 (512 B)
    const float* a_scale;                // e4m3 A only: per-rank-column scale [r]
    const uint16_t* bias; int act;
    int ksa;                             // d / 32
    int nct, nz, kpz;                    // rank column tiles (r/16), K splits, K blocks per split
    float* partial;                      // [nct][nz][256]
    unsigned int* tile_cnt;              // [nct]
    unsigned int* done;                  // published rank tiles
    uint16_t* rank_buf;                  // [16][r] bf16
    int spin_limit;                      // polls of `done` before computing the rank locally
};

// fp32 dot of rank column tile c over K blocks [kb0, kb1) for the 16 rows,
// this wave taking every 4th block from kb0 + wave (all loads issued first).
// A8: A holds e4m3 bytes, widened to bf16 at use.
template <bool A8>
__device__ __forceinline__ f32x4 decode_rank_partial(const DecodeKArgs& d, int M, int c, int kb0, int kb1,
                                                     int wave, int lane) {
    const int col = lane & 15, kg = lane >> 4;
    const bool mok = col < M;
    const uint16_t* hp = d.h + (int64_t)(mok ? col : 0) * d.ldh + kg * 8;
    u32x4 xv[kDecodeMaxJ], wv[kDecodeMaxJ];
#pragma unroll
    for (int j = 0; j < kDecodeMaxJ; ++j) {
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
    for (int j = 0; j < kDecodeMaxJ; ++j) {
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

// Phases 1 and 2: workgroup g computes the partial of rank tile g % nct over
// K slice g / nct and publishes it; the tile's last arrival reduces the tile,
// publishes the bf16 rank tile and counts it in `done`.
template <bool A8>
__device__ __forceinline__ void decode_publish_rank(const DecodeKArgs& d, int M, int r, float* red, int& s_last) {
#pragma clang fp contract(off)
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    const int c = (int)blockIdx.x % d.nct;
    const int z = (int)blockIdx.x / d.nct;
    {
        const int kb0 = z * d.kpz;
        const int kb1 = min(d.ksa, kb0 + d.kpz);
        const f32x4 acc = decode_rank_partial<A8>(d, M, c, kb0, kb1, wave, lane);
        decode_wave_sum(red, acc, wave, lane);
    }
    float* mine = d.partial + ((int64_t)c * d.nz + z) * 256;
    __hip_atomic_store(mine + threadIdx.x, red[threadIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);   // the partial has reached device coherence
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(&d.tile_cnt[c], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == (unsigned)(d.nz - 1);
    }
    __syncthreads();
    if (!s_last) return;
    float p[16];
    const float* tp = d.partial + (int64_t)c * d.nz * 256 + threadIdx.x;
    float v = 0.f;
    for (int z0 = 0; z0 < d.nz; z0 += 16) {
#pragma unroll
        for (int i = 0; i < 16; ++i)
            p[i] = z0 + i < d.nz ? __hip_atomic_load(tp + (int64_t)(z0 + i) * 256, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT)
                                 : 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) v += p[i];
    }
    __syncthreads();
    red[threadIdx.x] = v;
    __syncthreads();
    if (threadIdx.x < 128) {
        const int m = threadIdx.x >> 3, n = (threadIdx.x & 7) * 2;
        const uint32_t lo = decode_rank_epilogue(d, decode_tile_at(red, m, n), c * 16 + n);
        const uint32_t hi = decode_rank_epilogue(d, decode_tile_at(red, m, n + 1), c * 16 + n + 1);
        __hip_atomic_store(reinterpret_cast<uint32_t*>(d.rank_buf + (int64_t)m * r + c * 16 + n), lo | (hi << 16),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);   // the rank tile has reached device coherence
    __syncthreads();
    if (threadIdx.x == 0) {
        __hip_atomic_exchange(&d.tile_cnt[c], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_add(d.done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// Phase 3: wait (bounded) until every rank tile is published, then bring the
// rank ([16][r] bf16) into LDS: read once per workgroup with device-coherent
// loads, a 64-byte share per thread -- or, if the wait timed out, computed
// whole by this workgroup.  Ends with a barrier.
template <int R, bool A8>
__device__ __forceinline__ void decode_rank_into_lds(const DecodeKArgs& d, int M, float* red, int& s_ready,
                                                     uint16_t* s_rank) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    if (threadIdx.x == 0) {
        int it = 0;
        while (__hip_atomic_load(d.done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)d.nct &&
               it < d.spin_limit) {
            __builtin_amdgcn_s_sleep(8);
            ++it;
        }
        s_ready = it < d.spin_limit;
    }
    __syncthreads();
    if (s_ready) {
        constexpr int kPer = R / 64;   // 8-byte words per thread
        const unsigned long long* src = reinterpret_cast<const unsigned long long*>(d.rank_buf);
        unsigned long long* dst = reinterpret_cast<unsigned long long*>(s_rank);
        unsigned long long w[kPer];
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            w[i] = __hip_atomic_load(src + threadIdx.x + 256 * i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < kPer; ++i) dst[threadIdx.x + 256 * i] = w[i];
    } else {
        for (int cc = 0; cc < d.nct; ++cc) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            for (int kb0 = 0; kb0 < d.ksa; kb0 += 4 * kDecodeMaxJ)
                acc += decode_rank_partial<A8>(d, M, cc, kb0, min(d.ksa, kb0 + 4 * kDecodeMaxJ), wave, lane);
            decode_wave_sum(red, acc, wave, lane);
            {
                const int m = threadIdx.x >> 4, n = threadIdx.x & 15;
                s_rank[m * R + cc * 16 + n] = decode_rank_epilogue(d, decode_tile_at(red, m, n), cc * 16 + n);
            }
            __syncthreads();   // red is rewritten by the next tile's sum
        }
    }
    __syncthreads();
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

template <int KSTEPS, typename BaseT, typename PriorT>
__global__ __launch_bounds__(256) void lowrank_decode_kernel(DecodeKArgs d) {
#pragma clang fp contract(off)
    const ArgmaxKArgs& a = d.am;
    constexpr int r = KSTEPS * 32;
    __shared__ float red[512];
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;
    __shared__ int s_ready;
    __shared__ __attribute__((aligned(16))) uint16_t s_rank[16 * r];   // the rank, [16][r] bf16

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    const int col = lane & 15;
    const int kg = lane >> 4;

    decode_publish_rank<false>(d, a.M, r, red, s_last);

    const int nwaves = gridDim.x * 4;
    int t = blockIdx.x * 4 + wave;
    float al[4], be[4], best[4];
    int bidx[4];
    bool use_prior[4];
    const BaseT* brow[4];
    const PriorT* prior = static_cast<const PriorT*>(a.prior);
    decode_rows<BaseT, PriorT>(a, kg, al, be, use_prior, brow, best, bidx);
    // The first two tiles of the argmax stream go in flight while the rank is finished.
    const int ntiles = (a.V + 15) >> 4;
    TileRegs<KSTEPS> ta, tb;
    const bool have_a = t < ntiles;
    const bool have_b = t + nwaves < ntiles;
    if (have_a) load_tile<KSTEPS, B_PACKED_EXACT>(a, t, lane, brow, prior, ta);
    if (have_b) load_tile<KSTEPS, B_PACKED_EXACT>(a, t + nwaves, lane, brow, prior, tb);

    decode_rank_into_lds<r, false>(d, a.M, red, s_ready, s_rank);
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
            float sc = acc[q] * al[q];
            sc = sc + tr.base[q];
            if (use_prior[q]) sc = sc - be[q] * tr.prior;
            const bool take = (v < a.V) & argmax_better(sc, v, best[q], bidx[q]);   // no short circuit: branch-free
            best[q] = take ? sc : best[q];
            bidx[q] = take ? v : bidx[q];
        }
    };
    // Invariant at the loop top: ta holds tile t and tb tile t + nwaves.  The
    // prefetch inside the loop is unconditional on the continuing path, so the
    // wait before each contraction covers only the older register set.
    if (have_b) {
        while (true) {
            consume(ta, t);
            if (t + 2 * nwaves >= ntiles) {
                consume(tb, t + nwaves);
                break;
            }
            load_tile<KSTEPS, B_PACKED_EXACT>(a, t + 2 * nwaves, lane, brow, prior, ta);
            t += nwaves;
            consume(tb, t);
            if (t + 2 * nwaves >= ntiles) {
                consume(ta, t + nwaves);
                break;
            }
            load_tile<KSTEPS, B_PACKED_EXACT>(a, t + 2 * nwaves, lane, brow, prior, tb);
            t += nwaves;
        }
    } else if (have_a) {
        consume(ta, t);
    }

    // ---- 5. cross-workgroup argmax --------------------------------------------
    argmax_wg_finish(a, best, bidx, 0, s_val, s_idx, s_last, d.done);
}

// fp8 variant: A e4m3 (K32 blocks) with per-column scales in the rank
// projection; rank quantised per row to e4m3; B e4m3 (K128 blocks) with
// per-row scales in the argmax.  KS8 = r / 128.
constexpr int kDecode8Ring = 3;   // LDS ring slots per wave (the rank takes 16 KB of LDS too)

template <int KS8, typename BaseT, typename PriorT, bool RING>
__global__ __launch_bounds__(256) void lowrank_decode8_kernel(DecodeKArgs d) {
#pragma clang fp contract(off)
    const ArgmaxKArgs& a = d.am;
    constexpr int r = KS8 * 128;
    __shared__ float red[512];
    __shared__ float s_val[4][16];
    __shared__ int s_idx[4][16];
    __shared__ int s_last;
    __shared__ int s_ready;
    __shared__ __attribute__((aligned(16))) uint16_t s_rank[16 * r];   // the rank, [16][r] bf16
    __shared__ __attribute__((aligned(1024))) char s_ring[RING ? 4 : 1][RING ? kDecode8Ring : 1]
                                                        [RING ? Ring8<KS8>::kSlot : 16];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // uniform: scalar loop control
    const int col = lane & 15;
    const int kg = lane >> 4;

    decode_publish_rank<true>(d, a.M, r, red, s_last);

    const int nwaves = gridDim.x * 4;
    const int t = blockIdx.x * 4 + wave;
    float al[4], be[4], best[4];
    int bidx[4];
    bool use_prior[4];
    const BaseT* brow[4];
    const PriorT* prior = static_cast<const PriorT*>(a.prior);
    decode_rows<BaseT, PriorT>(a, kg, al, be, use_prior, brow, best, bidx);
    const int ntiles = (a.V + 15) >> 4;
    // The first tiles of the argmax stream go in flight while the rank is finished.
    TileRegs8<KS8> ta, tb;
    uint32_t row_off = 0;
    int issued = 0;
    if constexpr (RING) {
        row_off = ring8_row_off<BaseT>(a, 0, lane);
        for (int i = 0; i < kDecode8Ring && t + i * nwaves < ntiles; ++i, ++issued)
            issue_tile8_lds<KS8, BaseT, PriorT>(a, t + i * nwaves, lane, row_off, &s_ring[wave][i][0]);
    } else {
        if (t < ntiles) load_tile8<KS8>(a, t, lane, brow, prior, ta);
        if (t + nwaves < ntiles) load_tile8<KS8>(a, t + nwaves, lane, brow, prior, tb);
    }

    decode_rank_into_lds<r, true>(d, a.M, red, s_ready, s_rank);
    __shared__ __attribute__((aligned(16))) uint8_t s_rq[16 * (r + 16)];
    __shared__ float s_rsc[16];
    quantize_rank_coop<r>(s_rank, r, a.M, s_rq, s_rsc);
    i32x8 rq[KS8];
    float rsc[4];
    load_rank_operand<KS8>(s_rq, s_rsc, lane, rq, rsc);
    if constexpr (RING)
        stream_tiles8_lds<KS8, kDecode8Ring, BaseT, PriorT>(a, rq, rsc, t, nwaves, ntiles, lane, row_off,
                                                            &s_ring[wave][0][0], issued, al, be, use_prior, best,
                                                            bidx);
    else
        stream_tiles8<KS8>(a, rq, rsc, t, nwaves, ntiles, lane, brow, prior, al, be, use_prior, best, bidx, ta, tb,
                           true);
    argmax_wg_finish(a, best, bidx, 0, s_val, s_idx, s_last, d.done);
}

// Dispatch over K steps of B (r / 32) and the prior type for one base dtype.
template <typename BaseT>
hipError_t launch_decode_for_base(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s) {
    auto go = [&](auto ks_tag, auto prior_tag) -> hipError_t {
        constexpr int KS = decltype(ks_tag)::value;
        using PT = decltype(prior_tag);
        hipLaunchKernelGGL((lowrank_decode_kernel<KS, BaseT, PT>), dim3(kDecodeWGs), dim3(256), 0, s, ka);
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
        const int pb = is_no_prior<PT>::value ? 0 : elem_bytes<PT>::value;
        if (ring8_eligible(ka.am, elem_bytes<BaseT>::value, pb))
            hipLaunchKernelGGL((lowrank_decode8_kernel<KS8, BaseT, PT, true>), dim3(kDecodeWGs), dim3(256), 0, s, ka);
        else
            hipLaunchKernelGGL((lowrank_decode8_kernel<KS8, BaseT, PT, false>), dim3(kDecodeWGs), dim3(256), 0, s, ka);
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

hipError_t launch_decode_f32(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s);
hipError_t launch_decode_bf16(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s);
hipError_t launch_decode_f16(const DecodeKArgs& ka, int ksteps, int prior_kind, hipStream_t s);
hipError_t launch_decode8_f32(const DecodeKArgs& ka, int prior_kind, hipStream_t s);
hipError_t launch_decode8_bf16(const DecodeKArgs& ka, int prior_kind, hipStream_t s);
hipError_t launch_decode8_f16(const DecodeKArgs& ka, int prior_kind, hipStream_t s);

}  // namespace dels

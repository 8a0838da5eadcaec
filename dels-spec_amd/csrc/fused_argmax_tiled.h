// Fused low-rank LM-head combine + vocabulary argmax: the batched (MFMA-tiled)
// kernel for many draft rows (batch x block verification, M >= 64).
//
// Semantics as the GEMV kernel (code/kernel/dels.py:42-138):
//     s[m, v] = fp32(rank_m . B[v]) * alpha_m + base[m, v] - beta_m * prior[v]
// and per row the lowest v attaining max_v s[m, v].
//
// Here the contraction rank[M, r] x B[V, r]^T is a real dense GEMM, computed
// transposed: each v_mfma_f32_16x16x32_bf16 takes a 16-vocabulary x 32-K slab of
// B (straight from the MFMA-16 block layout) as its A operand and a 32-K x
// 16-row slab of rank as its B operand, so lane l ends up holding four
// consecutive vocabulary columns 4*(l/16)+q of row l%16.  That puts one row per
// lane: the running argmax stays in the lane over the whole vocabulary chunk
// and the base logits it needs are four consecutive elements of one row.
//
// Workgroup: 8 waves, 2 waves per SIMD.  Wave w keeps the rank operand of its
// 32 rows (two 16-row tiles) in VGPRs for the whole kernel; a workgroup covers
// 256 rows and a contiguous chunk of the vocabulary.  The chunk is streamed in
// stages of TV 16-column tiles: B's stage is one contiguous run of the packed
// layout and is copied HBM -> LDS with direct-to-LDS loads
// (global_load_lds_dwordx4, no VGPR staging), together with each wave's
// base-logit tile (laid out so the epilogue reads it lane-contiguously) and the
// prior slice.  Stages are double-buffered in LDS with one barrier per stage,
// so the next stage's loads stay in flight across the contraction and
// epilogue of the current one.
//
// Workgroups sharing a vocabulary chunk (the row groups) have linear ids that
// differ by a multiple of 8, so they run on the same XCD and the second read of
// each B tile is served by that XCD's L2.
//
// Cross-workgroup reduction: each workgroup writes one 64-bit key per row
// (order(score) << 32 | ~index, 0 = no candidate) to a partials array
// [chunks, M]; a second small kernel takes the unsigned maximum over chunks
// -- the argmax with the lowest-index tie rule -- and decodes it.  No atomics,
// no counters, nothing to reset.
#pragma once

#include <algorithm>
#include <climits>
#include <type_traits>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

struct TiledKArgs {
    const uint16_t* rank; int64_t ldrank;
    const uint16_t* B;          // MFMA-16 blocks, ksteps = r / 32 exactly
    const void* base; int64_t ldbase;
    const void* prior;          // nullptr when there is no prior
    const float* alpha; int64_t alpha_stride;
    const float* beta; int64_t beta_stride;
    int M, V, ntiles;           // ntiles = ceil(V / 16)
    unsigned long long* part;   // [gridDim.x, M]
};

namespace tiled {

constexpr int kWaves = 8;
constexpr int kThreads = kWaves * 64;
constexpr int kRowTiles = 2;                      // 16-row tiles per wave
constexpr int kRowsPerWG = kWaves * kRowTiles * 16;
constexpr int kTV = 2;                            // 16-column vocabulary tiles per stage
constexpr int kStageCols = kTV * 16;

// LDS bytes of the parts of one stage buffer.
template <int KSTEPS, typename BaseT>
constexpr int b_bytes() { return kTV * KSTEPS * 1024; }
template <typename BaseT>
constexpr int base_bytes_per_wave() { return kRowTiles * 16 * kStageCols * (int)sizeof(BaseT); }
constexpr int kPriorBytesPerWave = 256;

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ void dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds, 16, 0, 0);
}
__device__ __forceinline__ void dma4(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)lds, 4, 0, 0);
}

// Workgroup barrier for the stage buffers.  Before it, each wave waits for all
// of its own memory operations, in particular its direct-to-LDS loads: those
// count in vmcnt, and the LDS-only release fence does not wait for them on
// every path (the loop back edge), so the wait is explicit.  Other waves read
// the B tiles this wave loaded as soon as they pass the barrier.  The fences
// keep the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_waitcnt(0);   // vmcnt(0) expcnt(0) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename BaseT>
__device__ __forceinline__ void base4_from_lds(const char* p, float (&o)[4]) {
    if constexpr (sizeof(BaseT) == 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(p);
        o[0] = v[0]; o[1] = v[1]; o[2] = v[2]; o[3] = v[3];
    } else {
        const uint2 v = *reinterpret_cast<const uint2*>(p);
        const uint32_t w[2] = {v.x, v.y};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            if constexpr (std::is_same<BaseT, bf16_t>::value) {
                o[2 * i] = bf16_bits_to_f32(w[i] & 0xffffu);
                o[2 * i + 1] = bf16_bits_to_f32(w[i] >> 16);
            } else {
                _Float16 h0, h1;
                const uint16_t b0 = (uint16_t)(w[i] & 0xffffu), b1 = (uint16_t)(w[i] >> 16);
                __builtin_memcpy(&h0, &b0, 2);
                __builtin_memcpy(&h1, &b1, 2);
                o[2 * i] = (float)h0;
                o[2 * i + 1] = (float)h1;
            }
        }
    }
}

}  // namespace tiled

template <int KSTEPS, typename BaseT, typename PriorT>
__global__ __launch_bounds__(tiled::kThreads) void fused_argmax_tiled_kernel(TiledKArgs a) {
#pragma clang fp contract(off)
    using namespace tiled;
    constexpr int kB = b_bytes<KSTEPS, BaseT>();
    constexpr int kBaseW = base_bytes_per_wave<BaseT>();
    constexpr bool kPrior = !is_no_prior<PriorT>::value;
    // One stage buffer: B tiles, every wave's base tile, every wave's prior slice.
    struct __attribute__((aligned(1024))) Stage {
        char b[kB];
        char base[kWaves][kBaseW];
        char prior[kWaves][kPriorBytesPerWave];
    };
    // Two distinct LDS objects rather than one array indexed by parity: the
    // compiler can then tell that reads of one buffer do not depend on the
    // direct-to-LDS loads in flight into the other, and inserts no wait for them.
    __shared__ Stage lds0, lds1;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int col = lane & 15;      // row (within a 16-row tile) of this lane
    const int kg = lane >> 4;       // K group of the operands / vocabulary quad of the results
    const int mw = blockIdx.y * kRowsPerWG + wave * (kRowTiles * 16);   // first row of this wave
    const bool wave_active = mw < a.M;

    // Vocabulary chunk of this workgroup: tiles [t0, t1).
    const int t0 = (int)(((int64_t)blockIdx.x * a.ntiles) / gridDim.x);
    const int t1 = (int)(((int64_t)(blockIdx.x + 1) * a.ntiles) / gridDim.x);
    const int nst = (t1 - t0 + kTV - 1) / kTV;
    const int vend = min(a.V, t1 * 16);

    // Rank operand of the wave's rows, resident for the whole kernel.
    bf16x8 ra[kRowTiles][KSTEPS];
    float al[kRowTiles], be[kRowTiles], best[kRowTiles];
    int bidx[kRowTiles];
    bool use_prior[kRowTiles];
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
        const int m = min(mw + rt * 16 + col, a.M - 1);
        const uint16_t* rp = a.rank + (int64_t)m * a.ldrank + kg * 8;
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) ra[rt][s] = load_bf16x8(rp + s * 32);
        al[rt] = a.alpha[(int64_t)m * a.alpha_stride];
        be[rt] = a.beta[(int64_t)m * a.beta_stride];
        use_prior[rt] = kPrior && be[rt] != 0.f;
        best[rt] = -__builtin_inff();
        bidx[rt] = INT_MAX;
    }

    const char* Bg = reinterpret_cast<const char*>(a.B);
    const char* baseg = static_cast<const char*>(a.base);
    const char* priorg = static_cast<const char*>(a.prior);

    // Issue the direct-to-LDS loads of stage `st` into buffer S.  Addresses past
    // the chunk are clamped to valid memory (their results are masked in the
    // epilogue).
    auto issue_stage = [&](Stage& S, int st) {
        const int tb = t0 + st * kTV;
        // B: kTV * KSTEPS blocks of 1 KiB, contiguous in the packed layout.
        constexpr int nb = kTV * KSTEPS / kWaves;
#pragma unroll
        for (int j = 0; j < nb; ++j) {
            const int blk = wave * nb + j;                  // block within the stage
            const int t = min(tb + blk / KSTEPS, t1 - 1);   // clamped tile
            const int64_t goff = ((int64_t)t * KSTEPS + blk % KSTEPS) * 1024 + lane * 16;
            dma16(Bg + goff, S.b + blk * 1024);
        }
        // Base logits of the wave's rows: lane L of each 1 KiB load is row L%16,
        // 16-byte chunk L/16 of the stage's columns.
        const int vs = tb * 16;
#pragma unroll
        for (int rt = 0; rt < kRowTiles; ++rt) {
            const int m = min(mw + rt * 16 + col, a.M - 1);
            const char* rowp = baseg + (int64_t)m * a.ldbase * (int64_t)sizeof(BaseT);
            if constexpr (sizeof(BaseT) == 4) {
#pragma unroll
                for (int t = 0; t < kTV; ++t) {
                    const int v = min(vs + t * 16 + kg * 4, a.V - 4);
                    dma16(rowp + (int64_t)v * 4, S.base[wave] + (rt * kTV + t) * 1024);
                }
            } else {
                const int v = min(vs + kg * 8, a.V - 8);
                dma16(rowp + (int64_t)v * 2, S.base[wave] + rt * 1024);
            }
        }
        // Prior slice of the stage's columns (one dword per lane).
        if constexpr (kPrior) {
            if constexpr (sizeof(PriorT) == 4) {
                const int v = min(vs + (lane & 31), a.V - 1);
                dma4(priorg + (int64_t)v * 4, S.prior[wave]);
            } else {
                const int v = min(vs + 2 * (lane & 15), a.V - 2);
                dma4(priorg + (int64_t)v * 2, S.prior[wave]);
            }
        }
    };

    // Epilogue operands of one stage, read from LDS into registers before the
    // next stage's loads are issued (so no read of this stage can be made to
    // wait for them).
    struct EpiRegs {
        float base[kTV][kRowTiles][4];
        float prior[kTV][4];
    };
    auto read_epilogue = [&](const Stage& S, EpiRegs& e) {
        const char* Lb = S.base[wave];
        const char* Lp = S.prior[wave];
#pragma unroll
        for (int t = 0; t < kTV; ++t) {
            if constexpr (kPrior) {
                if constexpr (sizeof(PriorT) == 4) {
                    const f32x4 p = *reinterpret_cast<const f32x4*>(Lp + (t * 16 + kg * 4) * 4);
                    e.prior[t][0] = p[0]; e.prior[t][1] = p[1]; e.prior[t][2] = p[2]; e.prior[t][3] = p[3];
                } else {
                    base4_from_lds<PriorT>(Lp + (t * 16 + kg * 4) * 2, e.prior[t]);
                }
            } else {
                e.prior[t][0] = e.prior[t][1] = e.prior[t][2] = e.prior[t][3] = 0.f;
            }
#pragma unroll
            for (int rt = 0; rt < kRowTiles; ++rt) {
                if constexpr (sizeof(BaseT) == 4)
                    base4_from_lds<BaseT>(Lb + (rt * kTV + t) * 1024 + lane * 16, e.base[t][rt]);
                else
                    base4_from_lds<BaseT>(Lb + rt * 1024 + (col + 16 * (2 * t + (kg >> 1))) * 16 + (kg & 1) * 8,
                                          e.base[t][rt]);
            }
        }
    };

    auto consume_stage = [&](const Stage& S, const EpiRegs& e, int st) {
        f32x4 acc[kTV][kRowTiles];
#pragma unroll
        for (int t = 0; t < kTV; ++t)
#pragma unroll
            for (int rt = 0; rt < kRowTiles; ++rt) acc[t][rt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
            for (int t = 0; t < kTV; ++t) {
                const bf16x8 bv = *reinterpret_cast<const bf16x8*>(S.b + (t * KSTEPS + s) * 1024 + lane * 16);
#pragma unroll
                for (int rt = 0; rt < kRowTiles; ++rt)
                    acc[t][rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bv, ra[rt][s], acc[t][rt], 0, 0, 0);
            }
        }
        const int vs = (t0 + st * kTV) * 16;
#pragma unroll
        for (int t = 0; t < kTV; ++t) {
#pragma unroll
            for (int rt = 0; rt < kRowTiles; ++rt) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int v = vs + t * 16 + kg * 4 + q;
                    float sc = acc[t][rt][q] * al[rt];
                    sc = sc + e.base[t][rt][q];
                    const float scp = sc - be[rt] * e.prior[t][q];
                    sc = use_prior[rt] ? scp : sc;
                    // branch-free: (in chunk) and (larger, or equal at a lower index)
                    const bool take = (v < vend) & ((sc > best[rt]) | ((sc == best[rt]) & (v < bidx[rt])));
                    best[rt] = take ? sc : best[rt];
                    bidx[rt] = take ? v : bidx[rt];
                }
            }
        }
    };

    // Double-buffered pipeline, one barrier per stage: past the barrier, stage st
    // has landed for every wave and the other buffer (read during stage st-1) is
    // free, so stage st+1 is issued into it and streams in while stage st is
    // contracted.  Unrolled by two so each half names its buffers statically.
    if (nst > 0) issue_stage(lds0, 0);
    for (int st = 0; st < nst; st += 2) {
        EpiRegs e;
        lds_barrier();
        read_epilogue(lds0, e);
        if (st + 1 < nst) issue_stage(lds1, st + 1);
        if (wave_active) consume_stage(lds0, e, st);
        if (st + 1 >= nst) break;
        lds_barrier();
        read_epilogue(lds1, e);
        if (st + 2 < nst) issue_stage(lds0, st + 2);
        if (wave_active) consume_stage(lds1, e, st + 1);
    }

    // Reduce the four vocabulary quads of each row (lanes l, l^16, l^32, l^48).
#pragma unroll
    for (int rt = 0; rt < kRowTiles; ++rt) {
#pragma unroll
        for (int off = 16; off < 64; off <<= 1) {
            const float ov = __shfl_xor(best[rt], off, 64);
            const int oi = __shfl_xor(bidx[rt], off, 64);
            if (argmax_better(ov, oi, best[rt], bidx[rt])) {
                best[rt] = ov;
                bidx[rt] = oi;
            }
        }
        const int m = mw + rt * 16 + col;
        if (kg == 0 && m < a.M) {
            const unsigned long long key = bidx[rt] == INT_MAX ? 0ull : pack_argmax(best[rt], (uint32_t)bidx[rt]);
            a.part[(int64_t)blockIdx.x * a.M + m] = key;
        }
    }
}

// Grid of the tiled kernel: row groups of 256 rows times vocabulary chunks,
// about one workgroup per CU, chunk count a multiple of 8 (XCD pairing).
inline void tiled_grid(int M, int V, int cus, int* gx, int* gy) {
    const int groups = (M + tiled::kRowsPerWG - 1) / tiled::kRowsPerWG;
    const int ntiles = (V + 15) / 16;
    int x = std::max(1, cus / groups);
    if (x >= 8) x -= x % 8;
    x = std::max(1, std::min(x, (ntiles + tiled::kTV - 1) / tiled::kTV));
    *gx = x;
    *gy = groups;
}

template <int KSTEPS, typename BaseT, typename PriorT>
hipError_t launch_tiled_inst(const TiledKArgs& ka, int gx, int gy, hipStream_t s) {
    hipLaunchKernelGGL((fused_argmax_tiled_kernel<KSTEPS, BaseT, PriorT>), dim3(gx, gy, 1), dim3(tiled::kThreads), 0,
                       s, ka);
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

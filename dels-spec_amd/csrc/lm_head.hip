// The target LM head of a draft block, base = hidden . W^T (code/dflash.py:468:
// target.lm_head(parallel_hiddens), bf16 output), with the argmax of chosen
// rows fused into the GEMM so that their logits never reach memory
// (sample(base_logits[:, :1]), code/dflash.py:475).
//
// Shape: M rows of hidden (a draft block's batch x k positions, about a
// hundred) against W [V, K] (K = 4096, V = 151936: 1.245 GB of bf16).  At this
// M the product is bound by streaming W from HBM once (about M FLOP per byte,
// far under the MFMA ridge), so the kernel is built around that stream.  W is
// packed once (dels_pack_lm_head) into MFMA-16 blocks in K-chunk-major order:
// the 4 KiB of one 16-row tile in one K chunk (128 K) are contiguous, and so
// are the tiles of one chunk, so that the whole GPU reads W as one sweep per
// chunk (DRAM-page friendly) instead of thousands of 128 KiB-strided pieces.
//   * one wave per SIMD, each owning 64 vocabulary columns at a time (four
//     16-row tiles) for all 128 rows of its row group; W goes straight from
//     HBM into registers, double-buffered by K chunk (register sets of 8 K
//     steps of 16), the loads of the next chunk spread between the MFMAs of
//     the current one (four sets were no faster: register pressure made the
//     compiler wait for them early);
//   * hidden, shared by every column, is staged through LDS in chunks of
//     128 rows x 128 K (32 KiB, a ring of three), copied two chunks ahead by
//     direct-to-LDS loads.  A CU returns its loads in issue order, so waiting
//     for hidden chunk g+1 waits for every W load issued before it: issuing
//     it two chunks ahead keeps the two youngest W chunks in flight through
//     that wait (one ahead made every wait drain all but the newest W set);
//   * v_mfma_f32_32x32x16_bf16: A = 32 rows x 16 K of hidden (one LDS KiB),
//     B = 32 columns x 16 K of W gathered from two MFMA-16 blocks (two
//     contiguous 512-byte runs per load); every LDS read feeds two MFMAs.
// Accumulators: row 32 rb + 8 (j/4) + 4 (l/32) + j%4, column 32 cb + l%32.
//
// Epilogue of a pass (64 columns): the values are rounded to bf16 (as
// nn.Linear's output) and staged through the wave's 4 KiB of LDS per 16
// columns.  Rows m with argmax_period > 0 and m % argmax_period == 0 are argmax
// rows: their bf16 values enter the argmax (lowest index on ties, the first
// NaN wins, as torch.argmax) as 64-bit keys merged by LDS atomic maxima into
// one key per row of the workgroup, and are not stored; every other row is
// stored to `base` (16-byte stores) when it is given.  (A device-scope atomic
// per tile here would make the wave wait for its returned value -- and so,
// loads returning in order, for all of its W loads in flight -- at every
// epilogue.)  At the end each workgroup merges its row keys into the global
// ones; the last workgroup to finish decodes them and returns keys and
// counter to zero.
#include <algorithm>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

namespace {

constexpr int kLhWaves = 4;                 // one per SIMD: two W sets and 128 accumulators
constexpr int kLhThreads = kLhWaves * 64;
constexpr int kLhRows = 128;                // rows per workgroup: 4 blocks of 32
constexpr int kLhRB = kLhRows / 32;
constexpr int kLhCB = 2;                    // 32-column blocks per wave and pass: each LDS read feeds two MFMAs
constexpr int kLhKC = kLmHeadKChunk;       // 32-K blocks per chunk (8 MFMA K steps of 16)
constexpr int kLhS = 2 * kLhKC;
constexpr int kLhChunkBytes = kLhRB * kLhS * 1024;    // 32 KiB of hidden per chunk
constexpr int kLhHLoads = kLhRB * kLhS / kLhWaves;    // 16-byte hidden loads per lane and chunk
constexpr int kLhWLoads = kLhCB * kLhS;               // 16-byte W loads per lane and chunk
constexpr int kLhRing = 3;                  // hidden chunks in LDS: in use, landed, in flight

struct LmHeadArgs {
    const uint16_t* hidden; int64_t ldh;
    const uint16_t* W;                      // [V, K] in MFMA-16 blocks
    int M, K, V;
    uint16_t* base; int64_t ldo;            // bf16 output (nullptr: none)
    bool vec_store;                         // base 16-byte aligned and ldo % 8 == 0
    int argmax_period;                      // 0: no argmax rows
    int64_t* out_ids; float* out_score; int64_t ld_out;
    unsigned long long* keys; int64_t key_stride;
    unsigned int* counter;
};

__device__ __forceinline__ unsigned long long lh_key(float v, uint32_t idx) {
    return pack_argmax(v != v ? __uint_as_float(0x7fc00000u) : v, idx);
}

__device__ __forceinline__ unsigned long long lh_shfl_xor(unsigned long long x, int off) {
    const uint32_t lo = __shfl_xor((uint32_t)x, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(x >> 32), off, 64);
    return ((unsigned long long)hi << 32) | lo;
}

typedef bf16x8 WSet[kLhCB][kLhS];

// Wait until at most N of this wave's vector-memory operations are
// outstanding (its direct-to-LDS loads included, which the compiler does not
// track) and its LDS operations are done, then the workgroup barrier.
template <int N>
__device__ __forceinline__ void lh_wait_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__global__ __launch_bounds__(kLhThreads) void lm_head_kernel(LmHeadArgs a) {
    __shared__ __attribute__((aligned(1024))) char ring[kLhRing][kLhChunkBytes];
    __shared__ __attribute__((aligned(16))) uint16_t stage[kLhWaves][kLhRows * 16];
    __shared__ int s_last;
    __shared__ unsigned long long s_keys[kLhRows];   // argmax keys of the workgroup's rows

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, hk = lane >> 5;
    const int row0 = blockIdx.y * kLhRows;
    const int KB = a.K / 32;                 // 32-K blocks per 16-row tile of W
    const int nchunks = KB / kLhKC;

    // 16-row vocabulary tiles [T0, T1) of this workgroup, 16 per pass: in pass p
    // wave w takes tiles T0 + 16p + 4w + i (slots i < 4; column block i / 2), so
    // at every chunk the workgroup reads one contiguous run of W (16 tiles x
    // 4 KiB in the K-chunk-major layout) and all workgroups together one
    // contiguous range.  In a last, partial pass a column block whose tiles all
    // lie past T1 skips its MFMAs.  (Dealing the slots round-robin over the
    // waves, so that a partial pass has fewer live blocks per wave, measured
    // 5 % slower.)
    const int ntiles = (a.V + 15) / 16;
    const int T0 = (int)(((int64_t)blockIdx.x * ntiles) / gridDim.x);
    const int T1 = (int)(((int64_t)(blockIdx.x + 1) * ntiles) / gridDim.x);
    constexpr int kTilesPerPass = 2 * kLhCB * kLhWaves;
    const int npass = (T1 - T0 + kTilesPerPass - 1) / kTilesPerPass;
    const int G = npass * nchunks;           // chunks of the walk, the same for every wave

    // tile of slot i of this wave in pass p; past T1 it repeats the workgroup's last tile (L2 hits, results dropped)
    auto tile16 = [&](int p, int i) {
        const int x = T0 + p * kTilesPerPass + 2 * kLhCB * wave + i;
        return x < T1 ? x : T1 - 1;
    };
    auto tile_live = [&](int p, int i) { return T0 + p * kTilesPerPass + 2 * kLhCB * wave + i < T1; };
    auto kchunk = [&](int g) { return g % nchunks; };

    // ---- hidden: chunk c = K blocks [c*KC, (c+1)*KC); LDS block (rb, s) holds the
    // 32x16 A operand of row block rb and K step s in lane order (row l%32, K 16 s + 8 (l/32)).
    // Chunk g of the walk goes to ring buffer g % 3 by kLhHLoads direct-to-LDS
    // loads per lane (past the walk: its last chunk again); byte offsets fit
    // 32 bits (the hidden rows span less than 2 GiB, checked at launch).
    auto issue_hidden_one = [&](int g, int i) {
        const int c = kchunk(g < G ? g : G - 1);
        char* buf = ring[g % kLhRing];
        const int j = wave * kLhHLoads + i;
        const int rb = j / kLhS, s = j % kLhS;
        const int row = min(row0 + rb * 32 + l32, a.M - 1);
        const uint32_t off = (uint32_t)(((int64_t)row * a.ldh + c * (kLhKC * 32) + s * 16 + hk * 8) * 2);
        dma16(a.hidden, off, buf + j * 1024);
    };

    // ---- W: the B operand of column block cb, K step s of chunk g: column 32 cb + l%32
    // of the pass -> slot 2 cb + (l%32)/16, row l%16; K 16 s + 8 (l/32) -> 32-K block
    // c*KC + s/2, lane (l%16) + 16 (2 (s%2) + l/32) of that 1 KiB block, which the
    // K-chunk-major layout keeps at block ((c * ntiles + tile) * KC + s/2).
    // Load q (0 <= q < kLhWLoads) of chunk g: column block q / kLhS, K step q % kLhS.
    auto load_w_one = [&](int g, WSet& w, int q) {
        const int gg = g < G ? g : G - 1;
        const int p = gg / nchunks, c = kchunk(gg);
        const int cb = q / kLhS, s = q % kLhS;
        const int t = tile16(p, 2 * cb + (l32 >> 4));
        const uint16_t* bp = a.W + ((int64_t)c * ntiles + t) * (kLhKC * 512) + ((l32 & 15) + 16 * hk) * 8;
        w[cb][s] = load_bf16x8_nt(bp + (s >> 1) * 512 + (s & 1) * 256);
    };

    f32x16 acc[kLhRB][kLhCB];
#pragma unroll
    for (int rb = 0; rb < kLhRB; ++rb)
#pragma unroll
        for (int cb = 0; cb < kLhCB; ++cb)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[rb][cb][j] = 0.f;

    // Contraction of chunk g for the first NCB column blocks, with the loads of
    // the step (W chunk gw into `ahead`, hidden chunk gh) spread between the
    // MFMA slots k = (s * kLhRB + rb) * kLhCB + cb of 64: W load q at slot
    // 4q + 1, hidden load i at slot 4i + 3, so the loads go out in the order
    // W0 H0 W1 H1 .. W7 H7 W8 .. W15 whatever NCB is (a skipped column block
    // keeps its slots, without the MFMA).  A operands (hidden) are read from
    // LDS one K step ahead.
    static_assert(kLhS * kLhRB * kLhCB == 64 && kLhWLoads == 16 && kLhHLoads == 8, "slot plan");
    auto contract_issue = [&](auto ncb_tag, int g, const WSet& w, int gw, WSet& ahead, int gh) {
        constexpr int NCB = decltype(ncb_tag)::value;
        const char* buf = ring[g % kLhRing] + lane * 16;
        bf16x8 hq[2][kLhRB];
        if constexpr (NCB > 0) {
#pragma unroll
            for (int rb = 0; rb < kLhRB; ++rb) hq[0][rb] = *reinterpret_cast<const bf16x8*>(buf + rb * kLhS * 1024);
        }
#pragma unroll
        for (int s = 0; s < kLhS; ++s) {
            if (NCB > 0 && s + 1 < kLhS) {
#pragma unroll
                for (int rb = 0; rb < kLhRB; ++rb)
                    hq[(s + 1) & 1][rb] = *reinterpret_cast<const bf16x8*>(buf + (rb * kLhS + s + 1) * 1024);
            }
#pragma unroll
            for (int rb = 0; rb < kLhRB; ++rb)
#pragma unroll
                for (int cb = 0; cb < kLhCB; ++cb) {
                    const int k = (s * kLhRB + rb) * kLhCB + cb;
                    __builtin_amdgcn_sched_barrier(0);
                    if (cb < NCB)
                        acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hq[s & 1][rb], w[cb][s], acc[rb][cb],
                                                                              0, 0, 0);
                    __builtin_amdgcn_sched_barrier(0);
                    if ((k & 3) == 1) load_w_one(gw, ahead, k >> 2);
                    if ((k & 3) == 3 && (k >> 2) < kLhHLoads) issue_hidden_one(gh, k >> 2);
                }
        }
    };

    // ---- epilogue of pass p, 16 columns (one tile) at a time through the wave's 4 KiB of LDS
    uint16_t* stg = stage[wave];
    auto epilogue = [&](int p) {
#pragma unroll
        for (int cb = 0; cb < kLhCB; ++cb) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int i = 2 * cb + half;          // slot of the pass
                if ((l32 >> 4) == half) {
#pragma unroll
                    for (int rb = 0; rb < kLhRB; ++rb)
#pragma unroll
                        for (int j = 0; j < 16; ++j)
                            stg[(rb * 32 + 8 * (j >> 2) + 4 * hk + (j & 3)) * 16 + (l32 & 15)] =
                                f32_to_bf16_bits(acc[rb][cb][j]);
                }
                if (half == 1) {
#pragma unroll
                    for (int rb = 0; rb < kLhRB; ++rb)
#pragma unroll
                        for (int j = 0; j < 16; ++j) acc[rb][cb][j] = 0.f;
                }
                if (!tile_live(p, i)) continue;       // wave-uniform
                const int v0 = tile16(p, i) * 16;
                const int vend = min(a.V, v0 + 16);
                if (a.base != nullptr) {
                    for (int q = lane; q < kLhRows * 2; q += 64) {
                        const int r = q >> 1, c8 = (q & 1) * 8;
                        const int m = row0 + r;
                        if (m >= a.M || v0 + c8 >= vend || (a.argmax_period > 0 && m % a.argmax_period == 0)) continue;
                        uint16_t* dst = a.base + (int64_t)m * a.ldo + v0 + c8;
                        if (a.vec_store && v0 + c8 + 8 <= vend) {
                            *reinterpret_cast<u32x4*>(dst) = *reinterpret_cast<const u32x4*>(stg + r * 16 + c8);
                        } else {
                            for (int e = 0; e < 8 && v0 + c8 + e < vend; ++e) dst[e] = stg[r * 16 + c8 + e];
                        }
                    }
                }
                if (a.argmax_period > 0) {
                    // argmax rows m = j * period of this row group, four per round (16 lanes each)
                    const int j0 = (row0 + a.argmax_period - 1) / a.argmax_period;
                    const int mend = min(row0 + kLhRows, a.M);
                    const int c16 = lane & 15, q4 = lane >> 4;
                    for (int jb = j0; jb * a.argmax_period < mend; jb += 4) {
                        const int jr = jb + q4;
                        const int m = jr * a.argmax_period;
                        const int v = v0 + c16;
                        unsigned long long key = 0ull;
                        if (m < mend && v < vend) key = lh_key(bf16_bits_to_f32(stg[(m - row0) * 16 + c16]), (uint32_t)v);
#pragma unroll
                        for (int off = 1; off < 16; off <<= 1) {
                            const unsigned long long o = lh_shfl_xor(key, off);
                            key = o > key ? o : key;
                        }
                        if (c16 == 0 && key != 0ull)
                            __hip_atomic_fetch_max(&s_keys[m - row0], key, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_WORKGROUP);
                    }
                }
            }
        }
    };

    // ---- walk over chunks g = p * nchunks + c: chunk g uses W set g % 2 and
    // hidden buffer g % 3.  Step g contracts chunk g while it issues the W
    // loads of g+1 (unconditionally: past the walk they reload its last chunk)
    // and the hidden loads of g+2, then waits for hidden g+1 and synchronises
    // the workgroup.  Every step issues the same loads in the same order, so at
    // its end exactly kAfter loads are younger than the last load of hidden
    // g+1 (the 8 W loads that follow it in the previous step and the 24 of this
    // one; epilogue stores only add to them): waiting for vmcnt(kAfter) lands
    // g+1 and leaves those in flight.  The prologue issues the loads of the two
    // steps before step 0.  nchunks is even, so both steps of a loop turn
    // belong to one pass; the epilogue of a pass runs between passes.
    constexpr int kAfter = (kLhWLoads - kLhHLoads) + kLhWLoads + kLhHLoads;
    static_assert(kAfter < 64, "vmcnt range");
    for (int r = threadIdx.x; r < kLhRows; r += kLhThreads) s_keys[r] = 0ull;   // published by the first barrier
    WSet wa, wb;
#pragma unroll
    for (int i = 0; i < kLhHLoads; ++i) issue_hidden_one(0, i);
#pragma unroll
    for (int q = 0; q < kLhWLoads; ++q) {
        load_w_one(0, wa, q);
        if (q < kLhHLoads) issue_hidden_one(1, q);
    }
    lh_wait_barrier<kLhWLoads + kLhHLoads>();               // hidden 0 landed
    auto step = [&](int g, const WSet& cur, WSet& ahead) {
        const int p = g / nchunks;                          // wave-uniform
        if (tile_live(p, 2)) contract_issue(std::integral_constant<int, 2>{}, g, cur, g + 1, ahead, g + 2);
        else if (tile_live(p, 0)) contract_issue(std::integral_constant<int, 1>{}, g, cur, g + 1, ahead, g + 2);
        else contract_issue(std::integral_constant<int, 0>{}, g, cur, g + 1, ahead, g + 2);
        lh_wait_barrier<kAfter>();                          // hidden g+1 landed everywhere
    };
    for (int p = 0; p < npass; ++p) {
        for (int c = 0; c < nchunks; c += 2) {
            step(p * nchunks + c, wa, wb);
            step(p * nchunks + c + 1, wb, wa);
        }
        epilogue(p);
    }
    // the reloads past the walk are still in flight: no direct-to-LDS write may
    // outlive the workgroup
    __builtin_amdgcn_s_waitcnt(0x0070 | (0xf << 8));   // vmcnt(0)

    if (a.argmax_period <= 0) return;
    __syncthreads();   // every wave's LDS maxima are in s_keys
    unsigned long long seen = 0;
    for (int r = threadIdx.x; r < kLhRows; r += kLhThreads) {
        const int m = row0 + r;
        const unsigned long long key = s_keys[r];
        if (m < a.M && m % a.argmax_period == 0 && key != 0ull)
            seen |= __hip_atomic_fetch_max(&a.keys[(int64_t)(m / a.argmax_period) * a.key_stride], key,
                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    // Using the returned values orders the maxima before the barrier, and so
    // before the workgroup is counted in (the write is never taken).
    if (seen == ~0ull) s_last = 2;
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned total = gridDim.x * gridDim.y;
        const unsigned prev = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == total - 1;
    }
    __syncthreads();
    if (s_last != 1) return;
    const int nrows = (a.M + a.argmax_period - 1) / a.argmax_period;
    for (int r = threadIdx.x; r < nrows; r += blockDim.x) {
        const unsigned long long key = __hip_atomic_exchange(&a.keys[(int64_t)r * a.key_stride], 0ull,
                                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        uint32_t idx = ~(uint32_t)(key & 0xffffffffull);
        float val = f32_from_order_key((uint32_t)(key >> 32));
        if (key == 0ull || idx >= (uint32_t)a.V) {
            idx = 0;
            val = -__builtin_inff();
        }
        a.out_ids[(int64_t)r * a.ld_out] = (int64_t)idx;
        if (a.out_score) a.out_score[(int64_t)r * a.ld_out] = val;
    }
    if (threadIdx.x == 0) __hip_atomic_exchange(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

bool lm_head_supported(int64_t M, int64_t K, int64_t V, int64_t argmax_period) {
    if (M < 1 || M > (int64_t)kLhRows * 64 || V < 1 || V >= INT32_MAX) return false;
    if (K < 1 || K >= (int64_t(1) << 26) || K % (64 * kLhKC) != 0) return false;   // an even chunk count
    if (argmax_period < 0 || argmax_period >= (int64_t(1) << 24)) return false;
    return argmax_period == 0 || (M - 1) / argmax_period + 1 <= kMaxKeyRows;
}

hipError_t launch_lm_head(const void* hidden, int64_t ldh, const void* W, int M, int K, int V, void* base,
                          int64_t ldo, int argmax_period, int64_t* out_ids, float* out_score, int64_t ld_out,
                          void* ws, hipStream_t s) {
    char* w = static_cast<char*>(ws);
    LmHeadArgs a{};
    a.hidden = static_cast<const uint16_t*>(hidden); a.ldh = ldh;
    a.W = static_cast<const uint16_t*>(W);
    a.M = M; a.K = K; a.V = V;
    a.base = static_cast<uint16_t*>(base); a.ldo = ldo;
    a.vec_store = (reinterpret_cast<uintptr_t>(base) & 15) == 0 && ldo % 8 == 0;
    a.argmax_period = argmax_period;
    a.out_ids = out_ids; a.out_score = out_score; a.ld_out = ld_out;
    a.counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
    a.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    const int nrows = argmax_period > 0 ? (M + argmax_period - 1) / argmax_period : 0;
    a.key_stride = (int64_t)nrows * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
    const int groups = (M + kLhRows - 1) / kLhRows;
    const int ntiles = (V + 15) / 16;
    const int gx = std::max(1, std::min(ntiles, device_cu_count() / groups));
    hipLaunchKernelGGL(lm_head_kernel, dim3(gx, groups, 1), dim3(kLhThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dels

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
//     steps of 16);
//   * hidden, shared by every column, is staged through LDS in chunks of
//     128 rows x 128 K (32 KiB, two buffers), loaded one chunk ahead with
//     ordinary loads and written with ds_write, so every wait stays the
//     compiler's;
//   * v_mfma_f32_32x32x16_bf16: A = 32 rows x 16 K of hidden (one LDS KiB),
//     B = 32 columns x 16 K of W gathered from two MFMA-16 blocks (two
//     contiguous 512-byte runs per load); every LDS read feeds two MFMAs.
// Accumulators: row 32 rb + 8 (j/4) + 4 (l/32) + j%4, column 32 cb + l%32.
//
// Epilogue of a pass (64 columns): the values are rounded to bf16 (as
// nn.Linear's output) and staged through the wave's 4 KiB of LDS per 16
// columns.  Rows m with argmax_period > 0 and m % argmax_period == 0 are argmax
// rows: their bf16 values enter the argmax (lowest index on ties, the first
// NaN wins, as torch.argmax) through one device-scope atomic max per row and
// 16 columns on a 64-bit key, and are not stored; every other row is stored to
// `base` (16-byte stores) when it is given.  The last workgroup to finish
// decodes the argmax keys and returns keys and counter to zero.
#include <algorithm>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

namespace {

constexpr int kLhWaves = 4;                 // one per SIMD (512 registers: three W sets and 128 accumulators)
constexpr int kLhThreads = kLhWaves * 64;
constexpr int kLhRows = 128;                // rows per workgroup: 4 blocks of 32
constexpr int kLhRB = kLhRows / 32;
constexpr int kLhCB = 2;                    // 32-column blocks per wave and pass: each LDS read feeds two MFMAs
constexpr int kLhKC = kLmHeadKChunk;       // 32-K blocks per chunk (8 MFMA K steps of 16)
constexpr int kLhS = 2 * kLhKC;
constexpr int kLhChunkBytes = kLhRB * kLhS * 1024;    // 32 KiB of hidden per chunk
constexpr int kLhHLoads = kLhRB * kLhS / kLhWaves;    // 16-byte hidden loads per lane and chunk
constexpr int kLhRing = 2;                  // hidden chunks in LDS: the one in use and the next

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

__global__ __launch_bounds__(kLhThreads) void lm_head_kernel(LmHeadArgs a) {
    __shared__ __attribute__((aligned(1024))) char ring[kLhRing][kLhChunkBytes];
    __shared__ __attribute__((aligned(16))) uint16_t stage[kLhWaves][kLhRows * 16];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int l32 = lane & 31, hk = lane >> 5;
    const int row0 = blockIdx.y * kLhRows;
    const int KB = a.K / 32;                 // 32-K blocks per 16-row tile of W
    const int nchunks = KB / kLhKC;

    // 16-row vocabulary tiles [T0, T1) of this workgroup; in pass p wave w takes
    // tiles T0 + 16p + 4w .. + 3 (two 32-column blocks), so at every
    // chunk the workgroup reads one contiguous run of W (16 tiles x 4 KiB in the
    // K-chunk-major layout) and all workgroups together one contiguous range.
    const int ntiles = (a.V + 15) / 16;
    const int T0 = (int)(((int64_t)blockIdx.x * ntiles) / gridDim.x);
    const int T1 = (int)(((int64_t)(blockIdx.x + 1) * ntiles) / gridDim.x);
    constexpr int kTilesPerPass = 2 * kLhCB * kLhWaves;
    const int npass = (T1 - T0 + kTilesPerPass - 1) / kTilesPerPass;
    const int G = npass * nchunks;           // chunks of the walk, the same for every wave

    // tile i (0, 1) of wave w in pass p; past T1 it repeats the workgroup's last tile (L2 hits, results dropped)
    auto tile16 = [&](int p, int i) {
        const int x = T0 + p * kTilesPerPass + 2 * kLhCB * wave + i;
        return x < T1 ? x : T1 - 1;
    };
    auto tile_live = [&](int p, int i) { return T0 + p * kTilesPerPass + 2 * kLhCB * wave + i < T1; };
    auto kchunk = [&](int g) { return g % nchunks; };

    // ---- hidden: chunk c = K blocks [c*KC, (c+1)*KC); LDS block (rb, s) holds the
    // 32x16 A operand of row block rb and K step s in lane order (row l%32, K 16 s + 8 (l/32))
    u32x4 hs[kLhHLoads];
    auto load_hidden = [&](int g) {
        const int c = kchunk(g < G ? g : G - 1);
#pragma unroll
        for (int i = 0; i < kLhHLoads; ++i) {
            const int j = wave * kLhHLoads + i;
            const int rb = j / kLhS, s = j % kLhS;
            const int row = min(row0 + rb * 32 + l32, a.M - 1);
            hs[i] = *reinterpret_cast<const u32x4*>(a.hidden + (int64_t)row * a.ldh + c * (kLhKC * 32) + s * 16 +
                                                    hk * 8);
        }
    };
    auto store_hidden = [&](int g) {
        char* buf = ring[g % kLhRing];
#pragma unroll
        for (int i = 0; i < kLhHLoads; ++i)
            *reinterpret_cast<u32x4*>(buf + (wave * kLhHLoads + i) * 1024 + lane * 16) = hs[i];
    };

    // ---- W: the B operand of column block cb, K step s of chunk g: column 32 cb + l%32
    // of the pass -> tile 2 cb + (l%32)/16, row l%16; K 16 s + 8 (l/32) -> 32-K block
    // c*KC + s/2, lane (l%16) + 16 (2 (s%2) + l/32) of that 1 KiB block, which the
    // K-chunk-major layout keeps at block ((c * ntiles + tile) * KC + s/2)
    auto load_w = [&](int g, WSet& w) {
        const int gg = g < G ? g : G - 1;
        const int p = gg / nchunks, c = kchunk(gg);
#pragma unroll
        for (int cb = 0; cb < kLhCB; ++cb) {
            const int t = tile16(p, 2 * cb + (l32 >> 4));
            const uint16_t* bp = a.W + ((int64_t)c * ntiles + t) * (kLhKC * 512) + ((l32 & 15) + 16 * hk) * 8;
#pragma unroll
            for (int s = 0; s < kLhS; ++s) w[cb][s] = load_bf16x8_nt(bp + (s >> 1) * 512 + (s & 1) * 256);
        }
    };

    f32x16 acc[kLhRB][kLhCB];
#pragma unroll
    for (int rb = 0; rb < kLhRB; ++rb)
#pragma unroll
        for (int cb = 0; cb < kLhCB; ++cb)
#pragma unroll
            for (int j = 0; j < 16; ++j) acc[rb][cb][j] = 0.f;

    // A operands (hidden) read from LDS one K step ahead of their MFMAs.  A wave
    // whose tiles of this pass all lie past the workgroup's range (the tail of
    // the last pass) skips the contraction (wave-uniform branch).
    auto contract = [&](int g, const WSet& w) {
        if (!tile_live(g / nchunks, 0)) return;
        const char* buf = ring[g % kLhRing] + lane * 16;
        bf16x8 hq[2][kLhRB];
#pragma unroll
        for (int rb = 0; rb < kLhRB; ++rb) hq[0][rb] = *reinterpret_cast<const bf16x8*>(buf + rb * kLhS * 1024);
#pragma unroll
        for (int s = 0; s < kLhS; ++s) {
            if (s + 1 < kLhS) {
#pragma unroll
                for (int rb = 0; rb < kLhRB; ++rb)
                    hq[(s + 1) & 1][rb] = *reinterpret_cast<const bf16x8*>(buf + (rb * kLhS + s + 1) * 1024);
            }
#pragma unroll
            for (int rb = 0; rb < kLhRB; ++rb)
#pragma unroll
                for (int cb = 0; cb < kLhCB; ++cb)
                    acc[rb][cb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hq[s & 1][rb], w[cb][s], acc[rb][cb], 0, 0, 0);
        }
    };

    // ---- epilogue of pass p, 16 columns (one tile) at a time through the wave's 4 KiB of LDS
    unsigned long long seen = 0;   // returned key values: makes the maxima returning atomics
    uint16_t* stg = stage[wave];
    auto epilogue = [&](int p) {
#pragma unroll
        for (int cb = 0; cb < kLhCB; ++cb) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int i = 2 * cb + half;          // tile of the pass
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
                            seen |= __hip_atomic_fetch_max(&a.keys[(int64_t)jr * a.key_stride], key, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
            }
        }
    };

    // ---- walk over chunks g = p * nchunks + c: chunk g uses W set g % 2 and
    // hidden buffer g % 2.  At the top of chunk g the hidden loads and the W
    // loads of g+1 are issued (unconditionally: past the walk they reload its
    // last chunk), chunk g is contracted, the hidden of g+1 is written to LDS
    // (its wait leaves the W loads in flight) and the workgroup synchronises.
    // nchunks is even, so both steps of a loop turn belong to one pass; the
    // epilogue of a pass runs between passes.
    WSet wa, wb;
    load_hidden(0);
    store_hidden(0);
    load_w(0, wa);
    __syncthreads();
    auto step = [&](int g, const WSet& cur, WSet& ahead) {
        __builtin_amdgcn_sched_barrier(0);
        load_hidden(g + 1);
        load_w(g + 1, ahead);
        __builtin_amdgcn_sched_barrier(0);
        contract(g, cur);
        store_hidden(g + 1);
        __syncthreads();
    };
    for (int p = 0; p < npass; ++p) {
        for (int c = 0; c < nchunks; c += 2) {
            step(p * nchunks + c, wa, wb);
            step(p * nchunks + c + 1, wb, wa);
        }
        epilogue(p);
    }

    if (a.argmax_period <= 0) return;
    // Using the returned values orders each wave's maxima before the barrier,
    // and so before the workgroup is counted in (the write is never taken).
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

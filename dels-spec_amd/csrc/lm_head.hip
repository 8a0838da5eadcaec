// The target LM head of a draft block, base = hidden . W^T (code/dflash.py:468:
// target.lm_head(parallel_hiddens), bf16 output), with the argmax of chosen
// rows fused into the GEMM so that their logits never reach memory
// (sample(base_logits[:, :1]), code/dflash.py:475).
//
// Shape: M rows of hidden (a draft block's batch x k positions, about a
// hundred) against W [V, K] (K = 4096, V = 151936: 1.245 GB of bf16).  At this
// M the product is bound by streaming W from HBM once (about M FLOP per byte,
// far under the MFMA ridge), and on this GPU by what a CU can pull through its
// L1 from L2 (about 25 GB/s per CU under a streaming load, ~6.5 TB/s over the
// chip): every byte that reaches a CU counts, whether it comes from HBM or
// from L2.  W (4.9 MB per CU) has to arrive once; hidden (1 MB per row group
// of 128) arrives once per pass over a CU's columns.  So a workgroup keeps the
// accumulators of ALL its columns at once -- one pass, hidden staged once per
// CU -- where a pass of 256 columns staged it about three times (805 MB over
// the chip against W's 1.245 GB).
//   * W is packed once (dels_pack_lm_head) into MFMA-16 blocks in
//     K-chunk-major order: the 4 KiB of one 16-row tile in one K chunk
//     (128 K) are contiguous, and so are the tiles of one chunk, so that the
//     whole GPU reads W as one sweep per chunk (DRAM-page friendly).
//   * One workgroup per CU, eight waves (two per SIMD).  The workgroup's
//     16-row vocabulary tiles are dealt to the waves (tile T0 + w + 8j to wave
//     w), at most kLhNT = 5 per wave and pass: 8 row blocks x 5 tiles of 16x16
//     fp32 accumulators = 160 registers.  At V = 151936 over 256 CUs a
//     workgroup has 37-38 tiles, so one pass.
//   * W goes from HBM into LDS by direct-to-LDS loads: one 1 KiB block per
//     tile and K step of 32, already in v_mfma_f32_16x16x32_bf16's operand
//     layout (lane l = vocabulary row l%16, K 8(l/16)..+7), into two step
//     slots private to the wave; the loads of step t+1 are issued before the
//     wait for step t, so one step of loads stays in flight through every
//     wait.  (With the in-flight step in registers instead, 160 accumulators
//     + two register sets left the compiler short of registers at two waves
//     per SIMD: it spilled.)
//   * hidden is staged through LDS by direct-to-LDS loads of whole 128-byte
//     lines: a chunk is 128 rows x 128 K (32 KiB: [64-K half][row][16-byte
//     slot], piece q of a row in slot q ^ (row % 8) so that the operand reads
//     of 16 rows spread over the banks), a ring of two: the barrier that
//     starts chunk g publishes it and frees the buffer of g-1, into which
//     each wave then issues its four loads of chunk g+1.
//   * D = W . hidden^T: lane l ends with hidden row l%16 and vocabulary rows
//     4(l/16)..+3 of the tile, i.e. four consecutive logits of one row: one
//     8-byte store.
// Rows m with argmax_period > 0 and m % argmax_period == 0 are argmax rows:
// their bf16 values enter the argmax (lowest index on ties, the first NaN
// wins, as torch.argmax) as 64-bit keys, reduced over the wave's tiles in
// registers and over the waves by LDS atomic maxima, and are not stored;
// every other row is stored to `base` when it is given.  At the end each
// workgroup merges its row keys into the global ones; the last workgroup to
// finish decodes them and returns keys and counter to zero.
#include <algorithm>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

namespace {

constexpr int kLhWaves = 8;                          // two per SIMD
constexpr int kLhThreads = kLhWaves * 64;
constexpr int kLhRows = 128;                         // rows per row group: 8 blocks of 16
constexpr int kLhRB = kLhRows / 16;
constexpr int kLhNT = 5;                             // 16-row vocabulary tiles per wave and pass
constexpr int kLhTilesPerPass = kLhWaves * kLhNT;
constexpr int kLhKC = kLmHeadKChunk;                 // 32-K blocks (K steps) per chunk
constexpr int kLhChunkBytes = kLhRows * kLhKC * 64;  // 128 rows x 128 K of bf16 = 32 KiB
constexpr int kLhHalfBytes = kLhRows * 128;          // one 64-K half of a chunk: a 128-byte line per row
constexpr int kLhHLoads = kLhChunkBytes / 1024 / kLhWaves;   // direct-to-LDS loads per wave and chunk
constexpr int kLhRing = 2;                           // hidden chunks in LDS: in use, in flight
static_assert(kLhHLoads == kLhKC, "one hidden load per wave and K step");

struct LmHeadArgs {
    const uint16_t* hidden; int64_t ldh;
    const uint16_t* W;                      // [V, K] in MFMA-16 blocks, K-chunk-major
    int M, K, V;
    uint16_t* base; int64_t ldo;            // bf16 output (nullptr: none)
    bool vec_store;                         // base 8-byte aligned and ldo % 4 == 0
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

// Wait until at most N of this wave's vector-memory operations are
// outstanding (its direct-to-LDS loads included, which the compiler does not
// track; they return in issue order).
template <int N>
__device__ __forceinline__ void lh_wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070 | 0x0f00);   // vmcnt(N) only
    asm volatile("" ::: "memory");
}

// Workgroup barrier after this wave's LDS operations are done.
__device__ __forceinline__ void lh_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

struct LmHeadCtx {
    const LmHeadArgs* a;
    char (*ring)[kLhChunkBytes];            // hidden chunks
    char* wslots;                           // this wave's two W step slots
    unsigned long long* s_keys;
    int lane, wave, row0, ntiles, nchunks, G;   // G: chunks of the walk (passes x chunks per pass)
};

// Direct-to-LDS load j (0 .. kLhHLoads-1) of this wave for hidden chunk g
// (K columns [c*128, c*128+128) with c = g % nchunks) into ring buffer g % 2.
// Load i = wave * kLhHLoads + j of the chunk covers half i / 16, rows
// 8 (i % 16) .. +7: lane l fetches row 8 (i % 16) + l/8, the piece that lands
// in slot l % 8.  Rows past M repeat row M-1 (never stored).  Byte offsets fit
// 32 bits (the hidden rows span less than 2 GiB, checked at launch).
__device__ __forceinline__ void lh_issue_hidden(const LmHeadCtx& x, int g, int j) {
    const LmHeadArgs& a = *x.a;
    const int c = g % x.nchunks;
    const int i = x.wave * kLhHLoads + j;
    const int half = i >> 4;
    const int row = 8 * (i & 15) + (x.lane >> 3);
    const int q = (x.lane & 7) ^ (row & 7);
    const int m = min(x.row0 + row, a.M - 1);
    const uint32_t off = (uint32_t)(((int64_t)m * a.ldh + c * (kLhKC * 32) + half * 64 + q * 8) * 2);
    dma16(a.hidden, off, x.ring[g % kLhRing] + i * 1024);
}

// One pass of a wave that owns NT tiles (tile j = tile0 + 8 j), chunks
// [g0, g0 + nchunks) of the walk.  Every load is a direct-to-LDS load that the
// compiler does not track: the waits below count them.
template <int NT>
__device__ __forceinline__ void lh_pass(const LmHeadCtx& x, int g0, int tile0) {
    const LmHeadArgs& a = *x.a;
    const int lane = x.lane, l16 = lane & 15, lq = lane >> 4;

    f32x4 acc[kLhRB][NT > 0 ? NT : 1];
#pragma unroll
    for (int rb = 0; rb < kLhRB; ++rb)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[rb][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // W block of tile j at chunk c, K step s: ((c * ntiles + tile) * KC + s) KiB,
    // copied to KiB j of the step's slot (lane l's 16 bytes at 16 l: the
    // operand layout as it lies in memory).
    auto issue_w = [&](int c, int s, int slot) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint16_t* blk = a.W + ((int64_t)c * x.ntiles + tile0 + 8 * j) * (kLhKC * 512) + s * 512;
            dma16(blk, (uint32_t)lane * 16u, x.wslots + slot * (kLhNT * 1024) + j * 1024);
        }
    };

    // K step s of chunk g with the W blocks of slot `slot`: B operand = 16
    // hidden rows x 32 K from the ring (row 16 rb + l%16, K 32 s + 8 (l/16):
    // half s/2, piece 4 (s%2) + l/16).
    auto contract = [&](int g, int s, int slot) {
        if constexpr (NT > 0) {
            bf16x8 w[NT];
#pragma unroll
            for (int j = 0; j < NT; ++j)
                w[j] = *reinterpret_cast<const bf16x8*>(x.wslots + slot * (kLhNT * 1024) + j * 1024 + lane * 16);
            const char* buf = x.ring[g % kLhRing] + (s >> 1) * kLhHalfBytes;
#pragma unroll
            for (int rb = 0; rb < kLhRB; ++rb) {
                const int row = rb * 16 + l16;
                const int q = (((s & 1) << 2) | lq) ^ (row & 7);
                const bf16x8 hb = *reinterpret_cast<const bf16x8*>(buf + row * 128 + q * 16);
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[rb][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[j], hb, acc[rb][j], 0, 0, 0);
            }
        }
    };

    // Step (g, s): W of the next step into the other slot (whose reads, by the
    // previous step, are done); wait for this step's W -- in issue order, so
    // everything older has landed too (the hidden loads of chunk g among
    // them); at s == 0 the barrier that publishes hidden chunk g and frees the
    // buffer of g-1, and the loads of chunk g+1 into it; then the MFMAs.
    // Younger than this step's W at the wait: the next step's NT loads
    // (unless LAST) and, at s == 1, the kLhHLoads hidden loads of step s == 0.
    auto step = [&](auto last_tag, int g, int s) {
        constexpr bool LAST = decltype(last_tag)::value;
        const int c = g % x.nchunks;
        if constexpr (!LAST) {
            if (s + 1 < kLhKC) issue_w(c, s + 1, (s + 1) & 1);
            else issue_w(c + 1, 0, 0);
        }
        constexpr int N = LAST ? 0 : NT;
        if (s == 1 && g + 1 < x.G) lh_wait_vm<N + kLhHLoads>();
        else lh_wait_vm<N>();
        if (s == 0) {
            lh_barrier();
            if (g + 1 < x.G) {
#pragma unroll
                for (int j = 0; j < kLhHLoads; ++j) lh_issue_hidden(x, g + 1, j);
            }
        }
        contract(g, s, s & 1);
    };

    issue_w(0, 0, 0);
    const int g1 = g0 + x.nchunks - 1;    // last chunk of the pass: its last step prefetches nothing
    for (int g = g0; g < g1; ++g) {
        step(std::false_type{}, g, 0);
        step(std::false_type{}, g, 1);
        step(std::false_type{}, g, 2);
        step(std::false_type{}, g, 3);
    }
    step(std::false_type{}, g1, 0);
    step(std::false_type{}, g1, 1);
    step(std::false_type{}, g1, 2);
    step(std::true_type{}, g1, 3);
    static_assert(kLhKC == 4, "four K steps per chunk, two W slots");

    // Epilogue: lane l holds D[vocabulary 16 tile + 4 (l/16) + e][row 16 rb + l%16].
    // (Its lane and row values pass through empty asm statements here, so that
    // the compiler cannot compute the store addresses before the K loop and
    // hold them in registers across it.)
    if constexpr (NT > 0) {
        const bool any_argmax = a.argmax_period > 0;
        int e16 = l16, eq = lq, erow0 = x.row0;
        asm volatile("" : "+v"(e16), "+v"(eq), "+s"(erow0));
#pragma unroll
        for (int rb = 0; rb < kLhRB; ++rb) {
            const int m = erow0 + rb * 16 + e16;
            const bool argmax_row = any_argmax && m % a.argmax_period == 0;
            unsigned long long key = 0ull;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int v = (tile0 + 8 * j) * 16 + 4 * eq;
                float r[4];
                uint32_t bits[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    bits[e] = f32_to_bf16_bits(acc[rb][j][e]);
                    r[e] = bf16_bits_to_f32(bits[e]);
                }
                if (argmax_row) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const unsigned long long k = v + e < a.V ? lh_key(r[e], (uint32_t)(v + e)) : 0ull;
                        key = k > key ? k : key;
                    }
                } else if (a.base != nullptr && m < a.M) {
                    uint16_t* dst = a.base + (int64_t)m * a.ldo + v;
                    if (a.vec_store && v + 4 <= a.V) {
                        *reinterpret_cast<u32x2*>(dst) = u32x2{bits[0] | (bits[1] << 16), bits[2] | (bits[3] << 16)};
                    } else {
                        for (int e = 0; e < 4 && v + e < a.V; ++e) dst[e] = (uint16_t)bits[e];
                    }
                }
            }
            if (any_argmax) {
                // over the four lanes that hold row m (l/16 = 0..3), then one LDS maximum per row
                key = max(key, lh_shfl_xor(key, 16));
                key = max(key, lh_shfl_xor(key, 32));
                if (eq == 0 && argmax_row && m < a.M && key != 0ull)
                    __hip_atomic_fetch_max(&x.s_keys[rb * 16 + e16], key, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
    }
}

__global__ __launch_bounds__(kLhThreads) void lm_head_kernel(LmHeadArgs a) {
    __shared__ __attribute__((aligned(1024))) char ring[kLhRing][kLhChunkBytes];
    __shared__ __attribute__((aligned(1024))) char wbuf[kLhWaves][2 * kLhNT * 1024];
    __shared__ int s_last;
    __shared__ unsigned long long s_keys[kLhRows];   // argmax keys of the workgroup's rows

    LmHeadCtx x;
    x.a = &a;
    x.ring = ring;
    x.s_keys = s_keys;
    x.wslots = wbuf[__builtin_amdgcn_readfirstlane(threadIdx.x >> 6)];
    x.lane = threadIdx.x & 63;
    x.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    x.row0 = blockIdx.y * kLhRows;
    x.ntiles = (a.V + 15) / 16;
    x.nchunks = a.K / (kLhKC * 32);

    // 16-row vocabulary tiles [T0, T1) of this workgroup, up to 40 per pass:
    // in pass p wave w owns tiles T0 + 40 p + w + 8 j.
    const int T0 = (int)(((int64_t)blockIdx.x * x.ntiles) / gridDim.x);
    const int T1 = (int)(((int64_t)(blockIdx.x + 1) * x.ntiles) / gridDim.x);
    const int npass = (T1 - T0 + kLhTilesPerPass - 1) / kLhTilesPerPass;
    x.G = npass * x.nchunks;

    for (int r = threadIdx.x; r < kLhRows; r += kLhThreads) s_keys[r] = 0ull;   // published by the first barrier
    // hidden chunk 0 (chunk g+1 is issued at the start of chunk g)
#pragma unroll
    for (int j = 0; j < kLhHLoads; ++j) lh_issue_hidden(x, 0, j);

    for (int p = 0; p < npass; ++p) {
        const int first = T0 + p * kLhTilesPerPass;
        const int n = min(kLhTilesPerPass, T1 - first);
        const int nt = n > x.wave ? min(kLhNT, (n - x.wave + kLhWaves - 1) / kLhWaves) : 0;   // wave-uniform
        const int tile0 = first + x.wave;
        const int g0 = p * x.nchunks;
        switch (nt) {
            case 5: lh_pass<5>(x, g0, tile0); break;
            case 4: lh_pass<4>(x, g0, tile0); break;
            case 3: lh_pass<3>(x, g0, tile0); break;
            case 2: lh_pass<2>(x, g0, tile0); break;
            case 1: lh_pass<1>(x, g0, tile0); break;
            default: lh_pass<0>(x, g0, tile0); break;
        }
    }
    static_assert(kLhNT == 5, "the switch covers 0 .. kLhNT tiles");
    // every direct-to-LDS write has landed before the workgroup's LDS is reused or released
    __builtin_amdgcn_s_waitcnt(0x0070 | (0xf << 8));   // vmcnt(0)

    if (a.argmax_period <= 0) return;
    __syncthreads();   // every wave's LDS maxima are in s_keys
    unsigned long long seen = 0;
    for (int r = threadIdx.x; r < kLhRows; r += kLhThreads) {
        const int m = x.row0 + r;
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
    if (K < 1 || K >= (int64_t(1) << 26) || K % 256 != 0) return false;
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
    a.vec_store = (reinterpret_cast<uintptr_t>(base) & 7) == 0 && ldo % 4 == 0;
    a.argmax_period = argmax_period;
    a.out_ids = out_ids; a.out_score = out_score; a.ld_out = ld_out;
    a.counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
    a.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    const int nrows = argmax_period > 0 ? (M + argmax_period - 1) / argmax_period : 0;
    a.key_stride = (int64_t)nrows * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
    const int groups = (M + kLhRows - 1) / kLhRows;
    const int ntiles = (V + 15) / 16;
    // one workgroup per CU, at least two tiles per wave where the vocabulary allows
    const int gx = std::max(1, std::min((ntiles + 2 * kLhWaves - 1) / (2 * kLhWaves),
                                        std::max(1, device_cu_count() / groups)));
    hipLaunchKernelGGL(lm_head_kernel, dim3(gx, groups, 1), dim3(kLhThreads), 0, s, a);
    return hipGetLastError();
}

}  // namespace dels

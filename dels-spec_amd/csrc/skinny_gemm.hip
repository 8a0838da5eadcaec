// Skinny bf16 GEMM on gfx950 MFMA: C[M, N] = X[M, K] . W[N, K]^T with few rows.
//
// Used for the rank projection rank = bf16(act(bf16(h . A^T + bias)))
// (code/kernel/dels.py:437-443) and, with three gate tiles per column tile and
// a fused gate epilogue, for the GRU step gh = bf16(h . W_hh^T + b_hh) followed
// by the (r, z, n) gates (code/kernel/dels.py:140-211, 359-373).
//
// Work decomposition: a workgroup (4 wave64s) owns a (16*WM) x (16*WN) output
// tile and a slice of K; its waves interleave over the slice's 32-wide K
// steps with v_mfma_f32_16x16x32_bf16 (operands loaded straight from global
// memory in MFMA layout: lane l reads 16 bytes of row l%16 at k-group l/16).
// Waves are summed through LDS in a fixed order.  When K is split across
// KSPLIT workgroups, each writes its fp32 partial tile to the workspace and the
// last one to arrive (atomic counter) sums all partials in split order -- so
// the result is deterministic -- runs the epilogue and resets the counter.
#include <algorithm>

#include "dels_device.h"
#include "fp8.h"
#include "dels_internal.h"

namespace dels {

enum : int { EPI_RANK = 0, EPI_GRU = 1 };

constexpr int kMaxKSplit = 16;   // workgroups per output tile along K (loads unrolled to this)

struct SkinnyKArgs {
    const uint16_t* x; int64_t ldx;     // [M, K]; NULL means an all-zero X (GRU zero state)
    const uint16_t* w; int64_t ldw;     // [wrows, K] row-major, or blocks of 16 rows x 32 K (WMODE)
    int M, K, wrows;
    int ncols;                          // output columns (N for rank, G for GRU)
    int ksteps, ksplit;
    float* partial;                     // [ksplit][m_wg][n_wg][WM*WN*256]
    unsigned int* counters;             // [m_wg][n_wg]
    // rank epilogue
    const float* col_scale;             // e4m3 W only: per-column scale, applied before the bias
    const uint16_t* bias; int act;
    uint16_t* out; int64_t ldout;
    uint8_t* out_q; float* out_qscale;  // split-K rank epilogue: also e4m3 per row (rank_proj_quantizes)
    // GRU epilogue
    const uint16_t* gi_table; int64_t ld_gi; int64_t table_rows;
    const int64_t* tokens; int64_t tok_stride;
};

// Column (row of W) of gate/sub-tile j for a workgroup whose first column is c0.
template <int EPI>
__device__ __forceinline__ int wcol(int c0, int j, int ncols) {
    return EPI == EPI_GRU ? c0 + j * ncols : c0 + j * 16;
}

template <int WM, int WN, int EPI>
__device__ __forceinline__ void skinny_epilogue(const SkinnyKArgs& a, const float* vals,
                                                int m0, int c0) {
#pragma clang fp contract(off)
    constexpr int T = WM * WN;
    (void)T;
    if constexpr (EPI == EPI_RANK) {
        // vals: [WM][WN][64 lanes][4]
        for (int e = threadIdx.x; e < WM * WN * 256; e += blockDim.x) {
            const int q = e & 3, lane = (e >> 2) & 63, t = e >> 8;
            const int i = t / WN, j = t % WN;
            const int m = m0 + i * 16 + 4 * (lane >> 4) + q;
            const int n = c0 + j * 16 + (lane & 15);
            if (m < a.M && n < a.ncols) {
                float v = vals[e];
                if (a.col_scale) v = v * a.col_scale[n];
                if (a.bias) v = v + bf16_bits_to_f32(a.bias[n]);
                v = round_bf16(v);
                if (a.act == 1) v = round_bf16(silu_f32(v));
                a.out[(int64_t)m * a.ldout + n] = f32_to_bf16_bits(v);
            }
        }
    } else {
        // GRU: WN == 3 gate tiles (r, z, n) sharing one lane layout.
        const int G = a.ncols;
        for (int e = threadIdx.x; e < WM * 256; e += blockDim.x) {
            const int q = e & 3, lane = (e >> 2) & 63, i = e >> 8;
            const int b = m0 + i * 16 + 4 * (lane >> 4) + q;
            const int g = c0 + (lane & 15);
            if (b >= a.M || g >= G) continue;
            const int base_e = (i * WN) * 256 + lane * 4 + q;
            float ghr = vals[base_e], ghz = vals[base_e + 256], ghn = vals[base_e + 512];
            if (a.bias) {
                ghr = ghr + bf16_bits_to_f32(a.bias[g]);
                ghz = ghz + bf16_bits_to_f32(a.bias[G + g]);
                ghn = ghn + bf16_bits_to_f32(a.bias[2 * G + g]);
            }
            ghr = round_bf16(ghr);
            ghz = round_bf16(ghz);
            ghn = round_bf16(ghn);
            int64_t tok = a.tokens[(int64_t)b * a.tok_stride];
            tok = tok < 0 ? 0 : (tok >= a.table_rows ? a.table_rows - 1 : tok);
            const uint16_t* gi = a.gi_table + tok * a.ld_gi;
            const float gir = bf16_bits_to_f32(gi[g]);
            const float giz = bf16_bits_to_f32(gi[G + g]);
            const float gin = bf16_bits_to_f32(gi[2 * G + g]);
            const float hp = a.x ? bf16_bits_to_f32(a.x[(int64_t)b * a.ldx + g]) : 0.0f;
            a.out[(int64_t)b * a.ldout + g] = f32_to_bf16_bits(gru_unit(gir, giz, gin, ghr, ghz, ghn, hp));
        }
    }
}

// How W is stored: row-major bf16, MFMA-16 bf16 blocks (zero-padded, so no
// masking and every operand load is one contiguous KiB per wave), or e4m3 in
// the same block order (512-byte blocks, widened to bf16 at use).
enum : int { W_ROWMAJOR = 0, W_PACKED = 1, W_PACKED_E4M3 = 2 };

template <int WM, int WN, int EPI, int WMODE>
__global__ __launch_bounds__(256) void skinny_gemm_kernel(SkinnyKArgs a) {
    constexpr int T = WM * WN;
    __shared__ float red[2 * T * 256];
    __shared__ int s_last;

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int lrow = lane & 15;        // row within a 16-row operand tile
    const int kg = lane >> 4;          // k-group (8 elements) within a 32-wide step
    const int m0 = blockIdx.y * (16 * WM);
    const int c0 = blockIdx.x * (EPI == EPI_GRU ? 16 : 16 * WN);
    const int z = blockIdx.z;

    f32x4 acc[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    if (a.x != nullptr) {
        const int sps = (a.ksteps + a.ksplit - 1) / a.ksplit;
        const int ks0 = z * sps;
        const int ks1 = min(a.ksteps, ks0 + sps);
        // Row pointers, clamped in range; out-of-range rows load zeros.
        const uint16_t* xp[WM];
        bool xok[WM];
#pragma unroll
        for (int i = 0; i < WM; ++i) {
            const int m = m0 + i * 16 + lrow;
            xok[i] = m < a.M;
            xp[i] = a.x + (int64_t)(xok[i] ? m : 0) * a.ldx + kg * 8;
        }
        const uint16_t* wp[WN];
        bool wok[WN];
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int c = wcol<EPI>(c0, j, a.ncols);   // first W row of sub-tile j (a multiple of 16)
            if constexpr (WMODE == W_PACKED) {
                wok[j] = true;
                wp[j] = a.w + ((int64_t)(c >> 4) * a.ksteps) * 512 + lane * 8;
            } else if constexpr (WMODE == W_PACKED_E4M3) {
                wok[j] = true;   // byte offset, in 16-bit units: 256 per block, 4 per lane
                wp[j] = a.w + ((int64_t)(c >> 4) * a.ksteps) * 256 + lane * 4;
            } else {
                const int n = c + lrow;
                wok[j] = (n - (EPI == EPI_GRU ? j * a.ncols : 0)) < a.ncols && n < a.wrows;
                wp[j] = a.w + (int64_t)(wok[j] ? n : 0) * a.ldw + kg * 8;
            }
        }
        // Wave w takes K steps ks0 + w + 4*it.  Operands are prefetched D
        // iterations ahead in a register ring; every load is unconditional
        // (clamped address; the data is masked when used), so the loop body is
        // branch-free and each wait covers only the slot about to be used.
        // Iterations past the wave's range contribute exact zeros.
        constexpr int D = (WM + WN) <= 2 ? 8 : ((WM + WN) <= 4 ? 4 : 3);
        const int n_iter = (ks1 - ks0 + 3) / 4;
        const int s_fallback = min(ks0, a.ksteps - 1);
        // Raw operand loads of iteration `it` (masks are applied at use, so no
        // instruction needs the data before its MFMA).
        auto load_iter = [&](int it, u32x4 (&xv)[WM], u32x4 (&wv)[WN]) {
            const int s_raw = ks0 + wave + 4 * it;
            const bool sok = s_raw < ks1;
            const int s = sok ? s_raw : s_fallback;
            const int k = s * 32;
            const bool kok = sok && (k + kg * 8) < a.K;
#pragma unroll
            for (int i = 0; i < WM; ++i) xv[i] = *reinterpret_cast<const u32x4*>(xp[i] + (kok ? k : 0));
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                if constexpr (WMODE == W_PACKED && EPI == EPI_GRU) {
                    // cached: a rollout re-reads W_hh every step (14-step rollout
                    // at G = 512: 379 -> 362 us against non-temporal loads)
                    wv[j] = *reinterpret_cast<const u32x4*>(wp[j] + (int64_t)s * 512);
                } else if constexpr (WMODE == W_PACKED) {
                    wv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp[j] + (int64_t)s * 512));
                } else if constexpr (WMODE == W_PACKED_E4M3) {
                    const u32x2 q = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(wp[j] + (int64_t)s * 256));
                    wv[j] = u32x4{q[0], q[1], 0u, 0u};
                } else
                    wv[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wp[j] + (kok ? k : 0)));
            }
        };
        auto mma_iter = [&](int it, const u32x4 (&xv)[WM], const u32x4 (&wv)[WN]) {
            const int s_raw = ks0 + wave + 4 * it;
            const bool sok = s_raw < ks1;
            const bool kok = sok && (s_raw * 32 + kg * 8) < a.K;
            bf16x8 xo[WM], wo[WN];
#pragma unroll
            for (int i = 0; i < WM; ++i) xo[i] = masked_bf16x8(xv[i], (kok && xok[i]) ? 0xffffffffu : 0u);
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                if constexpr (WMODE == W_PACKED)
                    wo[j] = masked_bf16x8(wv[j], sok ? 0xffffffffu : 0u);
                else if constexpr (WMODE == W_PACKED_E4M3)
                    wo[j] = masked_bf16x8(widen_e4m3x8(wv[j][0], wv[j][1]), sok ? 0xffffffffu : 0u);
                else
                    wo[j] = masked_bf16x8(wv[j], (kok && wok[j]) ? 0xffffffffu : 0u);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i)
#pragma unroll
                for (int j = 0; j < WN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xo[i], wo[j], acc[i][j], 0, 0, 0);
        };
        u32x4 rx[D][WM], rw[D][WN];
#pragma unroll
        for (int u = 0; u < D; ++u) load_iter(u, rx[u], rw[u]);
        for (int it0 = 0; it0 < n_iter; it0 += D) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                mma_iter(it0 + u, rx[u], rw[u]);
                load_iter(it0 + u + D, rx[u], rw[u]);
            }
        }
    }

    // Sum the four waves through LDS in a fixed order: (w0 + w2) + (w1 + w3).
    if (wave >= 2) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                *reinterpret_cast<f32x4*>(&red[(((wave - 2) * T) + i * WN + j) * 256 + lane * 4]) = acc[i][j];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                acc[i][j] += *reinterpret_cast<const f32x4*>(&red[((wave * T) + i * WN + j) * 256 + lane * 4]);
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j)
                *reinterpret_cast<f32x4*>(&red[(i * WN + j) * 256 + lane * 4]) = acc[i][j];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < WM; ++i)
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                f32x4* p = reinterpret_cast<f32x4*>(&red[(i * WN + j) * 256 + lane * 4]);
                *p = acc[i][j] + *p;
            }
    }
    __syncthreads();

    if (a.ksplit == 1) {
        skinny_epilogue<WM, WN, EPI>(a, red, m0, c0);
        return;
    }

    // Split K: publish the partial tile, the last workgroup reduces.  No cache
    // fences: the partials are written and read with device-scope (coherent)
    // atomic stores/loads, every store is waited for before the one counter
    // read-modify-write, and the summation runs in split order, so the result
    // does not depend on which workgroup arrives last.
    const int tile_id = blockIdx.y * gridDim.x + blockIdx.x;
    const int ntile = gridDim.x * gridDim.y;
    float* mine = a.partial + ((int64_t)z * ntile + tile_id) * (T * 256);
    for (int e = threadIdx.x; e < T * 256; e += blockDim.x)
        __hip_atomic_store(mine + e, red[e], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);   // the stores above have reached device coherence
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned prev = __hip_atomic_fetch_add(&a.counters[tile_id], 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (unsigned)(a.ksplit - 1));
    }
    __syncthreads();
    if (!s_last) return;
    for (int e = threadIdx.x; e < T * 256; e += blockDim.x) {
        // all split loads in flight at once, then the sum in split order
        float p[kMaxKSplit];
#pragma unroll
        for (int zz = 0; zz < kMaxKSplit; ++zz)
            p[zz] = zz < a.ksplit ? __hip_atomic_load(a.partial + ((int64_t)zz * ntile + tile_id) * (T * 256) + e,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                  : 0.f;
        float v = 0.f;
#pragma unroll
        for (int zz = 0; zz < kMaxKSplit; ++zz) v += p[zz];
        red[e] = v;
    }
    if (threadIdx.x == 0)
        __hip_atomic_exchange(&a.counters[tile_id], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    skinny_epilogue<WM, WN, EPI>(a, red, m0, c0);
}

// ---------------------------------------------------------------------------
// Many rows (M >= 64): an LDS-tiled rank projection.
//
// The skinny kernel reads its operands straight from global memory, each
// wave's load touching 32 B of 32 different rows; at M = 512 that re-reads h
// and A sixteen times over through the caches and is latency bound (16 us at
// the Qwen3-8B shape).  Here a workgroup owns a TM x TN output tile and a
// range of 64-deep K chunks.  Each chunk's slices of h (TM rows) and of A (TN
// rows) are copied HBM -> LDS with direct-to-LDS loads of whole 128-byte
// lines (eight rows per instruction), into a ring of kRgStages chunk
// buffers, so that kRgStages - 1 chunks of loads are in flight; each of its
// (TM/32)(TN/32) waves contracts one 32 x 32 quadrant with
// v_mfma_f32_32x32x16_bf16 from LDS.  The 16-byte pieces of a row are stored
// XOR-swizzled by row (piece q of row r in slot q ^ (r % 8)), so the operand
// reads of 32 rows spread over all LDS banks.
// What bounds it is what the CUs pull from L2 (about 25 GB/s per CU under
// load): each workgroup pulls (TM + TN) x its K range of operand bytes, so
// bigger tiles pull less in total -- (M N K)(1/TM + 1/TN) -- but leave fewer
// tiles, so K is split over more workgroups (ksplit) to cover the device and
// the fp32 partials grow (ksplit x M x N x 4 bytes, written here, read by the
// epilogue kernel).  The plan picks the shape.  The partials go to the
// workspace with plain stores and a second kernel sums them in split order
// (deterministic) and runs the epilogue.
// Needs K % 64 == 0 and r % 8 == 0 (the plan falls back to the skinny kernel otherwise).
// ---------------------------------------------------------------------------

constexpr int kRgChunk = 64;                // K per LDS chunk
constexpr int kRgStages = 4;                // chunk buffers in the LDS ring

// Direct-to-LDS loads per wave and chunk: h (TM/8 instructions of 8 rows) and
// A (row-major: TN/8 like h; MFMA-16 blocks: TN/8 of 1 KiB; e4m3 blocks:
// TN/4 of 256 B), spread over the (TM/32)(TN/32) waves.
template <int WMODE, int TM, int TN>
constexpr int rg_loads_per_wave() {
    return (TM / 8 + (WMODE == W_PACKED_E4M3 ? TN / 4 : TN / 8)) / ((TM / 32) * (TN / 32));
}
template <int TM, int TN>
constexpr int rg_threads() { return (TM / 32) * (TN / 32) * 64; }

template <int N>
__device__ __forceinline__ void rg_wait_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt out of range");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);   // vmcnt(N), lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int WMODE, int TM, int TN>
__global__ __launch_bounds__((TM / 32) * (TN / 32) * 64) void rank_gemm_tiled_kernel(SkinnyKArgs a) {
    constexpr int kThreads = rg_threads<TM, TN>();
    constexpr int kWaves = kThreads / 64;
    constexpr int kHLoads = TM / 8;
    constexpr int kWLoads = WMODE == W_PACKED_E4M3 ? TN / 4 : TN / 8;
    constexpr int L = rg_loads_per_wave<WMODE, TM, TN>();
    static_assert(L * kWaves == kHLoads + kWLoads, "loads must spread evenly over the waves");
    constexpr int kWBytes = WMODE == W_PACKED_E4M3 ? TN * 64 : TN * 128;
    struct __attribute__((aligned(1024))) Chunk {
        char h[TM * 128];    // TM rows x 128 B, pieces swizzled
        char w[kWBytes];     // row-major: as h; blocked: (TN/16) row blocks x 2 K blocks
    };
    __shared__ Chunk ring[kRgStages];
    // the output tile (pitch TN + 4 floats) reuses the ring once the K loop is done
    static_assert(sizeof(Chunk) * kRgStages >= TM * (TN + 4) * sizeof(float), "ring too small");
    float* red = reinterpret_cast<float*>(&ring[0]);

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / (TN / 32), wn = wave % (TN / 32);    // quadrant of this wave
    // Grid (ksplit, column tiles, row tiles): consecutive workgroups -- which
    // the dispatcher deals round-robin over the 8 XCDs -- take different K
    // splits, so each XCD works on ksplit/8 K slices of h and A and its L2
    // fetches those slices once instead of all of h and A.
    const int z = blockIdx.x;
    const int n0 = blockIdx.y * TN, m0 = blockIdx.z * TM;
    const int nchunks = a.K / kRgChunk;
    const int cps = (nchunks + a.ksplit - 1) / a.ksplit;
    const int c0 = z * cps, c1 = min(nchunks, c0 + cps);
    const int nch = max(0, c1 - c0);

    // Load instruction g (0 .. kHLoads + kWLoads - 1) of chunk c into slot S:
    // g < kHLoads is h (rows 8g .. 8g+7), the rest A.  Rows past M or r repeat
    // the last row (their results are never stored).  Byte offsets are taken
    // from the tile's first row (or row block), so they stay far below 2^32
    // whatever the matrix size.
    const int prow = lane >> 3, piece = lane & 7;
    const uint16_t* hbase = a.x + (int64_t)m0 * a.ldx;
    const int nbw = (n0 >> 4);   // first row block of A (blocked layouts)
    const uint16_t* wbase = WMODE == W_ROWMAJOR ? a.w + (int64_t)n0 * a.ldw
                          : a.w + (int64_t)nbw * a.ksteps * (WMODE == W_PACKED ? 512 : 256);
    const int nbl = (a.wrows + 15) / 16 - 1 - nbw;   // last row block, relative to nbw
    auto issue = [&](int c, Chunk& S, int g) {
        const int k0 = c * kRgChunk;
        if (g < kHLoads) {
            const int row = 8 * g + prow;
            const int mr = min(m0 + row, a.M - 1) - m0;
            const int q = piece ^ (row & 7);   // the piece this lane fetches: slot `piece` holds piece q
            dma16(hbase, (uint32_t)(mr * a.ldx + k0 + 8 * q) * 2u, S.h + g * 1024);
        } else if constexpr (WMODE == W_ROWMAJOR) {
            const int row = 8 * (g - kHLoads) + prow;
            const int nr = min(n0 + row, a.wrows - 1) - n0;
            const int q = piece ^ (row & 7);
            dma16(wbase, (uint32_t)(nr * a.ldw + k0 + 8 * q) * 2u, S.w + (g - kHLoads) * 1024);
        } else if constexpr (WMODE == W_PACKED) {
            const int b = g - kHLoads;                // block (row block b/2, K block b%2)
            const int blk = min(b >> 1, nbl) * a.ksteps + (k0 >> 5) + (b & 1);
            dma16(wbase, (uint32_t)(blk * 1024 + lane * 16), S.w + b * 1024);
        } else {
            const int b = (g - kHLoads) >> 1, half = (g - kHLoads) & 1;   // 512-byte e4m3 blocks, two halves
            const int blk = min(b >> 1, nbl) * a.ksteps + (k0 >> 5) + (b & 1);
            dma4(wbase, (uint32_t)(blk * 512 + half * 256 + lane * 4), S.w + b * 512 + half * 256);
        }
    };
    auto issue_chunk = [&](int c, Chunk& S) {
#pragma unroll
        for (int j = 0; j < L; ++j) issue(c, S, wave * L + j);
    };

    // v_mfma_f32_32x32x16_bf16 with the h quadrant as the A operand (lane l:
    // row l%32, K 8*(l/32) .. +7 of the step) and the W quadrant as the B
    // operand: lane l ends with columns n = l%32 and rows 8*(i/4) + 4*(l/32) + i%4.
    const int rl = lane & 31, kh = lane >> 5;
    auto contract = [&](const Chunk& S, f32x16& acc) {
        const int hr = 32 * wm + rl, wr = 32 * wn + rl;
#pragma unroll
        for (int s = 0; s < kRgChunk / 16; ++s) {
            const int q = 2 * s + kh;   // 16-byte piece of the row
            const bf16x8 av = *reinterpret_cast<const bf16x8*>(S.h + hr * 128 + ((q ^ (hr & 7)) << 4));
            bf16x8 bv;
            if constexpr (WMODE == W_ROWMAJOR) {
                bv = *reinterpret_cast<const bf16x8*>(S.w + wr * 128 + ((q ^ (wr & 7)) << 4));
            } else if constexpr (WMODE == W_PACKED) {
                const int b = (wr >> 4) * 2 + (s >> 1);
                bv = *reinterpret_cast<const bf16x8*>(S.w + b * 1024 + ((wr & 15) + 16 * (2 * (s & 1) + kh)) * 16);
            } else {
                const int b = (wr >> 4) * 2 + (s >> 1);
                const u32x2 e = *reinterpret_cast<const u32x2*>(S.w + b * 512 + ((wr & 15) + 16 * (2 * (s & 1) + kh)) * 8);
                bv = __builtin_bit_cast(bf16x8, widen_e4m3x8(e[0], e[1]));
            }
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
        }
    };

    f32x16 acc;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.f;
    // Ring: chunks 0 .. kRgStages-2 issued up front; at chunk i each wave waits
    // for its own loads of i (younger chunks stay in flight), the barrier
    // publishes i and frees the slot of i-1, which takes chunk i + kRgStages-1.
    constexpr int P = kRgStages - 1;
#pragma unroll
    for (int i = 0; i < P; ++i)
        if (i < nch) issue_chunk(c0 + i, ring[i]);
    for (int i0 = 0; i0 < nch; i0 += kRgStages) {
#pragma unroll
        for (int u = 0; u < kRgStages; ++u) {
            const int i = i0 + u;
            if (i >= nch) break;
            const int younger = min(P - 1, nch - 1 - i);   // chunks issued after i, in flight
            static_assert(kRgStages <= 4, "the wait switch covers up to 2 younger chunks");
            switch (younger) {
                case 2: rg_wait_barrier<2 * L>(); break;
                case 1: rg_wait_barrier<1 * L>(); break;
                default: rg_wait_barrier<0>(); break;
            }
            if (i + P < nch) issue_chunk(c0 + i + P, ring[(u + P) % kRgStages]);
            contract(ring[u], acc);
        }
    }

    // the quadrant into the tile red[m][n] (pitch TN + 4 floats)
    constexpr int kPitch = TN + 4;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = 32 * wm + 8 * (i >> 2) + 4 * kh + (i & 3);
        red[m * kPitch + 32 * wn + rl] = acc[i];
    }
    __syncthreads();

    if (a.ksplit > 1) {
        // Split K: the fp32 partial tile goes to partial[z][M][ncols] with plain
        // stores; rank_splitk_epilogue_kernel, launched next on the same
        // stream, sums the splits in order (the kernel boundary makes every
        // partial visible to it) and runs the epilogue.
        float* mine = a.partial + (int64_t)z * a.M * a.ncols;
        for (int e = tid; e < TM * TN / 4; e += kThreads) {
            const int mm = e / (TN / 4), nn = 4 * (e % (TN / 4));
            const int m = m0 + mm, n = n0 + nn;
            if (m >= a.M || n >= a.ncols) continue;
            const float* src = &red[mm * kPitch + nn];
            // ncols is a multiple of 8, so the 4 columns are in range
            *reinterpret_cast<f32x4*>(mine + (int64_t)m * a.ncols + n) = f32x4{src[0], src[1], src[2], src[3]};
        }
        return;
    }

    // Epilogue: rank = bf16(act(bf16(v * col_scale + bias))), two columns per store.
    {
#pragma clang fp contract(off)
        for (int e = tid; e < TM * TN / 2; e += kThreads) {
            const int mm = e / (TN / 2), nn = 2 * (e % (TN / 2));
            const int m = m0 + mm, n = n0 + nn;
            if (m >= a.M || n >= a.ncols) continue;
            uint32_t packed = 0;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                float v = red[mm * kPitch + nn + t];
                if (a.col_scale) v = v * a.col_scale[n + t];
                if (a.bias) v = v + bf16_bits_to_f32(a.bias[n + t]);
                v = round_bf16(v);
                if (a.act == 1) v = round_bf16(silu_f32(v));
                packed |= (uint32_t)f32_to_bf16_bits(v) << (16 * t);
            }
            // ncols is a multiple of 8, so both columns are in range
            uint16_t* dst = a.out + (int64_t)m * a.ldout + n;
            if ((((uintptr_t)a.out & 3) | (uintptr_t)(a.ldout & 1)) == 0) {
                *reinterpret_cast<uint32_t*>(dst) = packed;
            } else {   // an output view without 4-byte rows: element stores
                dst[0] = (uint16_t)packed;
                dst[1] = (uint16_t)(packed >> 16);
            }
        }
    }
}

// Sum of the split-K partials of the LDS-tiled rank projection, in split
// order, and the rank epilogue; one thread per 4 output columns (16-byte loads).
// Q: the rank is also quantised per row to e4m3 with the rule of the e4m3
// argmax's own quantisation (amax = max |rank[m, :]| of the bf16 values,
// q = e4m3(rank * (448 / amax)), scale = amax / 448; 1 for an all-zero row):
// r = 256 or 512, so a workgroup holds whole rows (one or two waves each).
template <bool Q>
__global__ __launch_bounds__(256) void rank_splitk_epilogue_kernel(SkinnyKArgs a) {
#pragma clang fp contract(off)
    const int64_t quads = (int64_t)a.M * a.ncols / 4;
    int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (!Q && t >= quads) return;
    const bool valid = t < quads;
    if (!valid) t = quads - 1;   // Q: every thread reaches the barrier; its row is not written
    const int m = (int)(t / (a.ncols / 4)), n = (int)(t % (a.ncols / 4)) * 4;
    const int64_t off = (int64_t)m * a.ncols + n;
    const int64_t zs = (int64_t)a.M * a.ncols;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    for (int z0 = 0; z0 < a.ksplit; z0 += 8) {
        f32x4 pv[8];
#pragma unroll
        for (int zz = 0; zz < 8; ++zz)   // unconditional loads (clamped split), masked in the sum
            pv[zz] = *reinterpret_cast<const f32x4*>(a.partial + min(z0 + zz, a.ksplit - 1) * zs + off);
#pragma unroll
        for (int zz = 0; zz < 8; ++zz) {
            const bool ok = z0 + zz < a.ksplit;
#pragma unroll
            for (int q = 0; q < 4; ++q) v[q] = ok ? v[q] + pv[zz][q] : v[q];
        }
    }
    uint32_t packed[2] = {0u, 0u};
    float xs[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        float x = v[q];
        if (a.col_scale) x = x * a.col_scale[n + q];
        if (a.bias) x = x + bf16_bits_to_f32(a.bias[n + q]);
        x = round_bf16(x);
        if (a.act == 1) x = round_bf16(silu_f32(x));
        xs[q] = x;   // the bf16 value itself
        packed[q >> 1] |= (uint32_t)f32_to_bf16_bits(x) << (16 * (q & 1));
    }
    uint16_t* dst = a.out + (int64_t)m * a.ldout + n;
    if (valid) {
        if ((((uintptr_t)a.out & 7) | (uintptr_t)(a.ldout & 3)) == 0) {
            *reinterpret_cast<u32x2*>(dst) = u32x2{packed[0], packed[1]};
        } else {   // an output view without 8-byte rows: element stores
            dst[0] = (uint16_t)packed[0]; dst[1] = (uint16_t)(packed[0] >> 16);
            dst[2] = (uint16_t)packed[1]; dst[3] = (uint16_t)(packed[1] >> 16);
        }
    }
    if constexpr (Q) {
        // row maximum of |rank|: the wave's 64 lanes, then the row's two waves at r = 512
        __shared__ float s_amax[4];
        float amax = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) amax = __builtin_fmaxf(amax, __builtin_fabsf(xs[q]));
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, off, 64));
        const int wave = threadIdx.x >> 6;
        if ((threadIdx.x & 63) == 0) s_amax[wave] = amax;
        __syncthreads();
        if (a.ncols == 512) amax = __builtin_fmaxf(s_amax[wave], s_amax[wave ^ 1]);
        const float inv = amax > 0.f ? kE4M3Max / amax : 1.f;
        const uint32_t qw = f32x4_to_e4m3(xs[0] * inv, xs[1] * inv, xs[2] * inv, xs[3] * inv);
        if (valid) {
            *reinterpret_cast<uint32_t*>(a.out_q + (int64_t)m * a.ncols + n) = qw;
            if (n == 0) a.out_qscale[m] = amax > 0.f ? amax / kE4M3Max : 1.f;
        }
    }
}

bool rank_proj_quantizes(const SkinnyPlan& p, int64_t r) { return p.tiled && p.ksplit > 1 && (r == 256 || r == 512); }

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------

static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

SkinnyPlan plan_skinny(int64_t rows, int64_t K, int64_t cols, bool gru) {
    SkinnyPlan p{};
    if (!gru && rows >= kRankTiledMinRows && K % kRgChunk == 0 && cols % 8 == 0) {
        // LDS-tiled kernel.  Tiles of 128 rows x 64 columns from 256 rows on
        // (64 x 64 below, where a 128-row tile would be mostly empty), K split
        // 8 ways unless the tiles alone fill the device, never below two chunks
        // per split.  At M = 512, r = 512, d = 4096 the shapes measured (GEMM
        // kernel, rocprof average): 64x64 / 8 splits 9.45 us, 128x64 / 8 8.89,
        // 128x128 / 16 10.44 (twice the partials), with the split-K epilogue
        // 4.9-5.2 us in each case.
        p.tiled = true;
        p.wm = p.wn = 0;
        p.tm = rows >= 256 ? 128 : 64;
        p.tn = 64;
        p.m_wg = (int)cdiv(rows, p.tm);
        p.n_wg = (int)cdiv(cols, p.tn);
        p.ksteps = (int)cdiv(K, 32);
        const int nchunks = (int)(K / kRgChunk);
        const int tiles = p.m_wg * p.n_wg;
        int ks = tiles >= 256 ? 1 : 8;
        ks = std::min(ks, std::max(1, nchunks / 2));
        p.ksplit = std::min(ks, kMaxKSplit);
        p.partial_bytes = p.ksplit > 1 ? (size_t)p.ksplit * rows * cols * sizeof(float) : 0;
        return p;
    }
    if (gru) {
        p.wn = 3;
        p.wm = rows <= 16 ? 1 : (rows <= 32 ? 2 : 4);
    } else if (rows <= 16) {
        p.wm = 1; p.wn = 1;
    } else {
        // 32 x 32 output tiles: at M=512 the 64 x 64 tiles leave only 64
        // workgroups before split-K and measured 29 us against 16 us here.
        p.wm = 2; p.wn = 2;
    }
    p.m_wg = (int)cdiv(rows, 16 * p.wm);
    p.n_wg = (int)cdiv(cols, gru ? 16 : 16 * p.wn);
    p.ksteps = (int)cdiv(K, 32);
    const int tiles = p.m_wg * p.n_wg;
    // Aim for about 256 workgroups with at least one K step per wave -- but
    // keep K whole while a wave has at most 16 K steps: the split-K hand-off
    // (device-coherent partials, a counter, the last workgroup's reads) costs
    // more than the longer K loop at these sizes.
    int ks = (int)std::max<int64_t>(1, 256 / std::max(tiles, 1));
    ks = std::min(ks, std::max(1, p.ksteps / 4));
    if (p.ksteps <= 64) ks = 1;
    p.ksplit = std::min(ks, kMaxKSplit);
    p.partial_bytes = p.ksplit > 1 ? (size_t)p.ksplit * tiles * p.wm * p.wn * 256 * sizeof(float) : 0;
    return p;
}

size_t skinny_data_bytes(const SkinnyPlan& p) { return align256(p.partial_bytes); }

bool skinny_supported(const SkinnyPlan& p) { return (int64_t)p.m_wg * p.n_wg <= kMaxCounters; }

template <int WM, int WN, int EPI>
static hipError_t launch_skinny(const SkinnyKArgs& ka, const SkinnyPlan& p, int wmode, hipStream_t s) {
    dim3 grid(p.n_wg, p.m_wg, p.ksplit);
    if (wmode == W_PACKED)
        hipLaunchKernelGGL((skinny_gemm_kernel<WM, WN, EPI, W_PACKED>), grid, dim3(256), 0, s, ka);
    else if (wmode == W_ROWMAJOR)
        hipLaunchKernelGGL((skinny_gemm_kernel<WM, WN, EPI, W_ROWMAJOR>), grid, dim3(256), 0, s, ka);
    else if constexpr (EPI == EPI_RANK)
        hipLaunchKernelGGL((skinny_gemm_kernel<WM, WN, EPI, W_PACKED_E4M3>), grid, dim3(256), 0, s, ka);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int TM, int TN>
static hipError_t launch_rank_tiled(const SkinnyKArgs& ka, dim3 grid, int wmode, hipStream_t s) {
    const dim3 block(rg_threads<TM, TN>());
    if (wmode == W_PACKED)
        hipLaunchKernelGGL((rank_gemm_tiled_kernel<W_PACKED, TM, TN>), grid, block, 0, s, ka);
    else if (wmode == W_PACKED_E4M3)
        hipLaunchKernelGGL((rank_gemm_tiled_kernel<W_PACKED_E4M3, TM, TN>), grid, block, 0, s, ka);
    else
        hipLaunchKernelGGL((rank_gemm_tiled_kernel<W_ROWMAJOR, TM, TN>), grid, block, 0, s, ka);
    return hipGetLastError();
}

static void fill_ws(SkinnyKArgs& ka, const SkinnyPlan& p, void* ws, size_t data_off) {
    char* w = static_cast<char*>(ws);
    ka.counters = reinterpret_cast<unsigned int*>(w + kCountersOff);
    ka.partial = p.ksplit > 1 ? reinterpret_cast<float*>(w + data_off) : nullptr;
    ka.ksteps = p.ksteps;
    ka.ksplit = p.ksplit;
}

hipError_t launch_rank_proj(const RankArgs& a, const SkinnyPlan& p, void* ws, size_t data_off, hipStream_t s) {
    SkinnyKArgs ka{};
    ka.x = a.h; ka.ldx = a.ldh;
    ka.w = a.A; ka.ldw = a.lda;
    ka.M = a.M; ka.K = a.d; ka.wrows = a.r; ka.ncols = a.r;
    ka.col_scale = a.a_scale;
    ka.bias = a.bias; ka.act = a.act;
    ka.out = a.rank; ka.ldout = a.ldrank;
    fill_ws(ka, p, ws, data_off);
    const int wmode = a.a_scale ? W_PACKED_E4M3 : (a.a_packed ? W_PACKED : W_ROWMAJOR);
    if (p.tiled) {
        const dim3 grid(p.ksplit, p.n_wg, p.m_wg);
        hipError_t e0 = hipSuccess;
        if (p.tm == 64 && p.tn == 64) e0 = launch_rank_tiled<64, 64>(ka, grid, wmode, s);
        else if (p.tm == 128 && p.tn == 64) e0 = launch_rank_tiled<128, 64>(ka, grid, wmode, s);
        else return hipErrorInvalidValue;
        if (e0 != hipSuccess) return e0;
        hipError_t e = hipGetLastError();
        if (e != hipSuccess || p.ksplit == 1) return e;
        const int64_t quads = (int64_t)ka.M * ka.ncols / 4;
        const dim3 egrid((unsigned)((quads + 255) / 256));
        if (a.rank_q != nullptr) {
            if (!rank_proj_quantizes(p, a.r)) return hipErrorInvalidValue;
            ka.out_q = a.rank_q;
            ka.out_qscale = a.rank_qscale;
            hipLaunchKernelGGL(rank_splitk_epilogue_kernel<true>, egrid, dim3(256), 0, s, ka);
        } else {
            hipLaunchKernelGGL(rank_splitk_epilogue_kernel<false>, egrid, dim3(256), 0, s, ka);
        }
        return hipGetLastError();
    }
    if (p.wm == 1) return launch_skinny<1, 1, EPI_RANK>(ka, p, wmode, s);
    return launch_skinny<2, 2, EPI_RANK>(ka, p, wmode, s);
}

hipError_t launch_gru_step(const GruArgs& a, const SkinnyPlan& p, void* ws, size_t data_off, hipStream_t s) {
    SkinnyKArgs ka{};
    ka.x = a.h_in; ka.ldx = a.ldh_in;
    ka.w = a.w_hh; ka.ldw = a.G;
    ka.M = a.batch; ka.K = a.G; ka.wrows = 3 * a.G; ka.ncols = a.G;
    ka.bias = a.b_hh; ka.act = 0;
    ka.out = a.h_out; ka.ldout = a.ldh_out;
    ka.gi_table = a.gi_table; ka.ld_gi = a.ld_gi; ka.table_rows = a.table_rows;
    ka.tokens = a.tokens; ka.tok_stride = a.tok_stride;
    // A zero state needs no K loop: every workgroup runs the epilogue alone.
    SkinnyPlan q = p;
    if (a.h_in == nullptr) q.ksplit = 1;
    fill_ws(ka, q, ws, data_off);
    const int wmode = a.w_packed ? W_PACKED : W_ROWMAJOR;
    if (q.wm == 1) return launch_skinny<1, 3, EPI_GRU>(ka, q, wmode, s);
    if (q.wm == 2) return launch_skinny<2, 3, EPI_GRU>(ka, q, wmode, s);
    return launch_skinny<4, 3, EPI_GRU>(ka, q, wmode, s);
}

}  // namespace dels

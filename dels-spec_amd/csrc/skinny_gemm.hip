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
            const float rg = sigmoid_f32(gir + ghr);
            const float zg = sigmoid_f32(giz + ghz);
            const float ng = 2.0f * sigmoid_f32(2.0f * (gin + rg * ghn)) - 1.0f;
            const float hn = (1.0f - zg) * ng + zg * hp;
            a.out[(int64_t)b * a.ldout + g] = f32_to_bf16_bits(hn);
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
                if constexpr (WMODE == W_PACKED) {
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
// Host side
// ---------------------------------------------------------------------------

static inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

SkinnyPlan plan_skinny(int64_t rows, int64_t K, int64_t cols, bool gru) {
    SkinnyPlan p{};
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
    // Aim for about 256 workgroups with at least one K step per wave.
    int ks = (int)std::max<int64_t>(1, 256 / std::max(tiles, 1));
    ks = std::min(ks, std::max(1, p.ksteps / 4));
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

// Host side of the fused combine + argmax: workspace layout and dispatch to
// the per-dtype instantiations of the GEMV kernel (fused_argmax_gemv.h, few
// rows) and of the MFMA-tiled kernel (fused_argmax_tiled.h, many rows).
#include <algorithm>

#include "fused_argmax_fp8.h"
#include "fused_argmax_gemv.h"
#include "fused_argmax_tiled.h"
#include "fused_argmax_tiled8.h"
#include "lowrank_decode.h"

namespace dels {

namespace {

// Rows from which the tiled kernel takes over from the GEMV kernel.
constexpr int kTiledMinRows = 64;
// CUs the tiled grid is planned for (MI355X).  A fixed figure keeps the
// partials size, and so every *_ws_bytes() result, independent of the device.
constexpr int kPlanCUs = 256;

int base_elem_bytes(int dtype) { return dtype == 0 ? 4 : 2; }

// The tiled kernel reads B in the packed layout with r a multiple of 32 (up to
// 512), and moves base/prior rows with 16-byte direct-to-LDS loads.
bool tiled_eligible(const ArgmaxArgs& a) {
    if (a.M < kTiledMinRows || !a.b_packed) return false;
    if (a.r % 32 != 0 || !(a.r == 128 || a.r == 256 || a.r == 512)) return false;
    const int eb = base_elem_bytes(a.base_dtype);
    const int vq = 16 / eb;   // elements per 16-byte base load
    if (a.V % vq != 0 || a.ldbase % vq != 0 || (reinterpret_cast<uintptr_t>(a.base) & 15) != 0) return false;
    // per-lane 32-bit byte offsets into base
    if ((int64_t)a.M * a.ldbase * eb >= ((int64_t)1 << 31)) return false;
    if (a.prior != nullptr) {
        const int pb = base_elem_bytes(a.prior_dtype);
        if ((reinterpret_cast<uintptr_t>(a.prior) & 3) != 0 || (pb == 2 && (a.V & 1) != 0)) return false;
    }
    return (reinterpret_cast<uintptr_t>(a.rank) & 15) == 0 && a.ldrank % 8 == 0;
}

}  // namespace

size_t argmax_data_bytes(int64_t /*M*/, int64_t /*r*/, int64_t /*V*/) { return 0; }

// The e4m3 argmax also keeps the rank quantised per row (tiled kernel).
size_t argmax_fp8_data_bytes(int64_t M, int64_t r, int64_t /*V*/) {
    if (M < kTiledMinRows) return 0;
    return align256((size_t)M * r) + align256((size_t)M * 4);
}

bool argmax_supported(int64_t M, int64_t r, int64_t /*V*/) { return r >= 8 && r <= 512 && M <= kMaxKeyRows; }

hipError_t launch_fused_argmax(const ArgmaxArgs& a, void* ws, size_t data_off, hipStream_t s) {
    // prior kind: 0 none, 1 fp32, 2 bf16, 3 fp16
    const int pk = a.prior == nullptr ? 0 : (a.prior_dtype == 1 ? 2 : (a.prior_dtype == 2 ? 3 : 1));
    char* w = static_cast<char*>(ws);
    if (tiled_eligible(a)) {
        int gx = 1, gy = 1;
        tiled_grid(a.M, a.V, kPlanCUs, &gx, &gy);
        TiledKArgs ka{};
        ka.rank = a.rank; ka.ldrank = a.ldrank;
        ka.rank_rows = a.rank_rows; ka.rank_rows_stride = a.rank_rows_stride; ka.rank_rows_count = a.rank_rows_count;
        ka.B = a.B;
        ka.base = a.base; ka.ldbase = a.ldbase;
        ka.prior = a.prior;
        ka.alpha = a.alpha; ka.alpha_stride = a.alpha_stride;
        ka.beta = a.beta; ka.beta_stride = a.beta_stride;
        ka.M = a.M; ka.V = a.V;
        ka.nblk16 = (a.V + 15) / 16;
        ka.ntiles = (a.V + tiled::kTileCols - 1) / tiled::kTileCols;
        ka.counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
        ka.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
        ka.key_stride = (int64_t)a.M * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
        ka.out_ids = a.out_ids; ka.out_score = a.out_score; ka.ld_out = a.ld_out;
        const int ks = a.r / 32;
        hipError_t e;
        if (a.base_dtype == 1) e = launch_tiled_bf16(ka, ks, pk, gx, gy, s);
        else if (a.base_dtype == 2) e = launch_tiled_f16(ka, ks, pk, gx, gy, s);
        else e = launch_tiled_f32(ka, ks, pk, gx, gy, s);
        return e;
    }
    ArgmaxKArgs ka{};
    ka.rank = a.rank; ka.ldrank = a.ldrank;
    ka.rank_rows = a.rank_rows; ka.rank_rows_stride = a.rank_rows_stride; ka.rank_rows_count = a.rank_rows_count;
    ka.B = a.B; ka.ldb = a.ldb;
    ka.base = a.base; ka.ldbase = a.ldbase;
    ka.prior = a.prior;
    ka.alpha = a.alpha; ka.alpha_stride = a.alpha_stride;
    ka.beta = a.beta; ka.beta_stride = a.beta_stride;
    ka.M = a.M; ka.r = a.r; ka.V = a.V;
    ka.ksteps = (a.r + 31) / 32;
    ka.out_ids = a.out_ids; ka.out_score = a.out_score; ka.ld_out = a.ld_out;
    ka.counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
    ka.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    // one 128-byte line per row while the rows fit the key area, else packed
    ka.key_stride = (int64_t)a.M * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
    if (a.base_dtype == 1) return launch_gemv_bf16(ka, a.b_packed, pk, s);
    if (a.base_dtype == 2) return launch_gemv_f16(ka, a.b_packed, pk, s);
    return launch_gemv_f32(ka, a.b_packed, pk, s);
}

// ---- plain row argmax ------------------------------------------------------------
//
// sample() at temperature 0 (code/dflash.py:31-33: torch.argmax over the last
// dimension): the lowest index of each row's maximum, where NaN counts as
// larger than every number (torch.argmax returns the index of the first NaN).
// Each candidate becomes its 64-bit key order(score) << 32 | ~index (every NaN
// as the same quiet NaN, whose key lies above +inf's), so an unsigned max is
// the argmax with both rules.  Rows are split into chunks over workgroups;
// each folds its best key into the row's key with a device-scope atomic max,
// and the last workgroup decodes and clears the keys and the counter (as the
// fused argmax).  An all -inf row gives index 0 with score -inf.

namespace {

__device__ __forceinline__ unsigned long long row_argmax_key(float v, uint32_t idx) {
    return pack_argmax(v != v ? __uint_as_float(0x7fc00000u) : v, idx);
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long x, int off) {
    const uint32_t lo = __shfl_xor((uint32_t)x, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(x >> 32), off, 64);
    return ((unsigned long long)hi << 32) | lo;
}

// Element e of 16 bytes of values of type T, widened.
template <typename T>
__device__ __forceinline__ float elem16(const u32x4& w, int e) {
    if constexpr (sizeof(T) == 4) {
        return __uint_as_float(w[e]);
    } else {
        const uint16_t b = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
        if constexpr (std::is_same<T, bf16_t>::value) {
            return bf16_bits_to_f32(b);
        } else {
            _Float16 h;
            __builtin_memcpy(&h, &b, 2);
            return (float)h;
        }
    }
}

constexpr int kRowsVecLoads = 4;   // 16-byte loads in flight per thread (VEC)

// VEC: rows 16-byte aligned, V and the chunk multiples of 16 / sizeof(T): each
// thread takes 16-byte pieces, kRowsVecLoads of them in flight at once.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void argmax_rows_kernel(const T* __restrict__ x, int64_t ldx, int M, int V,
                                                          int chunk, unsigned long long* keys, int64_t key_stride,
                                                          unsigned int* counter, int64_t* out_ids, float* out_score,
                                                          int64_t ld_out) {
    __shared__ unsigned long long s_key[4];
    __shared__ int s_last;
    const int m = blockIdx.y;
    const int v0 = blockIdx.x * chunk;
    const int v1 = min(V, v0 + chunk);
    const T* row = x + (int64_t)m * ldx;
    unsigned long long best = 0ull;   // below every candidate's key
    if constexpr (VEC) {
        constexpr int E = 16 / (int)sizeof(T);
        const int nv = (v1 - v0) / E;
        for (int i0 = threadIdx.x; i0 < nv; i0 += 256 * kRowsVecLoads) {
            u32x4 w[kRowsVecLoads];
#pragma unroll
            for (int u = 0; u < kRowsVecLoads; ++u) {
                const int i = i0 + 256 * u;
                w[u] = i < nv ? __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(row + v0 + i * E))
                              : u32x4{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int u = 0; u < kRowsVecLoads; ++u) {
                const int i = i0 + 256 * u;
                if (i < nv) {
#pragma unroll
                    for (int e = 0; e < E; ++e) {
                        const unsigned long long k = row_argmax_key(elem16<T>(w[u], e), (uint32_t)(v0 + i * E + e));
                        best = k > best ? k : best;
                    }
                }
            }
        }
    } else {
        for (int v = v0 + (int)threadIdx.x; v < v1; v += 256) {
            const unsigned long long k = row_argmax_key(load_f32(row + v), (uint32_t)v);
            best = k > best ? k : best;
        }
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned long long o = shfl_xor_u64(best, off);
        best = o > best ? o : best;
    }
    const int wave = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) s_key[wave] = best;
    __syncthreads();
    unsigned long long seen = 0;
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) best = s_key[w] > best ? s_key[w] : best;
        if (best != 0ull)
            seen = __hip_atomic_fetch_max(&keys[(int64_t)m * key_stride], best, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        // the returned value orders the count after the update
        const unsigned prev = __hip_atomic_fetch_add(counter, seen == ~0ull ? 2u : 1u, __ATOMIC_RELAXED,
                                                     __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == gridDim.x * gridDim.y - 1;
    }
    __syncthreads();
    if (!s_last) return;
    for (int r = threadIdx.x; r < M; r += blockDim.x) {
        const unsigned long long key = __hip_atomic_exchange(&keys[(int64_t)r * key_stride], 0ull, __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_AGENT);
        uint32_t idx = ~(uint32_t)(key & 0xffffffffull);
        float val = f32_from_order_key((uint32_t)(key >> 32));
        if (key == 0ull || idx >= (uint32_t)V) {
            idx = 0;
            val = -__builtin_inff();
        }
        out_ids[(int64_t)r * ld_out] = (int64_t)idx;
        if (out_score) out_score[(int64_t)r * ld_out] = val;
    }
    if (threadIdx.x == 0) __hip_atomic_exchange(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_argmax_rows(const void* x, int64_t ldx, int dtype, int M, int V, int64_t* out_ids,
                              float* out_score, int64_t ld_out, void* ws, hipStream_t s) {
    char* w = static_cast<char*>(ws);
    auto* counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
    auto* keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    const int64_t key_stride = (int64_t)M * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
    const int gx = std::max(1, std::min(64, (V + 8191) / 8192));   // chunks of ~8K: 4K and 16K measured slower
    const int E = dtype == 0 ? 4 : 8;   // elements per 16 bytes
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15) == 0 && ldx % E == 0 && V % E == 0;
    int chunk = (V + gx - 1) / gx;
    if (vec) chunk = (chunk + E - 1) / E * E;
    const dim3 grid((unsigned)((V + chunk - 1) / chunk), M);
    auto go = [&](auto tag, auto vec_tag) {
        using T = decltype(tag);
        hipLaunchKernelGGL((argmax_rows_kernel<T, decltype(vec_tag)::value>), grid, dim3(256), 0, s,
                           static_cast<const T*>(x), ldx, M, V, chunk, keys, key_stride, counter, out_ids, out_score,
                           ld_out);
    };
    using VecOn = std::integral_constant<bool, true>;
    using VecOff = std::integral_constant<bool, false>;
    if (dtype == 1) vec ? go(bf16_t{}, VecOn{}) : go(bf16_t{}, VecOff{});
    else if (dtype == 2) vec ? go(f16_t{}, VecOn{}) : go(f16_t{}, VecOff{});
    else vec ? go(float{}, VecOn{}) : go(float{}, VecOff{});
    return hipGetLastError();
}

// ---- fp8 argmax ------------------------------------------------------------

bool argmax_fp8_supported(int64_t M, int64_t r) {
    return (r == 128 || r == 256 || r == 512) && M >= 0 && M <= kMaxKeyRows;
}

namespace {

// Per-row e4m3 quantisation of the rank for the tiled kernel, with the fp8
// GEMV's rule: amax = max |rank[m, :]|, inv = 448 / amax, q = e4m3(rank * inv),
// scale = amax / 448 (1 and zeros for an all-zero row).  One wave per row, r <= 512.
__global__ __launch_bounds__(256) void quantize_rank_e4m3_kernel(const uint16_t* __restrict__ rank, int64_t ldrank,
                                                                 int M, int r, uint8_t* __restrict__ rank_q,
                                                                 float* __restrict__ rank_scale) {
#pragma clang fp contract(off)
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (m >= M) return;
    const uint16_t* row = rank + (int64_t)m * ldrank;
    const bool ok = 8 * lane < r;   // lane: values 8 * lane .. + 7
    const u32x4 v = ok ? *reinterpret_cast<const u32x4*>(row + 8 * lane) : u32x4{0u, 0u, 0u, 0u};
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        amax = __builtin_fmaxf(amax, __builtin_fabsf(__uint_as_float(v[e] << 16)));
        amax = __builtin_fmaxf(amax, __builtin_fabsf(__uint_as_float(v[e] & 0xffff0000u)));
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, off, 64));
    const float inv = amax > 0.f ? kE4M3Max / amax : 1.f;
    uint32_t w[2];
#pragma unroll
    for (int hw = 0; hw < 2; ++hw) {
        const uint32_t x0 = v[2 * hw], x1 = v[2 * hw + 1];
        w[hw] = f32x4_to_e4m3(__uint_as_float(x0 << 16) * inv, __uint_as_float(x0 & 0xffff0000u) * inv,
                              __uint_as_float(x1 << 16) * inv, __uint_as_float(x1 & 0xffff0000u) * inv);
    }
    if (ok) *reinterpret_cast<u32x2*>(rank_q + (int64_t)m * r + 8 * lane) = u32x2{w[0], w[1]};
    if (lane == 0) rank_scale[m] = amax > 0.f ? amax / kE4M3Max : 1.f;
}

}  // namespace

// The e4m3 tiled kernel: the bf16 tiled kernel's conditions, r = 256 or 512
// (B loads per stage split evenly over 8 waves) and 4-byte aligned B scales.
static bool tiled8_eligible(const ArgmaxArgs& a) {
    if (!(a.r == 256 || a.r == 512) || (reinterpret_cast<uintptr_t>(a.b_scale) & 3) != 0) return false;
    ArgmaxArgs t = a;
    t.b_packed = true;
    return tiled_eligible(t);
}

bool fp8_argmax_tiled(const ArgmaxArgs& a) { return tiled8_eligible(a); }

hipError_t launch_fused_argmax_fp8(const ArgmaxArgs& a, void* ws, size_t data_off, hipStream_t s) {
    const int pk = a.prior == nullptr ? 0 : (a.prior_dtype == 1 ? 2 : (a.prior_dtype == 2 ? 3 : 1));
    char* w = static_cast<char*>(ws);
    if (tiled8_eligible(a)) {
        int gx = 1, gy = 1;
        tiled_grid(a.M, a.V, kPlanCUs, &gx, &gy);
        TiledKArgs ka{};
        ka.rank = a.rank; ka.ldrank = a.ldrank;
        ka.B = a.B;
        ka.b_scale = a.b_scale;
        ka.base = a.base; ka.ldbase = a.ldbase;
        ka.prior = a.prior;
        ka.alpha = a.alpha; ka.alpha_stride = a.alpha_stride;
        ka.beta = a.beta; ka.beta_stride = a.beta_stride;
        ka.M = a.M; ka.V = a.V;
        ka.nblk16 = (a.V + 15) / 16;
        ka.ntiles = (a.V + tiled::kTileCols - 1) / tiled::kTileCols;
        ka.counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
        ka.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
        ka.key_stride = (int64_t)a.M * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
        ka.out_ids = a.out_ids; ka.out_score = a.out_score; ka.ld_out = a.ld_out;
        // the rank, quantised per row to e4m3
        uint8_t* rank_q = reinterpret_cast<uint8_t*>(w + data_off);
        float* rank_scale = reinterpret_cast<float*>(reinterpret_cast<char*>(rank_q) + align256((size_t)a.M * a.r));
        if (!a.rank_quantized)
            hipLaunchKernelGGL(quantize_rank_e4m3_kernel, dim3((a.M + 3) / 4), dim3(256), 0, s, a.rank, a.ldrank,
                               a.M, a.r, rank_q, rank_scale);
        ka.rank_q = rank_q;
        ka.ldrank = a.r;
        ka.rank_scale = rank_scale;
        const int ks8 = a.r / 128;
        hipError_t e;
        if (a.base_dtype == 1) e = launch_tiled8_bf16(ka, ks8, pk, gx, gy, s);
        else if (a.base_dtype == 2) e = launch_tiled8_f16(ka, ks8, pk, gx, gy, s);
        else e = launch_tiled8_f32(ka, ks8, pk, gx, gy, s);
        return e;
    }
    ArgmaxKArgs ka{};
    ka.rank = a.rank; ka.ldrank = a.ldrank;
    ka.B = a.B; ka.ldb = 0;
    ka.b_scale = a.b_scale;
    ka.base = a.base; ka.ldbase = a.ldbase;
    ka.prior = a.prior;
    ka.alpha = a.alpha; ka.alpha_stride = a.alpha_stride;
    ka.beta = a.beta; ka.beta_stride = a.beta_stride;
    ka.M = a.M; ka.r = a.r; ka.V = a.V;
    ka.ksteps = a.r / 32;
    ka.out_ids = a.out_ids; ka.out_score = a.out_score; ka.ld_out = a.ld_out;
    ka.counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
    ka.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    ka.key_stride = (int64_t)a.M * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
    if (a.base_dtype == 1) return launch_gemv8_bf16(ka, pk, s);
    if (a.base_dtype == 2) return launch_gemv8_f16(ka, pk, s);
    return launch_gemv8_f32(ka, pk, s);
}

// ---- fused decode step ------------------------------------------------------

namespace {
int g_decode_spin_limit = 1 << 14;
// K slices of the in-launch rank projection: nct * slices workgroups compute
// rank partials, the rest go straight to the argmax stream.
constexpr int kDecodeSlices = 4;

struct DecodePlan {
    int nct, nz, kpz, ksa;
};

DecodePlan decode_plan(int64_t d, int64_t r) {
    DecodePlan p{};
    p.nct = (int)(r / 16);
    // short K (a rollout's hidden size of 1024 or less): two slices (14-step
    // rollout at G=1024, r=256: 387 -> 381 us); four otherwise (Qwen3-8B step:
    // 31.6 us against 32.2 with two and 34.9 with eight)
    p.nz = std::min(d <= 1024 ? 2 : kDecodeSlices, kDecodeWGs / std::max(p.nct, 1));
    p.ksa = (int)(d / 32);
    p.kpz = (p.ksa + p.nz - 1) / std::max(p.nz, 1);
    return p;
}
}  // namespace

int set_decode_spin_limit(int limit) {
    const int prev = g_decode_spin_limit;
    g_decode_spin_limit = std::max(0, limit);
    return prev;
}

bool decode_eligible(int64_t M, int64_t d, int64_t r, bool a_packed, bool b_packed) {
    if (M < 1 || M > 16 || !a_packed || !b_packed) return false;
    if (!(r == 64 || r == 128 || r == 256 || r == kDecodeMaxRank)) return false;
    if (d < 32 || d % 32 != 0) return false;
    return kDecodeWGs % decode_plan(d, r).nct == 0;
}

bool decode_gru_eligible(int64_t M, int64_t G, int64_t r) {
    if (!decode_eligible(M, G, r, true, true) || G > kGruMaxG || G % 32 != 0) return false;
    const DecodePlan p = decode_plan(G, r);
    // GRU workgroups after the rank workgroups; the new state's words after the
    // partial words (at most 128 rank workgroups)
    return p.nct * p.nz + G / kGruUnits <= kDecodeWGs && p.nct * p.nz <= 128;
}

bool decode8_eligible(int64_t M, int64_t d, int64_t r) {
    return (r == 128 || r == 256 || r == 512) && decode_eligible(M, d, r, true, true);
}

static_assert(128 * 256 + 16 * (kGruMaxG / 2) <= kDecodeWGs * 256,
              "the fused GRU's state words fit after the partial words of 128 rank workgroups");
static_assert(kDecodeWordBytes >= align256((size_t)kDecodeWGs * 256 * sizeof(unsigned long long)) +
                                     (size_t)16 * (kDecodeMaxRank / 2) * sizeof(unsigned long long),
              "the reserved decode region holds every workgroup's partial words and the rank words");

hipError_t launch_lowrank_decode(const RankArgs& ra, const ArgmaxArgs& a, void* ws, hipStream_t s,
                                 const DecodeGru* gru) {
    const DecodePlan p = decode_plan(ra.d, ra.r);
    char* w = static_cast<char*>(ws);
    DecodeKArgs k{};
    ArgmaxKArgs& ka = k.am;
    ka.rank = nullptr; ka.ldrank = 0;
    ka.B = a.B; ka.ldb = a.ldb;
    ka.base = a.base; ka.ldbase = a.ldbase;
    ka.prior = a.prior;
    ka.alpha = a.alpha; ka.alpha_stride = a.alpha_stride;
    ka.beta = a.beta; ka.beta_stride = a.beta_stride;
    ka.M = a.M; ka.r = a.r; ka.V = a.V;
    ka.ksteps = a.r / 32;
    ka.out_ids = a.out_ids; ka.out_score = a.out_score; ka.ld_out = a.ld_out;
    unsigned int* counters = reinterpret_cast<unsigned int*>(w + kCountersOff);
    ka.counter = counters;                         // argmax arrivals
    ka.keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    ka.key_stride = 16;                            // M <= 16: one 128-byte line per row
    k.gen = counters + kDecodeGenWord;             // launch generation (never reset)
    k.h = ra.h; k.ldh = ra.ldh;
    k.A = ra.A;
    k.bias = ra.bias; k.act = ra.act;
    k.ksa = p.ksa; k.nct = p.nct; k.nz = p.nz; k.kpz = p.kpz;
    k.partial_words = reinterpret_cast<unsigned long long*>(w + kDecodeOff);
    k.rank_words = reinterpret_cast<unsigned long long*>(
        w + kDecodeOff + align256((size_t)kDecodeWGs * 256 * sizeof(unsigned long long)));
    k.spin_limit = g_decode_spin_limit;
    if (gru) {
        if (ra.a_scale != nullptr) return hipErrorInvalidValue;   // the fused GRU runs with bf16 weights only
        k.gi_table = gru->gi_table; k.ld_gi = gru->ld_gi; k.table_rows = gru->table_rows;
        k.tokens = gru->tokens; k.tok_stride = gru->tok_stride;
        k.w_hh = gru->w_hh; k.b_hh = gru->b_hh;
        k.h_prev = gru->h_prev; k.h_out = gru->h_out;
        k.h_words = k.partial_words + 128 * 256;   // past the partial words of <= 128 rank workgroups
    }
    const int pk = a.prior == nullptr ? 0 : (a.prior_dtype == 1 ? 2 : (a.prior_dtype == 2 ? 3 : 1));
    if (ra.a_scale != nullptr) {
        k.a_scale = ra.a_scale;
        ka.b_scale = a.b_scale;
        if (a.base_dtype == 1) return launch_decode8_bf16(k, pk, s);
        if (a.base_dtype == 2) return launch_decode8_f16(k, pk, s);
        return launch_decode8_f32(k, pk, s);
    }
    if (a.base_dtype == 1) return launch_decode_bf16(k, ka.ksteps, pk, s, gru != nullptr);
    if (a.base_dtype == 2) return launch_decode_f16(k, ka.ksteps, pk, s, gru != nullptr);
    return launch_decode_f32(k, ka.ksteps, pk, s, gru != nullptr);
}

}  // namespace dels

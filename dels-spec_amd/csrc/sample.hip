// Temperature sampling of rows of logits: sample() at temperature > 0
// (code/dflash.py:31-38: softmax(logits / T) then torch.multinomial), as a
// Gumbel-max in one pass that never writes probabilities.
//
// For row m and vocabulary index v:
//     y[m, v] = round_T(fp32(x[m, v]) / T)          # logits / temperature, in the logits' dtype
//     u[m, v] = ((bits >> 9) + 0.5) * 2^-23          # in (0, 1), exact in fp32
//     g[m, v] = -log(-log(u[m, v]))                  # standard Gumbel noise
//     id_m    = argmax_v (y[m, v] + g[m, v])         # distributed as softmax(y[m, :])
// where `bits` is word v%4 of Philox4x32-10 (Salmon et al., "Parallel random
// numbers: as easy as 1, 2, 3", SC 2011) at counter (v/4, m, offset_lo,
// offset_hi) and key (seed_lo, seed_hi).  Every element has its own counter,
// so the result depends only on (seed, offset, m, v): any grid, any chunking
// and any later call with the same arguments give the same ids.
//
// The reduction is the one of argmax_rows_kernel: one 64-bit key per
// candidate (order(score) << 32 | ~index, NaN above +inf), a device-scope
// atomic max per workgroup and row, and a last-arriver decode that returns
// keys and counter to zero.
#include <algorithm>

#include "dels_device.h"
#include "dels_internal.h"

namespace dels {

namespace {

constexpr uint32_t kPhiloxM0 = 0xD2511F53u, kPhiloxM1 = 0xCD9E8D57u;
constexpr uint32_t kPhiloxW0 = 0x9E3779B9u, kPhiloxW1 = 0xBB67AE85u;

// Ten rounds of Philox4x32 on counter c with key (k0, k1).
__device__ __forceinline__ void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
#pragma unroll
    for (int r = 0; r < 10; ++r) {
        const uint32_t lo0 = kPhiloxM0 * c[0], hi0 = __umulhi(kPhiloxM0, c[0]);
        const uint32_t lo1 = kPhiloxM1 * c[2], hi1 = __umulhi(kPhiloxM1, c[2]);
        const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
        c[0] = n0; c[1] = lo1; c[2] = n2; c[3] = lo0;
        k0 += kPhiloxW0;
        k1 += kPhiloxW1;
    }
}

// Gumbel noise from 32 random bits: u = ((bits >> 9) + 0.5) * 2^-23 lies in
// [2^-24, 1 - 2^-24] and is exact in fp32, so both logarithms are finite.
__device__ __forceinline__ float gumbel_from_bits(uint32_t bits) {
    const float u = ((float)(bits >> 9) + 0.5f) * 0x1p-23f;
    return -logf(-logf(u));
}

// logits / temperature rounded to the logits' dtype, as torch divides a
// bf16/fp16 tensor by a Python float (fp32 arithmetic, one rounding).
__device__ __forceinline__ float tempered(float x, float t, float) { return x / t; }
__device__ __forceinline__ float tempered(float x, float t, bf16_t) { return round_bf16(x / t); }
__device__ __forceinline__ float tempered(float x, float t, f16_t) { return (float)(_Float16)(x / t); }

__device__ __forceinline__ unsigned long long sample_key(float v, uint32_t idx) {
    return pack_argmax(v != v ? __uint_as_float(0x7fc00000u) : v, idx);
}

__device__ __forceinline__ unsigned long long shfl_xor_u64(unsigned long long x, int off) {
    const uint32_t lo = __shfl_xor((uint32_t)x, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(x >> 32), off, 64);
    return ((unsigned long long)hi << 32) | lo;
}

// Grid (chunks, M); a chunk is a multiple of 4 elements, a thread takes one
// group of 4 (one Philox call) per iteration.
template <typename T>
__global__ __launch_bounds__(256) void sample_rows_kernel(const T* __restrict__ x, int64_t ldx, int M, int V,
                                                          int chunk, float temperature, uint32_t k0, uint32_t k1,
                                                          uint32_t off_lo, uint32_t off_hi, unsigned long long* keys,
                                                          int64_t key_stride, unsigned int* counter,
                                                          int64_t* out_ids, float* out_score, int64_t ld_out) {
    __shared__ unsigned long long s_key[4];
    __shared__ int s_last;
    const int m = blockIdx.y;
    const int v0 = blockIdx.x * chunk;
    const int v1 = min(V, v0 + chunk);
    const T* row = x + (int64_t)m * ldx;
    unsigned long long best = 0ull;   // below every candidate's key
    for (int g = v0 + 4 * (int)threadIdx.x; g < v1; g += 4 * 256) {
        uint32_t c[4] = {(uint32_t)g >> 2, (uint32_t)m, off_lo, off_hi};
        philox4x32_10(c, k0, k1);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int v = g + q;
            if (v < v1) {
                const float y = tempered(load_f32(row + v), temperature, T{});
                const unsigned long long k = sample_key(y + gumbel_from_bits(c[q]), (uint32_t)v);
                best = k > best ? k : best;
            }
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
    if (threadIdx.x == 0) {
        unsigned long long seen = 0;
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

hipError_t launch_sample_rows(const void* x, int64_t ldx, int dtype, int M, int V, float temperature, uint64_t seed,
                              uint64_t offset, int64_t* out_ids, float* out_score, int64_t ld_out, void* ws,
                              hipStream_t s) {
    char* w = static_cast<char*>(ws);
    auto* counter = reinterpret_cast<unsigned int*>(w + kCountersOff);
    auto* keys = reinterpret_cast<unsigned long long*>(w + kKeysOff);
    const int64_t key_stride = (int64_t)M * 128 <= (int64_t)(kCtrlBytes - kKeysOff) ? 16 : 1;
    const int gx = std::max(1, std::min(64, (V + 4095) / 4096));
    const int chunk = ((V + gx - 1) / gx + 3) & ~3;
    const dim3 grid((V + chunk - 1) / chunk, M);
    const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    const uint32_t o0 = (uint32_t)offset, o1 = (uint32_t)(offset >> 32);
    if (dtype == 1)
        hipLaunchKernelGGL(sample_rows_kernel<bf16_t>, grid, dim3(256), 0, s, static_cast<const bf16_t*>(x), ldx, M,
                           V, chunk, temperature, k0, k1, o0, o1, keys, key_stride, counter, out_ids, out_score,
                           ld_out);
    else if (dtype == 2)
        hipLaunchKernelGGL(sample_rows_kernel<f16_t>, grid, dim3(256), 0, s, static_cast<const f16_t*>(x), ldx, M, V,
                           chunk, temperature, k0, k1, o0, o1, keys, key_stride, counter, out_ids, out_score, ld_out);
    else
        hipLaunchKernelGGL(sample_rows_kernel<float>, grid, dim3(256), 0, s, static_cast<const float*>(x), ldx, M, V,
                           chunk, temperature, k0, k1, o0, o1, keys, key_stride, counter, out_ids, out_score, ld_out);
    return hipGetLastError();
}

}  // namespace dels

// Device-side helpers shared by the gfx950 kernels of the DeLS draft path.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dels {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct bf16_t { uint16_t bits; };   // storage tag for bf16 base/prior
struct f16_t { uint16_t bits; };    // storage tag for fp16 base/prior
struct no_prior_t {};                // "no prior term" tag

template <typename T> struct is_no_prior { static constexpr bool value = false; };
template <> struct is_no_prior<no_prior_t> { static constexpr bool value = true; };

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t b) { return __uint_as_float(b << 16); }

// float -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float round_bf16(float f) { return bf16_bits_to_f32(f32_to_bf16_bits(f)); }

// Scalar element loads of base logits / prior, widened to fp32.
__device__ __forceinline__ float load_f32(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ float load_f32(const bf16_t* p) {
    return bf16_bits_to_f32(__builtin_nontemporal_load(&p->bits));
}
__device__ __forceinline__ float load_f32(const f16_t* p) {
    uint16_t b = __builtin_nontemporal_load(&p->bits);
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// The same loads kept as loaded (fp32 bits, or a 16-bit value zero-extended by
// the load itself) and widened by widen_raw<T> where the value is used: a
// conversion right after a load in a streaming loop makes the compiler wait for
// that load, and for every load issued before it.
__device__ __forceinline__ uint32_t load_raw(const float* p) {
    return __float_as_uint(__builtin_nontemporal_load(p));
}
__device__ __forceinline__ uint32_t load_raw(const bf16_t* p) { return __builtin_nontemporal_load(&p->bits); }
__device__ __forceinline__ uint32_t load_raw(const f16_t* p) { return __builtin_nontemporal_load(&p->bits); }
template <typename T>
__device__ __forceinline__ float widen_raw(uint32_t w) {
    if constexpr (std::is_same<T, float>::value) {
        return __uint_as_float(w);
    } else if constexpr (std::is_same<T, bf16_t>::value) {
        return __uint_as_float(w << 16);
    } else {
        const uint16_t b = (uint16_t)w;
        _Float16 h;
        __builtin_memcpy(&h, &b, 2);
        return (float)h;
    }
}

// 16-byte operand loads: eight bf16 values.
__device__ __forceinline__ bf16x8 load_bf16x8(const uint16_t* p) {
    u32x4 v = *reinterpret_cast<const u32x4*>(p);
    return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ bf16x8 load_bf16x8_nt(const uint16_t* p) {
    u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return __builtin_bit_cast(bf16x8, v);
}
__device__ __forceinline__ bf16x8 zero_bf16x8() { return __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u}); }

// Eight bf16 values kept (mask ~0) or zeroed (mask 0) without a branch.
__device__ __forceinline__ bf16x8 masked_bf16x8(u32x4 v, uint32_t mask) {
    v.x &= mask; v.y &= mask; v.z &= mask; v.w &= mask;
    return __builtin_bit_cast(bf16x8, v);
}

// Order-preserving map float -> uint32 (a < b  <=>  key(a) < key(b) for non-NaN).
// -0.0 is folded onto +0.0 so that equal scores compare equal.
__device__ __forceinline__ uint32_t f32_order_key(float f) {
    if (f == 0.0f) f = 0.0f;
    uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float f32_from_order_key(uint32_t k) {
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// (score, index) packed so that a larger key is a larger score, or the same
// score at a smaller index: unsigned 64-bit max is then the argmax with the
// lowest-index tie rule.  Key 0 is below every real candidate.
__device__ __forceinline__ unsigned long long pack_argmax(float v, uint32_t idx) {
    return ((unsigned long long)f32_order_key(v) << 32) | (unsigned long long)(~idx);
}

// Row of the rank matrix that draft row m reads: m itself, or -- when the rank
// is gathered from a table (the embedding rows of a Markov step) -- the token
// id rows[m * stride], clamped into [0, count) as an embedding lookup's index
// must lie.
__device__ __forceinline__ int64_t rank_row_of(const int64_t* rows, int64_t stride, int64_t count, int m) {
    if (rows == nullptr) return m;
    const int64_t t = rows[(int64_t)m * stride];
    return t < 0 ? 0 : (t >= count ? count - 1 : t);
}

// Candidate (v, i) beats (bv, bi): larger value, or equal value and lower index.
__device__ __forceinline__ bool argmax_better(float v, int i, float bv, int bi) {
    return (v > bv) || (v == bv && i < bi);
}

// Direct-to-LDS loads: lane l's 16 (or 4) bytes from `g` land at LDS address
// M0 + 16*l (4*l); `lds` must be wave-uniform.  Written as asm so that the
// compiler does not track them: its own tracking cannot tell the stage buffers
// apart and would make every LDS read wait for all loads in flight.  The waits
// they need are the explicit vmcnt counts of stage_barrier().
__device__ __forceinline__ uint32_t lds_addr(const void* lds) {
    return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)lds);
}
// Address = wave-uniform 64-bit base (SGPRs) + per-lane 32-bit byte offset.
// The base is read from the first lane so that it is an SGPR pair whatever the
// compiler can prove about its uniformity.
__device__ __forceinline__ const void* sgpr_ptr(const void* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const void*)(uintptr_t)(((uint64_t)hi << 32) | lo);
}
// The compiler's hazard recognizer does not look inside asm, so the statement
// carries its own wait states: a VMEM instruction needs 5 after a VALU write of
// an SGPR it reads (the base pair comes from v_readfirstlane, often just before)
// and an LDS-DMA instruction 1 after the SALU write of M0.  s_nop 4 gives 5.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, void* lds) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dwordx4 %0, %1"
                 : : "v"(off), "s"(sgpr_ptr(base)), "{m0}"(lds_addr(lds)) : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, void* lds) {
    asm volatile("s_nop 4\n\tglobal_load_lds_dword %0, %1"
                 : : "v"(off), "s"(sgpr_ptr(base)), "{m0}"(lds_addr(lds)) : "memory");
}

// Element of an LDS array of base/prior values, widened to fp32.
__device__ __forceinline__ float lds_f32(const float* p) { return *p; }
__device__ __forceinline__ float lds_f32(const bf16_t* p) { return bf16_bits_to_f32(p->bits); }
__device__ __forceinline__ float lds_f32(const f16_t* p) {
    const uint16_t b = p->bits;
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;
}

// Wait until at most `pending` groups of PER direct-to-LDS loads are in flight
// (pending is wave-uniform, 0 .. 4; s_waitcnt takes an immediate).
template <int PER>
__device__ __forceinline__ void wait_dma_groups(int pending) {
    static_assert(4 * PER <= 63, "vmcnt holds at most 63");
    if (pending <= 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if (pending == 1) asm volatile("s_waitcnt vmcnt(%0)" : : "n"(PER) : "memory");
    else if (pending == 2) asm volatile("s_waitcnt vmcnt(%0)" : : "n"(2 * PER) : "memory");
    else if (pending == 3) asm volatile("s_waitcnt vmcnt(%0)" : : "n"(3 * PER) : "memory");
    else asm volatile("s_waitcnt vmcnt(%0)" : : "n"(4 * PER) : "memory");
}

// Barrier for LDS traffic only: loads still in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.0f / (1.0f + expf(-x)); }

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

// New GRU state of one unit from its input-side (gi) and hidden-side (gh,
// already rounded to bf16) gate pre-activations and its previous state hp:
// PyTorch's (r, z, n) order with tanh(x) = 2 sigmoid(2x) - 1, in fp32, every
// product and sum rounded on its own (code/kernel/dels.py:202-211).
__device__ __forceinline__ float gru_unit(float gir, float giz, float gin, float ghr, float ghz, float ghn, float hp) {
#pragma clang fp contract(off)
    const float rg = sigmoid_f32(gir + ghr);
    const float zg = sigmoid_f32(giz + ghz);
    const float ng = 2.0f * sigmoid_f32(2.0f * (gin + rg * ghn)) - 1.0f;
    return (1.0f - zg) * ng + zg * hp;
}

// Agent-scope atomics used by the "last workgroup finishes" reductions.
__device__ __forceinline__ unsigned long long atomic_load_u64(unsigned long long* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_store_u64(unsigned long long* p, unsigned long long v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void atomic_store_u32(unsigned int* p, unsigned int v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace dels

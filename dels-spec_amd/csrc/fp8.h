// fp8 (OCP float8 e4m3fn) support: the format of the fp8 weights, its
// conversions, and the operand pieces of the fp8 argmax kernels.
//
// e4m3fn: sign, 4 exponent bits (bias 7), 3 mantissa bits; no infinities,
// 0x7F/0xFF are NaN, the largest finite magnitude is 448.  gfx950's fp8 MFMAs
// (v_mfma_scale_f32_16x16x128_f8f6f4 with format code 0) read this format.
//
// Packed fp8 layouts (built by pack.hip):
//  * K128 (B, the low-rank LM head): 16-row x 128-column blocks of 2 KiB,
//    row-block-major.  Lane l of a wave owns row l%16 and the 32 consecutive
//    columns 32*(l/16) .. +31 of the block, stored as two 1 KiB halves
//    [half][lane][16 bytes], so each half is one coalesced dwordx4 per lane.
//    The MFMA pairs the A and B operands by (lane group, byte), so any K order
//    that both operands share gives the same dot product; the rank operand is
//    built in this same order.
//  * K32 (A, the rank projection weight): the MFMA-16 bf16 block order with
//    one byte per element: 16-row x 32-column blocks of 512 bytes, lane l
//    holding row l%16, columns 8*(l/16) .. +7.  The rank projection keeps h in
//    bf16, so these bytes are widened to bf16 in registers (exactly: every
//    e4m3 value is a bf16 value) and fed to the bf16 MFMA.
#pragma once

#include "dels_device.h"

namespace dels {

typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr float kE4M3Max = 448.f;
constexpr int kFp8K128Block = 2048;   // bytes of a K128 block
constexpr int kFp8K32Block = 512;     // bytes of a K32 block

// Round a finite fp32 value to the e4m3fn grid (to nearest, ties to even;
// magnitudes from 464, the midpoint between 448 and the next binade step,
// saturate to 448) and encode it.
__device__ __forceinline__ uint32_t f32_to_e4m3(float x) {
    const uint32_t sign = (__float_as_uint(x) >> 24) & 0x80u;
    const float a = __builtin_fabsf(x);
    uint32_t code;
    if (a >= 464.f) {
        code = 0x7Eu;
    } else if (a < 0.015625f) {
        // below 2^-6: the subnormal grid, quantum 2^-9; 8 encodes 2^-6, the first normal
        code = (uint32_t)__builtin_rintf(a * 512.f);
    } else {
        uint32_t b = __float_as_uint(a);
        b += 0x7FFFFu + ((b >> 20) & 1u);                       // 3 mantissa bits, ties to even
        code = (((b >> 23) - 120u) << 3) | ((b >> 20) & 7u);    // exponent rebiased from 127 to 7
    }
    return sign | code;
}

// Four floats, each of magnitude below 464, to e4m3 bytes (a in the lowest)
// with gfx950's v_cvt_pk_fp8_f32, two per instruction.  Over every float of
// magnitude below 464, both signs, the instruction (low- and high-word forms)
// gives exactly the bytes of f32_to_e4m3 above (an exhaustive check on the
// MI355X); absmax-scaled values (|v| <= 448) are always in that range.
__device__ __forceinline__ uint32_t f32x4_to_e4m3(float a, float b, float c, float d) {
    const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, lo, true);
}

// e4m3fn byte -> bf16 bits (exact).  NaN codes are not produced by absmax
// quantisation and are not expected here.
__device__ __forceinline__ uint32_t e4m3_to_bf16_bits(uint32_t q) {
    const uint32_t s = (q & 0x80u) << 8, e = (q >> 3) & 15u, m = q & 7u;
    const uint32_t mag = e ? (((e + 120u) << 7) | (m << 4)) : (__float_as_uint((float)m * 0x1p-9f) >> 16);
    return s | mag;
}

// Eight e4m3 bytes (little-endian in lo, hi) widened to the bf16x8 operand by
// gfx950's v_cvt_scalef32_pk_bf16_fp8 (two bytes per instruction, scale 1).
// Every e4m3 value is exact in bf16; a check of all 256 codes on the MI355X
// found the instruction bit-identical to e4m3_to_bf16_bits above except the
// two NaN codes, which the packers never produce (they saturate at 448).
__device__ __forceinline__ u32x4 widen_e4m3x8(uint32_t lo, uint32_t hi) {
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    u32x4 o;
    o[0] = __builtin_bit_cast(uint32_t, (bf16x2_t)__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, false));
    o[1] = __builtin_bit_cast(uint32_t, (bf16x2_t)__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(lo, 1.0f, true));
    o[2] = __builtin_bit_cast(uint32_t, (bf16x2_t)__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, false));
    o[3] = __builtin_bit_cast(uint32_t, (bf16x2_t)__builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(hi, 1.0f, true));
    return o;
}

// 16x16 fp32 += A(16 x 128 e4m3) . B(128 x 16 e4m3), unit block scales.
__device__ __forceinline__ f32x4 mfma_e4m3_16x16x128(const i32x8& a, const i32x8& b, f32x4 acc) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, acc, 0, 0, 0, 127, 0, 127);
}

// Workgroup-cooperative e4m3 quantisation of the 16 rank rows m0 .. m0+15 (r =
// R bf16 values each, row stride ld) into LDS: thread x handles row x/16 and
// the R/16 consecutive values from (x%16)*R/16.  Each row: amax = absmax,
// inv = 448 / amax, q = e4m3(v * inv), scale = amax / 448 (1 and zeros for an
// all-zero row; rows from m_valid on are zeros).  s_rq holds [16][R + 16]
// bytes (the pad spreads the operand reads over the banks), s_rsc [16].
// Ends with a barrier that waits for LDS traffic only, so loads in flight
// (the first streamed tiles) stay in flight.
template <int R>
__device__ __forceinline__ void quantize_rank_coop(const uint16_t* rows, int64_t ld, int m_valid, uint8_t* s_rq,
                                                   float* s_rsc) {
#pragma clang fp contract(off)
    constexpr int PER = R / 16;   // values per thread: 8, 16 or 32
    static_assert(PER % 8 == 0, "whole 16-byte pieces");
    const int m = threadIdx.x >> 4, seg = threadIdx.x & 15;
    const bool ok = m < m_valid;
    const uint16_t* src = rows + (int64_t)(ok ? m : 0) * ld + seg * PER;
    u32x4 raw[PER / 8];
#pragma unroll
    for (int i = 0; i < PER / 8; ++i) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(src + 8 * i);
        raw[i] = ok ? v : u32x4{0u, 0u, 0u, 0u};
    }
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < PER / 8; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            amax = __builtin_fmaxf(amax, __builtin_fabsf(__uint_as_float(raw[i][e] << 16)));
            amax = __builtin_fmaxf(amax, __builtin_fabsf(__uint_as_float(raw[i][e] & 0xffff0000u)));
        }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) amax = __builtin_fmaxf(amax, __shfl_xor(amax, off, 64));
    const float inv = amax > 0.f ? kE4M3Max / amax : 1.f;
#pragma unroll
    for (int i = 0; i < PER / 8; ++i) {
        uint32_t w[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t x0 = raw[i][2 * h], x1 = raw[i][2 * h + 1];
            w[h] = f32x4_to_e4m3(__uint_as_float(x0 << 16) * inv, __uint_as_float(x0 & 0xffff0000u) * inv,
                                 __uint_as_float(x1 << 16) * inv, __uint_as_float(x1 & 0xffff0000u) * inv);
        }
        *reinterpret_cast<u32x2*>(s_rq + m * (R + 16) + seg * PER + 8 * i) = u32x2{w[0], w[1]};
    }
    if (seg == 0) s_rsc[m] = amax > 0.f ? amax / kE4M3Max : 1.f;
    lds_barrier();
}

// The lane's e4m3 A operand (row lane%16, bytes 32*(lane/16) .. of each K128
// block) and the scales of its output rows 4*(lane/16) + q, from LDS.
template <int KS8>
__device__ __forceinline__ void load_rank_operand(const uint8_t* s_rq, const float* s_rsc, int lane,
                                                  i32x8 (&rq)[KS8], float (&rsc)[4]) {
    constexpr int R = KS8 * 128;
    const int col = lane & 15, kg = lane >> 4;
#pragma unroll
    for (int j = 0; j < KS8; ++j) {
        const uint8_t* p = s_rq + col * (R + 16) + 128 * j + 32 * kg;
        const u32x4 lo = *reinterpret_cast<const u32x4*>(p);
        const u32x4 hi = *reinterpret_cast<const u32x4*>(p + 16);
        rq[j] = i32x8{(int)lo[0], (int)lo[1], (int)lo[2], (int)lo[3], (int)hi[0], (int)hi[1], (int)hi[2], (int)hi[3]};
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) rsc[q] = s_rsc[4 * kg + q];
}

}  // namespace dels

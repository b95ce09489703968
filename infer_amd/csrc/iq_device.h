// iq_device.h -- device-side helpers shared by the gfx950 kernels of the
// quantized-weight path: bf16 bit conversions, register dequantisation of
// int8 / int4 codes into MFMA operands, and the MFMA wrappers.
//
// Dequantisation into fp16 MFMA operands uses exponent-bias constants, so a
// code costs about one VALU op:
//   int8:  byte b (two's complement) -> u = b ^ 0x80 in 0..255; fp16 bits
//          0x6400 | u encode exactly 1024 + u; subtracting 1152 leaves b.
//   int4:  nibble n in 0..15 -> fp16 bits 0x6400 | n = 1024 + n, or with the
//          nibble left in bits 4..7, 0x6400 | (n << 4) = 1024 + 16 n; a packed
//          add of -(1024 + z), or a packed fma by 1/16 then -(64 + z), leaves
//          n - z.  Every intermediate is an integer (or 64 + n) that fp16
//          holds exactly, so the MFMA sees the exact integer q - z.
// The group scale is applied to fp32 partial sums after the MFMAs, so the
// weights entering the matrix core are exact small integers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace iq {

constexpr int kGroup = 128;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(uint16_t b) {
    return __uint_as_float(uint32_t(b) << 16);
}

// src/f16.h:41-51 on the device: RNE, NaN forced quiet.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
    const uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x0040u);
    return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ half2_t as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t h2_bits(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// Four dwords (8 fp16 lanes of an MFMA operand) <-> half8.
__device__ __forceinline__ half8_t pack_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    u32x4_t v = {a, b, c, d};
    return __builtin_bit_cast(half8_t, v);
}

// int8: 4 codes (one dword, column order c..c+3) -> 2 dwords of half2 in the
// same column order, exact.
__device__ __forceinline__ void dq_int8_x4(uint32_t d, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = d ^ 0x80808080u;
    const uint32_t a = __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u);  // [u0,64,u1,64]
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u);  // [u2,64,u3,64]
    const half2_t bias = as_h2(0xE480E480u);                                 // -1152, -1152
    lo = h2_bits(as_h2(a) + bias);
    hi = h2_bits(as_h2(b) + bias);
}

// int4: 8 nibbles (one dword, columns c..c+7, low nibble first) -> 4 dwords
// of half2 holding q - z in column order [0,4 | 1,5 | 2,6 | 3,7].
// zb = -(1024+z) pair, zc = -(64+z) pair (fp16 bits, both halves equal).
__device__ __forceinline__ void dq_int4_x8(uint32_t v, uint32_t zb, uint32_t zc, uint32_t& o0,
                                           uint32_t& o1, uint32_t& o2, uint32_t& o3) {
    const half2_t sixteenth = as_h2(0x2C002C00u);  // 1/16, 1/16
    const uint32_t v8 = v >> 8;
    // (m & mask) | 0x6400 in each half: one v_bitop3_b32 each (truth table
    // 0xEA = (src0 & src1) | src2); written as & then | the compiler emits
    // two instructions, since one instruction takes at most one literal
    const uint32_t a0 = __builtin_amdgcn_bitop3_b32(v, 0x000F000Fu, 0x64006400u, 0xEA);   // 1024+n0, 1024+n4
    const uint32_t a1 = __builtin_amdgcn_bitop3_b32(v, 0x00F000F0u, 0x64006400u, 0xEA);   // 1024+16n1, 1024+16n5
    const uint32_t a2 = __builtin_amdgcn_bitop3_b32(v8, 0x000F000Fu, 0x64006400u, 0xEA);  // 1024+n2, 1024+n6
    const uint32_t a3 = __builtin_amdgcn_bitop3_b32(v8, 0x00F000F0u, 0x64006400u, 0xEA);  // 1024+16n3, 1024+16n7
    o0 = h2_bits(as_h2(a0) + as_h2(zb));
    o1 = h2_bits(__builtin_elementwise_fma(as_h2(a1), sixteenth, as_h2(zc)));
    o2 = h2_bits(as_h2(a2) + as_h2(zb));
    o3 = h2_bits(__builtin_elementwise_fma(as_h2(a3), sixteenth, as_h2(zc)));
}

// Zero-point constants for dq_int4_x8.
__device__ __forceinline__ uint32_t zpair_1024(uint32_t z) { return (0xE400u + z) * 0x00010001u; }
__device__ __forceinline__ uint32_t zpair_64(uint32_t z) { return (0xD400u + 16u * z) * 0x00010001u; }

// Position inside an 8-column octet of the int4 operand order above:
// operand slot i holds column perm8(i).
__host__ __device__ constexpr int perm8(int i) { return (i >> 1) + 4 * (i & 1); }

// D(16x16, fp32) += A(16x32, fp16) * B(32x16, fp16).
// Lane l supplies A[l%16][8*(l/16)+i] and B[8*(l/16)+i][l%16], i = 0..7,
// and holds D[4*(l/16)+r][l%16], r = 0..3.
__device__ __forceinline__ float4_t mfma16(half8_t a, half8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// D(32x32, fp32) += A(32x16, bf16) * B(16x32, bf16).
// Lane l supplies A[l%32][8*(l/32)+i] and B[8*(l/32)+i][l%32], i = 0..7,
// and holds D[8*(r/4) + 4*(l/32) + r%4][l%32], r = 0..15.
__device__ __forceinline__ float16_t mfma32_bf16(bf16x8_t a, bf16x8_t b, float16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

}  // namespace iq

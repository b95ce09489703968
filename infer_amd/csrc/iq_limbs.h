// iq_limbs.h -- the exact integer form of fp32 activations that the GEMV
// kernels multiply on the int8 matrix core, and the helpers they share
// (DPP row reductions, buffer resources, the per-group fp32 combination).
//
// Per (activation row, 128-column group): 2^k with max|x| * 2^k in
// [2^21, 2^22), X = rint(x * 2^k), written as three signed byte limbs
// X = 2^16 X0 + 2^8 X1 + X2 (one "limb record" of 3 x 128 bytes), plus a
// meta record {2^-k, sum X0, 256 sum X1 + sum X2}.  v_mfma_i32_16x16x64_i8
// then forms exact int32 sums of codes times limbs, and combine() turns a
// group's three sums into fp32 with one rounding.
#pragma once

#include "iq_internal.h"

namespace iq {

typedef int int4v_t __attribute__((ext_vector_type(4)));

constexpr int kMeta = kMaxRowsGemv;   // meta records per group (one per row slot)
constexpr int kLimbRec = 3 * kGroup;  // bytes of limbs per (row, group)

__device__ __forceinline__ int4v_t mfma_i8(int4v_t a, int4v_t b, int4v_t c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int4v_t u4_to_i4v(uint4 v) {
    return int4v_t{int(v.x), int(v.y), int(v.z), int(v.w)};
}

// Position of natural column c (0..127) inside a group's limb record.
//   int8 weights: natural order.
//   int4 weights: the lane owning bytes [16j, 16j+16) of a row's 64-byte
//   group splits them into even columns (low nibbles) and odd columns (high
//   nibbles); record = [even columns of j = 0..3 | odd columns of j = 0..3].
__host__ __device__ constexpr int limb_pos(int c, bool perm) {
    return perm ? (c & 1) * 64 + (c >> 5) * 16 + ((c & 31) >> 1) : c;
}

// ------------------------------------------------------------------ xprep
// Rotation of a value inside its 16-lane DPP row (row_ror:N).
template <int N>
__device__ __forceinline__ int row_ror(int v) {
    // bound_ctrl set: lets the compiler fold the move into the consumer
    // (v_add/v_max with a DPP operand); row_ror reads only valid lanes.
    return __builtin_amdgcn_update_dpp(0, v, 0x120 + N, 0xF, 0xF, true);
}
// All-reduce over the 16 lanes of a DPP row (4 rotations, no LDS traffic).
__device__ __forceinline__ int row16_sum(int v) {
    v += row_ror<8>(v);
    v += row_ror<4>(v);
    v += row_ror<2>(v);
    v += row_ror<1>(v);
    return v;
}
__device__ __forceinline__ float row16_max(float v) {
    v = fmaxf(v, __int_as_float(row_ror<8>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(row_ror<4>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(row_ror<2>(__float_as_int(v))));
    v = fmaxf(v, __int_as_float(row_ror<1>(__float_as_int(v))));
    return v;
}
__device__ __forceinline__ int row16_and(int v) {
    v &= row_ror<8>(v);
    v &= row_ror<4>(v);
    v &= row_ror<2>(v);
    v &= row_ror<1>(v);
    return v;
}

__device__ __forceinline__ uint32_t row16_or(uint32_t v) {
    v |= uint32_t(row_ror<8>(int(v)));
    v |= uint32_t(row_ror<4>(int(v)));
    v |= uint32_t(row_ror<2>(int(v)));
    v |= uint32_t(row_ror<1>(int(v)));
    return v;
}
__device__ __forceinline__ uint32_t row16_max_u32(uint32_t v) {
    v = max(v, uint32_t(row_ror<8>(int(v))));
    v = max(v, uint32_t(row_ror<4>(int(v))));
    v = max(v, uint32_t(row_ror<2>(int(v))));
    v = max(v, uint32_t(row_ror<1>(int(v))));
    return v;
}

// Three limb words (records 0, 1, 2 = X0, X1, X2) of the four values whose
// biased integers U = X + 0x808080 are u0..u3, in that byte order: limb L of
// a value is byte 2-L of U minus 128, i.e. that byte with its top bit flipped.
__device__ __forceinline__ void pack_limbs(uint32_t u0, uint32_t u1, uint32_t u2, uint32_t u3, uint32_t (&w)[3]) {
    const uint32_t p = __builtin_amdgcn_perm(u1, u0, 0x05010400u);   // u0.b0 u1.b0 u0.b1 u1.b1
    const uint32_t q = __builtin_amdgcn_perm(u3, u2, 0x05010400u);   // u2.b0 u3.b0 u2.b1 u3.b1
    const uint32_t p2 = __builtin_amdgcn_perm(u1, u0, 0x07030602u);  // u0.b2 u1.b2 ..
    const uint32_t q2 = __builtin_amdgcn_perm(u3, u2, 0x07030602u);  // u2.b2 u3.b2 ..
    w[0] = __builtin_amdgcn_perm(q2, p2, 0x05040100u) ^ 0x80808080u;
    w[1] = __builtin_amdgcn_perm(q, p, 0x07060302u) ^ 0x80808080u;
    w[2] = __builtin_amdgcn_perm(q, p, 0x05040100u) ^ 0x80808080u;
}

// Converts one (activation row, 128-column group) whose columns 8j..8j+7
// are v[] of the lane with j = lane % 16 (the 16 lanes of a DPP row hold the
// whole group; all 16 must call this together).  Writes this lane's limb
// bytes into the group's record `rec` (when `store`) and returns the group's
// meta record {2^-k as fp32 bits, sum X0, 256 sum X1 + sum X2, 0} (every lane).
//
// X = rint(x * 2^k) is formed as the bits of fma(x, 2^k, 1.5 * 2^23): with
// |x * 2^k| <= 2^22 the sum lies in [2^23, 2^24], where the float's bits
// minus those of 1.5 * 2^23 are X, rounded to nearest even by the fma.
// Adding 0x808080 makes each byte of the 24-bit result its limb + 128
// (balanced limbs in [-128, 127]).
template <bool PERM>
__device__ __forceinline__ int4 convert_group(const float (&v)[8], int j, bool store, int8_t* rec) {
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) am = fmaxf(am, __builtin_fabsf(v[i]));  // NaN ignored here
    const uint32_t mb = row16_max_u32(__float_as_uint(am));
    // amax = f * 2^E, f in [0.5, 1): k = 22 - E puts amax * 2^k in [2^21, 2^22)
    const int k0 = mb < 0x7F800000u ? 22 - __builtin_amdgcn_frexp_expf(__uint_as_float(mb)) : 0;
    int k = k0;
    float xv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) xv[i] = v[i];
    if (k > 126) {
        // amax below 2^-104: scale up exactly first so that 2^k stays a float
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = __builtin_amdgcn_ldexpf(xv[i], k - 126);
        k = 126;
    }
    const float p2k = __uint_as_float(uint32_t(k + 127) << 23);
    uint32_t u[8], hi = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        u[i] = __float_as_uint(__builtin_fmaf(xv[i], p2k, 12582912.0f)) + (0x808080u - 0x4B400000u);
        hi |= u[i];
    }
    // A finite group leaves byte 3 of every U zero; NaN / inf (either from
    // the input or, for a group whose amax is inf, from the scaling) do not.
    const bool fin = row16_or(hi >> 24) == 0;
    uint32_t a[3], b[3];
    if (PERM) {
        // columns 8j..8j+7: evens -> one word per limb, odds -> one word per limb
        pack_limbs(u[0], u[2], u[4], u[6], a);
        pack_limbs(u[1], u[3], u[5], u[7], b);
    } else {
        pack_limbs(u[0], u[1], u[2], u[3], a);
        pack_limbs(u[4], u[5], u[6], u[7], b);
    }
    int sl[3];
#pragma unroll
    for (int L = 0; L < 3; L++)
        sl[L] = row16_sum(__builtin_amdgcn_sdot4(int(a[L]), 0x01010101, __builtin_amdgcn_sdot4(int(b[L]), 0x01010101, 0, false), false));
    if (store) {
        if (PERM) {
            const int pe = limb_pos(j * 8, true), po = limb_pos(j * 8 + 1, true);
#pragma unroll
            for (int L = 0; L < 3; L++) {
                *reinterpret_cast<uint32_t*>(rec + L * kGroup + pe) = a[L];
                *reinterpret_cast<uint32_t*>(rec + L * kGroup + po) = b[L];
            }
        } else {
#pragma unroll
            for (int L = 0; L < 3; L++) *reinterpret_cast<uint2*>(rec + L * kGroup + j * 8) = make_uint2(a[L], b[L]);
        }
    }
    // 2^-k (NaN when the group holds a non-finite value, so it propagates)
    const float fx = fin ? __builtin_amdgcn_ldexpf(1.0f, -k0) : __builtin_nanf("");
    return make_int4(__float_as_int(fx), sl[0], (sl[1] << 8) + sl[2], 0);
}

// fp32 value of one group's exact integer limb sums (t_L = S_L - z * sum X_L;
// md = {2^-k, sum X0, 256 sum X1 + sum X2}, 24-bit multiplies: |z| <= 15,
// |256 sum X1 + sum X2| < 2^23), times the weight scale and the activation
// factor 2^-k, added to acc.
__device__ __forceinline__ float combine(float acc, int d0, int d1, int d2, int z, int4 md, float s) {
    // hi = t0, lo = 256 t1 + t2 exactly in int32 (|lo| < 2^30); float(lo)
    // rounds once, as fma(t1, 256, t2) would
    const int hi = d0 - __mul24(z, md.y);
    const int lo = (d1 << 8) + d2 - __mul24(z, md.z);
    const float v = __builtin_fmaf(float(hi), 65536.0f, float(lo));
    return __builtin_fmaf(v, s * __int_as_float(md.x), acc);
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;
constexpr uint32_t kOob = 0x80000000u;  // added to a buffer offset: reads zero, no memory access

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}

// make_rsrc for a base and size that are the same in every lane of the wave
// but derived from values the compiler cannot prove uniform (a tile picked
// out of a kernel-argument table): taken from the first lane, so the
// resource lives in scalar registers.  A per-lane resource compiles to a
// loop over its distinct values around every load that uses it.
__device__ __forceinline__ rsrc_t make_rsrc_wave(const void* base, int64_t bytes) {
    const uint64_t b = reinterpret_cast<uint64_t>(base);
    const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(b));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(b >> 32));
    const int n = __builtin_amdgcn_readfirstlane(int(bytes));
    return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>((uint64_t(hi) << 32) | lo), 0, n, 0x00020000);
}

// sum over s < S of part[s * stride + i], added in order of s: the requests
// go out eight slices at a time through a buffer resource over the S
// slices (slots past S read zero and are not added), so S slices cost about
// S / 8 memory latencies instead of S.  Bit-identical to the plain loop.
__device__ __forceinline__ float sum_slices(const float* part, int S, int64_t stride, int64_t i) {
    const rsrc_t r = make_rsrc(part, int64_t(S) * stride * 4);
    float sum = 0.0f;
    for (int s0 = 0; s0 < S; s0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t off = s0 + j < S ? uint32_t((int64_t(s0 + j) * stride + i) * 4) : kOob;
            v[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (s0 + j < S) sum += v[j];
    }
    return sum;
}

}  // namespace iq

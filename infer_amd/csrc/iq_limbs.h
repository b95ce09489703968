// iq_limbs.h -- the exact integer form of fp32 activations that the GEMV
// kernels multiply on the int8 matrix core, and the helpers they share
// (DPP row reductions, buffer resources, the per-group fp32 combination).
//
// Per (activation row, 128-column group): 2^k with max|x| * 2^k in
// (2^30, 0x7F7F7F7F] (k the largest power that fits; 30 or 31 significant
// bits), X = rint(x * 2^k), written as four signed byte limbs
// X = 2^24 X0 + 2^16 X1 + 2^8 X2 + X3 (one "limb record" of 4 x 128 bytes),
// plus a meta record {2^-k, 256 sum X0 + sum X1, 256 sum X2 + sum X3}.
// v_mfma_i32_16x16x64_i8 then forms exact int32 sums of codes times limbs,
// and combine() turns a group's four sums into fp32.
#pragma once

#include "iq_internal.h"

namespace iq {

typedef int int4v_t __attribute__((ext_vector_type(4)));

constexpr int kMeta = kMaxRowsGemv;   // meta records per group (one per row slot)
constexpr int kLimbs = 4;                // byte limbs per activation value
constexpr int kLimbRec = kLimbs * kGroup;  // bytes of limbs per (row, group)

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

// Four limb words (records 0..3 = X0..X3) of the four values whose biased
// integers U = X + 0x80808080 are u0..u3, in that byte order: limb L of a
// value is byte 3-L of U minus 128, i.e. that byte with its top bit flipped.
__device__ __forceinline__ void pack_limbs(uint32_t u0, uint32_t u1, uint32_t u2, uint32_t u3, uint32_t (&w)[kLimbs]) {
    const uint32_t p = __builtin_amdgcn_perm(u1, u0, 0x05010400u);   // u0.b0 u1.b0 u0.b1 u1.b1
    const uint32_t q = __builtin_amdgcn_perm(u3, u2, 0x05010400u);   // u2.b0 u3.b0 u2.b1 u3.b1
    const uint32_t p2 = __builtin_amdgcn_perm(u1, u0, 0x07030602u);  // u0.b2 u1.b2 u0.b3 u1.b3
    const uint32_t q2 = __builtin_amdgcn_perm(u3, u2, 0x07030602u);  // u2.b2 u3.b2 u2.b3 u3.b3
    w[0] = __builtin_amdgcn_perm(q2, p2, 0x07060302u) ^ 0x80808080u;
    w[1] = __builtin_amdgcn_perm(q2, p2, 0x05040100u) ^ 0x80808080u;
    w[2] = __builtin_amdgcn_perm(q, p, 0x07060302u) ^ 0x80808080u;
    w[3] = __builtin_amdgcn_perm(q, p, 0x05040100u) ^ 0x80808080u;
}

// Largest biased magnitude four balanced byte limbs hold: 127 * 0x01010101.
constexpr float kLimbMaxMant = 16711422.0f;  // 0x7F7F7F7F / 128, rounded down (0xFEFEFE)

// Converts one (activation row, 128-column group) whose columns 8j..8j+7
// are v[] of the lane with j = lane % 16 (the 16 lanes of a DPP row hold the
// whole group; all 16 must call this together).  Writes this lane's limb
// bytes into the group's record `rec` (when `store`) and returns the group's
// meta record {2^-k as fp32 bits, 256 sum X0 + sum X1, 256 sum X2 + sum X3, 0}
// (every lane).
//
// amax = f 2^E with f in [0.5, 1): k = 31 - E puts amax 2^k = f 2^31 in
// [2^30, 2^31); when f 2^31 would pass 0x7F7F7F7F (the largest value four
// balanced limbs hold, f 2^24 > 0xFEFEFE) k is one less.  x 2^k is exact
// and rint() rounds it once: |x 2^k - X| <= 1/2, at most 2^-30 of the
// group's largest |x|.  Adding 0x80808080 makes each byte of X its limb +
// 128 (balanced limbs in [-128, 127]).
template <bool PERM>
__device__ __forceinline__ int4 convert_group(const float (&v)[8], int j, bool store, int8_t* rec) {
    uint32_t ab = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t a = __float_as_uint(v[i]) & 0x7FFFFFFFu;  // NaN / inf sort above every finite value
        ab = a > ab ? a : ab;
    }
    const uint32_t mb = row16_max_u32(ab);
    const bool fin = mb < 0x7F800000u;
    const float amax = fin ? __uint_as_float(mb) : 1.0f;
    const int k0 = 31 - __builtin_amdgcn_frexp_expf(amax) -
                   (__builtin_amdgcn_frexp_mantf(amax) * 16777216.0f > kLimbMaxMant ? 1 : 0);
    int k = k0;
    float xv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) xv[i] = v[i];
    if (k > 126) {
        // amax below 2^-95: scale up exactly first so that 2^k stays a float
#pragma unroll
        for (int i = 0; i < 8; i++) xv[i] = __builtin_amdgcn_ldexpf(xv[i], k - 126);
        k = 126;
    }
    const float p2k = __uint_as_float(uint32_t(k + 127) << 23);
    uint32_t u[8];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        // (a non-finite group's integers are never used: its factor is NaN)
        const float r = fin ? __builtin_rintf(xv[i] * p2k) : 0.0f;
        u[i] = uint32_t(int(r)) + 0x80808080u;
    }
    uint32_t a[kLimbs], b[kLimbs];
    if (PERM) {
        // columns 8j..8j+7: evens -> one word per limb, odds -> one word per limb
        pack_limbs(u[0], u[2], u[4], u[6], a);
        pack_limbs(u[1], u[3], u[5], u[7], b);
    } else {
        pack_limbs(u[0], u[1], u[2], u[3], a);
        pack_limbs(u[4], u[5], u[6], u[7], b);
    }
    int sl[kLimbs];
#pragma unroll
    for (int L = 0; L < kLimbs; L++)
        sl[L] = row16_sum(__builtin_amdgcn_sdot4(int(a[L]), 0x01010101, __builtin_amdgcn_sdot4(int(b[L]), 0x01010101, 0, false), false));
    if (store) {
        if (PERM) {
            const int pe = limb_pos(j * 8, true), po = limb_pos(j * 8 + 1, true);
#pragma unroll
            for (int L = 0; L < kLimbs; L++) {
                *reinterpret_cast<uint32_t*>(rec + L * kGroup + pe) = a[L];
                *reinterpret_cast<uint32_t*>(rec + L * kGroup + po) = b[L];
            }
        } else {
#pragma unroll
            for (int L = 0; L < kLimbs; L++) *reinterpret_cast<uint2*>(rec + L * kGroup + j * 8) = make_uint2(a[L], b[L]);
        }
    }
    // 2^-k (NaN when the group holds a non-finite value, so it propagates)
    const float fx = fin ? __builtin_amdgcn_ldexpf(1.0f, -k0) : __builtin_nanf("");
    return make_int4(__float_as_int(fx), (sl[0] << 8) + sl[1], (sl[2] << 8) + sl[3], 0);
}

// fp32 value of one group's exact integer limb sums (t_L = S_L - z sum X_L;
// md = {2^-k, 256 sum X0 + sum X1, 256 sum X2 + sum X3}, 24-bit multiplies:
// |z| <= 15 and both limb-sum pairs are below 2^23), times the weight scale
// and the activation factor 2^-k, added to acc.  hi = 256 t0 + t1 and
// lo = 256 t2 + t3 are exact in int32 (|t_L| <= 128 * 127 * 128 < 2^21):
// the group's value 65536 hi + lo is rounded to fp32 with an error of a few
// ulps of the group's partial sum.
__device__ __forceinline__ float combine(float acc, int d0, int d1, int d2, int d3, int z, int4 md, float s) {
    const int hi = (d0 << 8) + d1 - __mul24(z, md.y);
    const int lo = (d2 << 8) + d3 - __mul24(z, md.z);
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

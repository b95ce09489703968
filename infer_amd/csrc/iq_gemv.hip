// iq_gemv.hip -- dequant GEMV for 1..32 activation rows on gfx950 int8 MFMA.
//
// Replaces the reference's gemv_q_direct_kernel / gemv_batched_q_kernel
// (kernels/ops/quant.cu:71-252) and their dispatch (quant.cu:312-345).
// Semantics: y[m,n] = sum_k dequant(W,n,k) * x[m,k] (+ bias[n]),
// dequant = s * q (int8) or s * (q - z) (int4), s a bf16 scale per
// 128-column group (src/quant.cpp:86-93).
//
// The weight codes are integers, so the matrix core multiplies them as
// integers: v_mfma_i32_16x16x64_i8.  The fp32 activations are turned into
// integers once per call (xprep):
//   per (activation row m, 128-column group g): 2^k with
//   max|x| * 2^k in [2^21, 2^22), X = rint(x * 2^k) (exact scaling, one
//   rounding: |x*2^k - X| <= 1/2, i.e. 2^-22 of the group's max), and X is
//   written as three signed byte limbs, X = 2^16 X0 + 2^8 X1 + X2.
// The GEMV then forms, per (row tile, group), three exact int32 sums
//   S_L = sum_k q_k * X_L,k        (L = 0, 1, 2; 6 MFMAs per 128 columns)
// and for int4 subtracts the zero point exactly in integers,
//   T_L = S_L - z * sum_k X_L,k    (the limb sums come with the limbs),
// so the only floating-point steps are
//   acc += ldexp(s * (65536 T_0 + 256 T_1 + T_2), -k)       (fp32).
// The int8 codes go to the MFMA untouched; int4 nibbles need one AND (even
// columns) or one shift + AND (odd columns) per 4 codes.
//
// Accuracy: the activation rounding is at most 2^-22 of the group's largest
// |x| per element, products and sums are exact integers, and the fp32
// combination adds a few ulps: far inside the reference's 5e-6 of the
// conditioning sum |w*x| (tests/test_ops_gpu.cu:199-206).  Non-finite
// activations make the affected outputs NaN.
//
// Two kernels:
//  * gemv1 (1 row, the decode step): workgroup = W waves on one tile of 16
//    output rows, the waves split K (reduced through LDS, deterministic; no
//    cross-workgroup traffic).  A wave requests all weight words, scales and
//    zero points of a batch of groups before it waits, stages the batch's
//    activation limbs in its own LDS slot and runs the MFMAs.
//  * gemv (2..32 rows): workgroup = 4 waves x R tiles of 16 rows on one slice
//    of K; the slice's activation limbs are staged once per workgroup in
//    LDS and shared by all 4R tiles.  Slices are split across workgroups
//    when the matrix is too short to fill the GPU; the last workgroup of a
//    row block adds the slice partials in slice order (deterministic) and
//    resets its counter, so no clearing is needed between launches.
#include <cstdlib>

#include "iq_internal.h"

namespace iq {

namespace {

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
    return __builtin_amdgcn_mov_dpp(v, 0x120 + N, 0xF, 0xF, false);
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

// Converts one (activation row, 128-column group) whose columns 8j..8j+7
// are v[] of the lane with j = lane % 16 (the 16 lanes of a DPP row hold the
// whole group; all 16 must call this together).  Writes this lane's limb
// bytes into the group's record `rec` (when `store`) and returns the group's
// meta record {2^-k as fp32 bits, sum X0, sum X1, sum X2} (every lane).
template <bool PERM>
__device__ __forceinline__ int4 convert_group(const float (&v)[8], int j, bool store, int8_t* rec) {
    // absmax; NaN must not be lost (fmaxf drops it), so track finiteness apart.
    float amax = 0.0f;
    int fin = 1;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float a = __builtin_fabsf(v[i]);
        fin &= int(a <= 3.402823466e38f);
        amax = fmaxf(amax, a);
    }
    amax = row16_max(amax);
    fin = row16_and(fin);
    // amax = f * 2^E, f in [0.5, 1): k = 22 - E puts amax * 2^k in [2^21, 2^22)
    const int k = (fin && amax > 0.0f) ? 22 - __builtin_amdgcn_frexp_expf(amax) : 0;
    int X[8];
#pragma unroll
    for (int i = 0; i < 8; i++) X[i] = fin ? int(__builtin_rintf(__builtin_amdgcn_ldexpf(v[i], k))) : 0;
    // balanced byte limbs: X = 2^16 x0 + 2^8 x1 + x2, each in [-128, 127]
    int l0[8], l1[8], l2[8];
    int s0 = 0, s1 = 0, s2 = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const int a2 = int(int8_t(X[i] & 0xFF));
        const int r1 = (X[i] - a2) >> 8;
        const int a1 = int(int8_t(r1 & 0xFF));
        const int a0 = (r1 - a1) >> 8;
        l0[i] = a0; l1[i] = a1; l2[i] = a2;
        s0 += a0; s1 += a1; s2 += a2;
    }
    s0 = row16_sum(s0);
    s1 = row16_sum(s1);
    s2 = row16_sum(s2);
    if (store) {
        const int* L[3] = {l0, l1, l2};
        if (PERM) {
            // columns 8j..8j+7: evens -> 4 contiguous bytes, odds -> 4 contiguous bytes
            const int pe = limb_pos(j * 8, true), po = limb_pos(j * 8 + 1, true);
#pragma unroll
            for (int li = 0; li < 3; li++) {
                uint32_t ev = 0, od = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    ev |= uint32_t(uint8_t(L[li][2 * e])) << (8 * e);
                    od |= uint32_t(uint8_t(L[li][2 * e + 1])) << (8 * e);
                }
                *reinterpret_cast<uint32_t*>(rec + li * kGroup + pe) = ev;
                *reinterpret_cast<uint32_t*>(rec + li * kGroup + po) = od;
            }
        } else {
#pragma unroll
            for (int li = 0; li < 3; li++) {
                uint32_t lo = 0, hi = 0;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    lo |= uint32_t(uint8_t(L[li][e])) << (8 * e);
                    hi |= uint32_t(uint8_t(L[li][e + 4])) << (8 * e);
                }
                *reinterpret_cast<uint2*>(rec + li * kGroup + j * 8) = make_uint2(lo, hi);
            }
        }
    }
    // 2^-k (NaN when the group holds a non-finite value, so it propagates);
    // a group of values below ~2^-149 * 2^22 contributes 0.
    const float fx = fin ? __builtin_amdgcn_ldexpf(1.0f, -k) : __builtin_nanf("");
    return make_int4(__float_as_int(fx), s0, s1, s2);
}

// Columns [c0, c0 + 8) of an activation row, zero past K.
template <bool VECX>
__device__ __forceinline__ void load_x8(const float* xr, int64_t c0, int64_t K, float (&v)[8]) {
    if (VECX && c0 + 8 <= K) {
        const float4 a = *reinterpret_cast<const float4*>(xr + c0);
        const float4 b = *reinterpret_cast<const float4*>(xr + c0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = c0 + i < K ? xr[c0 + i] : 0.0f;
    }
}

// One wave per (row, 4 groups); 16 lanes (one DPP row) per group, 8 columns
// per lane.
template <bool PERM, bool VECX>
__global__ __launch_bounds__(256) void xprep_kernel(const float* __restrict__ x, int M, int64_t K,
                                                    int64_t G, int64_t quads,
                                                    int8_t* __restrict__ xq, int4* __restrict__ meta) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (wave >= int64_t(M) * quads) return;
    const int m = int(wave / quads);
    const int64_t g = (wave % quads) * 4 + (lane >> 4);
    const bool gvalid = g < G;
    const int j = lane & 15;
    float v[8];
    load_x8<VECX>(x + int64_t(m) * K, (gvalid ? g : 0) * kGroup + j * 8, gvalid ? K : 0, v);
    const int4 md = convert_group<PERM>(v, j, gvalid, xq + (int64_t(m) * G + (gvalid ? g : 0)) * kLimbRec);
    if (gvalid && j == 0) meta[g * kMeta + m] = md;
}

// ------------------------------------------------------------------ shared pieces
constexpr int kMaxMulti = 4;  // matrices sharing one activation in one 1-row launch

// One matrix of a multi-matrix 1-row launch: its 16-row tiles are the
// workgroups [tile0, tile0 + ceil(N/16)).
struct MatRef {
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
    const uint16_t* bias;
    float* y;
    int64_t N;
    int tile0;
};

struct GemvParams {
    MatRef mat[kMaxMulti];
    int nmat;
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
    int64_t N, K, G;
    const float* x;  // fp32 activation row (1-row kernel)
    const int8_t* xq;
    const int4* meta;
    const uint16_t* bias;
    float* y;
    float* part;
    int M, S, gs, nrb;
};

// 16 bytes of a row at byte offset `off`, zero past `row_bytes` (unaligned
// rows / ragged tails; test shapes only).
__device__ __forceinline__ uint4 load16_slow(const uint8_t* row, int64_t off, int64_t row_bytes) {
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 16; i++)
        if (off + i < row_bytes) w[i / 4] |= uint32_t(row[off + i]) << (8 * (i % 4));
    return make_uint4(w[0], w[1], w[2], w[3]);
}

// The two B operands (k-steps of 64 columns) of one lane for one group.
//   int8: the two 16-byte loads as they are.
//   int4: the one 16-byte load split into low nibbles (even columns) and
//   high nibbles (odd columns), one byte per code.
template <int KIND>
__device__ __forceinline__ void weight_operands(const uint4* w, int4v_t& b0, int4v_t& b1) {
    if (KIND == 1) {
        const uint4 v = w[0];
        b0 = int4v_t{int(v.x & 0x0F0F0F0Fu), int(v.y & 0x0F0F0F0Fu), int(v.z & 0x0F0F0F0Fu), int(v.w & 0x0F0F0F0Fu)};
        b1 = int4v_t{int((v.x >> 4) & 0x0F0F0F0Fu), int((v.y >> 4) & 0x0F0F0F0Fu),
                     int((v.z >> 4) & 0x0F0F0F0Fu), int((v.w >> 4) & 0x0F0F0F0Fu)};
    } else {
        b0 = u4_to_i4v(w[0]);
        b1 = u4_to_i4v(w[1]);
    }
}

// fp32 value of one group's exact integer limb sums (t_L = S_L - z * sum X_L,
// computed with 24-bit multiplies: |z| <= 15, |sum X_L| < 2^15), times the
// weight scale and the activation factor 2^-k, added to acc.
__device__ __forceinline__ float combine(float acc, int d0, int d1, int d2, int z, int4 md, float s) {
    const int t0 = d0 - __mul24(z, md.y), t1 = d1 - __mul24(z, md.z), t2 = d2 - __mul24(z, md.w);
    const float v = __builtin_fmaf(float(t0), 65536.0f, __builtin_fmaf(float(t1), 256.0f, float(t2)));
    return __builtin_fmaf(v, s * __int_as_float(md.x), acc);
}

// ------------------------------------------------------------------ 1 row
// Weight words + scales + zero points of one batch of GB groups of a lane.
template <int KIND, int GB>
struct WBatch {
    static constexpr int WPG = KIND == 1 ? 1 : 2;
    uint4 w[GB][WPG];
    uint2 s[GB / 4];     // 4 bf16 scales per entry
    uint32_t z[GB / 4];  // 4 zero points per entry (int4)
};

// Loads batch [g0, g0 + GB) of one lane (columns of the lane's quarter of
// each group); groups at or past `gend` re-load group gend-1 (the compute
// skips them), so every load is unconditional and stays in bounds.
// MODE 0: unaligned rows (byte loads); 1: 16-byte weight loads, one scale /
// zero load per group; 2: also one 8-byte scale and one 4-byte zero-point
// load per 4 groups (G % 4 == 0, slices of whole 4-group blocks).
template <int KIND, int GB, int MODE>
__device__ __forceinline__ void load_batch(WBatch<KIND, GB>& b, const uint8_t* qrow, const uint16_t* srow,
                                           const uint8_t* zrow, int g0, int gend, int kg,
                                           int row_bytes) {
    constexpr int WPG = WBatch<KIND, GB>::WPG;
#pragma unroll
    for (int gl = 0; gl < GB; gl++) {
        const int g = g0 + gl < gend ? g0 + gl : gend - 1;
#pragma unroll
        for (int h = 0; h < WPG; h++) {
            const int off = KIND == 1 ? g * 64 + kg * 16 : g * 128 + h * 64 + kg * 16;
            b.w[gl][h] = MODE >= 1 ? *reinterpret_cast<const uint4*>(qrow + off) : load16_slow(qrow, off, row_bytes);
        }
    }
#pragma unroll
    for (int q4 = 0; q4 < GB / 4; q4++) {
        if (MODE == 2) {
            // gend is a multiple of 4 here (G % 4 == 0 and gs % 4 == 0)
            const int g = g0 + 4 * q4 < gend ? g0 + 4 * q4 : gend - 4;
            b.s[q4] = *reinterpret_cast<const uint2*>(srow + g);
            b.z[q4] = KIND == 1 ? *reinterpret_cast<const uint32_t*>(zrow + g) : 0u;
        } else {
            uint32_t s4[4], z4 = 0;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int g = g0 + 4 * q4 + e < gend ? g0 + 4 * q4 + e : gend - 1;
                s4[e] = srow[g];
                if (KIND == 1) z4 |= uint32_t(zrow[g]) << (8 * e);
            }
            b.s[q4] = make_uint2(s4[0] | (s4[1] << 16), s4[2] | (s4[3] << 16));
            b.z[q4] = z4;
        }
    }
}

// One activation row (the decode step).  Workgroup = TW x KS waves: TW tiles
// of 16 output rows, each tile's K split into KS slices (wave = one tile,
// one slice of gs <= NB*GB groups).  Every weight word, scale and zero point
// of a wave's slice is requested at kernel start (NB batches of GB groups,
// all loads unconditional - clamped into the slice - so nothing waits before
// the last one is issued).  The fp32 activations of the wave's slice are
// requested before the weights, and converted to byte limbs (as xprep does)
// into the workgroup's LDS copy of the row while the weight words are in
// flight: no separate conversion launch.  With KS > 1 the slice partials of
// a tile are added through LDS in slice order (deterministic): no
// cross-workgroup traffic, no device-scope fence.  The A operand carries the
// activation's three byte limbs as rows 0..2 of the 16-row MFMA tile (lanes
// l%16 = 0, 1, 2; the other lanes read a zero block, no branches), so two
// MFMAs per 128 columns yield all three exact limb sums, in D rows 0..2 of
// lanes 0..15.  MODE: see load_batch (MODE >= 1 also means K % 128 == 0 and
// a 16-byte aligned activation row).
template <int KIND, int TW, int KS, int GB, int NB, int MODE>
__global__ __launch_bounds__(64 * TW * KS) void gemv1_kernel(const GemvParams p) {
    constexpr int W = TW * KS;
    constexpr int XP = NB * GB / 4;  // conversion passes of 4 groups per wave
    extern __shared__ __attribute__((aligned(16))) int8_t xs1[];  // limbs [G][384], meta [G]
    __shared__ __attribute__((aligned(16))) int8_t xzero[16];
    __shared__ float red[W][16];
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, kg = lane >> 4, wave = tid >> 6;
    static_assert(TW == 1, "one tile per workgroup");
    const int ksl = wave;
    const int G = int(p.G);
    int mi = 0;
#pragma unroll
    for (int i = 1; i < kMaxMulti; i++)
        if (i < p.nmat && int(blockIdx.x) >= p.mat[i].tile0) mi = i;
    const MatRef& mr = p.mat[mi];
    const int64_t row = (int64_t(blockIdx.x) - mr.tile0) * 16 + ln;
    const int64_t rc = row < mr.N ? row : mr.N - 1;
    const int row_bytes = int(KIND == 1 ? p.K / 2 : p.K);
    const uint8_t* qrow = mr.q + rc * row_bytes;
    const uint16_t* srow = mr.scales + rc * G;
    const uint8_t* zrow = KIND == 1 ? mr.zeros + rc * G : nullptr;
    const int gbeg = ksl * p.gs < G ? ksl * p.gs : G;
    const int gend = gbeg + p.gs < G ? gbeg + p.gs : G;
    const bool active = gend > gbeg;
    // Clamp bound for idle waves (their loads re-read groups 0..3, in bounds;
    // the 4-group scale loads need a bound of at least 4).
    const int g0c = active ? gbeg : 0;
    const int gcl = active ? gend : (MODE == 2 ? 4 : 1);
    int4* ms1 = reinterpret_cast<int4*>(xs1 + G * kLimbRec);

    // 1. The slice's activations: pass t converts groups gbeg + 4t + kg,
    //    16 lanes (one DPP row) per group, 8 columns per lane.  Loads are
    //    clamped to the slice (idle waves: group 0), stores are masked.
    float xv[XP][8];
#pragma unroll
    for (int t = 0; t < XP; t++) {
        const int g = g0c + 4 * t + kg < gcl ? g0c + 4 * t + kg : gcl - 1;
        load_x8<MODE >= 1>(p.x, int64_t(g) * kGroup + ln * 8, p.K, xv[t]);
    }
    if (tid < 4) reinterpret_cast<uint32_t*>(xzero)[tid] = 0u;

    // 2. All weight batches of the slice.
    WBatch<KIND, GB> wb[NB];
#pragma unroll
    for (int bi = 0; bi < NB; bi++) load_batch<KIND, GB, MODE>(wb[bi], qrow, srow, zrow, g0c + bi * GB, gcl, kg, row_bytes);

    // 3. Convert (the weights stay in flight).
#pragma unroll
    for (int t = 0; t < XP; t++) {
        const int g = gbeg + 4 * t + kg;
        if (gbeg + 4 * t >= gend) break;  // wave-uniform
        const bool st = g < gend;
        const int4 md = convert_group<KIND == 1>(xv[t], ln, st, xs1 + (st ? g : gbeg) * kLimbRec);
        if (st && ln == 0) ms1[g] = md;
    }
    __syncthreads();

    // 3. Per batch: all activation operands, then all MFMAs, then the fp32
    //    combination (independent chains, so LDS / MFMA latencies overlap).
    float acc = 0.0f;
#pragma unroll
    for (int bi = 0; bi < NB; bi++) {
        // A operand rows 0, 1, 2 = the activation's three limbs (lanes with
        // l%16 = L), rows 3..15 zero: one MFMA per 64 columns gives all three
        // exact limb sums, in D rows 0..2 of lanes 0..15.
        int4v_t a[GB][2];
#pragma unroll
        for (int gl = 0; gl < GB; gl++) {
            const int g = gbeg + bi * GB + gl < gend ? gbeg + bi * GB + gl : gbeg;
#pragma unroll
            for (int st = 0; st < 2; st++) {
                const int8_t* pa = ln < 3 ? xs1 + g * kLimbRec + ln * kGroup + st * 64 + kg * 16 : xzero;
                a[gl][st] = *reinterpret_cast<const int4v_t*>(pa);
            }
        }
        int4v_t D[GB];
#pragma unroll
        for (int gl = 0; gl < GB; gl++) {
            int4v_t b0, b1;
            weight_operands<KIND>(wb[bi].w[gl], b0, b1);
            D[gl] = mfma_i8(a[gl][0], b0, int4v_t{0, 0, 0, 0});
            D[gl] = mfma_i8(a[gl][1], b1, D[gl]);
        }
#pragma unroll
        for (int gl = 0; gl < GB; gl++) {
            const int g = gbeg + bi * GB + gl;
            if (g >= gend) break;
            const uint32_t sw = (gl & 2) ? wb[bi].s[gl / 4].y : wb[bi].s[gl / 4].x;
            const float s = __uint_as_float((gl & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
            const int z = KIND == 1 ? int((wb[bi].z[gl / 4] >> (8 * (gl & 3))) & 0xFF) : 0;
            acc = combine(acc, D[gl][0], D[gl][1], D[gl][2], z, ms1[g], s);
        }
    }
    if (KS == 1) {
        if (lane < 16 && row < mr.N) mr.y[row] = acc + (mr.bias ? bf16_to_f32(mr.bias[row]) : 0.0f);
        return;
    }
    if (lane < 16) red[wave][lane] = acc;
    __syncthreads();
    if (tid < 16) {
        const int64_t n = (int64_t(blockIdx.x) - mr.tile0) * 16 + tid;
        if (n < mr.N) {
            float sum = red[0][tid];
#pragma unroll
            for (int k = 1; k < KS; k++) sum += red[k][tid];
            mr.y[n] = sum + (mr.bias ? bf16_to_f32(mr.bias[n]) : 0.0f);
        }
    }
}

// ------------------------------------------------------------------ 2..32 rows
// Workgroup = 8 waves, wave w owns the 16-row tile (blockIdx.x % nrb) * 8 + w;
// the workgroup walks its K slice (groups [ks*gs, ks*gs + gs)) in chunks of
// GC groups.  Per chunk the activation limbs of all M rows are staged in LDS
// once and shared by the 8 tiles; the weight words of the next chunk and the
// activation limbs of the next chunk are in flight (registers) while the
// current chunk is multiplied.
//
// Activation rows on the MFMA A operand (16 rows):
//   ROWS4 (M <= 8): row 4*mm + L = limb L of activation row mt*4 + mm, so a
//     tile of 4 activation rows needs 2 MFMAs per 128 columns, and lane
//     (l%16 = n, l/16 = mm) ends with the 3 limb sums of one (row, n).
//   otherwise: A row i = activation row mt*16 + i, one MFMA per limb
//     (6 per 128 columns for 16 rows); D register r of limb L's MFMA holds
//     (row mt*16 + 4*(l/16) + r, n = l%16).
// With S > 1 slices (matrices too short to fill the GPU) each slice writes
// fp32 partial sums and gemv_reduce adds them in slice order (deterministic).
template <int KIND, bool ROWS4, int MT, int GC, bool VEC>
__global__ __launch_bounds__(512) void gemvb_kernel(const GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) int8_t xsb[];  // [GC][M][384] limbs, [GC][32] meta
    __shared__ __attribute__((aligned(16))) int8_t xzero[16];
    constexpr int NT = 512;
    constexpr int WPG = KIND == 1 ? 1 : 2;
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, kg = lane >> 4, wave = tid >> 6;
    const int G = int(p.G), M = p.M;
    const int ks = blockIdx.x / p.nrb, rb = blockIdx.x % p.nrb;
    const int gbeg = ks * p.gs < G ? ks * p.gs : G;
    const int gend = gbeg + p.gs < G ? gbeg + p.gs : G;
    const int nchunk = (gend - gbeg + GC - 1) / GC;
    const int64_t row0 = (int64_t(rb) * 8 + wave) * 16;
    const int64_t row = row0 + ln;
    const int64_t rc = row < p.N ? row : p.N - 1;
    const int row_bytes = int(KIND == 1 ? p.K / 2 : p.K);
    const uint8_t* qrow = p.q + rc * row_bytes;
    const uint16_t* srow = p.scales + rc * G;
    const uint8_t* zrow = KIND == 1 ? p.zeros + rc * G : nullptr;
    const int xrec = M * kLimbRec;                 // bytes of limbs per group (all rows)
    const int xch = GC * xrec / 16;                // 16-byte chunks per activation chunk
    int4* msb = reinterpret_cast<int4*>(xsb + GC * xrec);
    constexpr int XPT = (GC * kMaxRowsGemv * kLimbRec / 16 + NT - 1) / NT;  // max chunks per thread
    if (tid < 4) reinterpret_cast<uint32_t*>(xzero)[tid] = 0u;

    // register copies of one chunk: weights of this wave's tile, the
    // activation limbs / meta slice of this thread
    uint4 wcur[GC][WPG], wnxt[GC][WPG];
    int4v_t xr[XPT];
    int4v_t mr;
#define IQ_LOAD_W(W_, C_)                                                                               \
    do {                                                                                                \
        const int g0_ = gbeg + (C_) * GC;                                                               \
        _Pragma("unroll") for (int gl = 0; gl < GC; gl++) {                                             \
            const int g = g0_ + gl < gend ? g0_ + gl : gend - 1;                                        \
            _Pragma("unroll") for (int h = 0; h < WPG; h++) {                                           \
                const int off = KIND == 1 ? g * 64 + kg * 16 : g * 128 + h * 64 + kg * 16;              \
                W_[gl][h] = VEC ? *reinterpret_cast<const uint4*>(qrow + off) : load16_slow(qrow, off, row_bytes); \
            }                                                                                           \
        }                                                                                               \
    } while (0)
#define IQ_LOAD_X(C_)                                                                                   \
    do {                                                                                                \
        const int g0_ = gbeg + (C_) * GC;                                                               \
        const int ng_ = gend - g0_ < GC ? gend - g0_ : GC;                                              \
        const int lim_ = ng_ * xrec / 16;                                                               \
        _Pragma("unroll") for (int i = 0; i < XPT; i++) {                                               \
            const int t = tid + i * NT < lim_ ? tid + i * NT : lim_ - 1;                                \
            const int gl = t / (xrec / 16), rem = t % (xrec / 16);                                      \
            xr[i] = *reinterpret_cast<const int4v_t*>(p.xq + (int64_t(rem / 24) * G + g0_ + gl) * kLimbRec + (rem % 24) * 16); \
        }                                                                                               \
        mr = reinterpret_cast<const int4v_t*>(p.meta)[(g0_ + (tid / kMeta < ng_ ? tid / kMeta : ng_ - 1)) * kMeta + tid % kMeta]; \
    } while (0)
#define IQ_STORE_X(C_)                                                                                  \
    do {                                                                                                \
        const int g0_ = gbeg + (C_) * GC;                                                               \
        const int ng_ = gend - g0_ < GC ? gend - g0_ : GC;                                              \
        const int lim_ = ng_ * xrec / 16;                                                               \
        _Pragma("unroll") for (int i = 0; i < XPT; i++) {                                               \
            const int t = tid + i * NT < lim_ ? tid + i * NT : lim_ - 1; /* clamped: identical bytes */ \
            reinterpret_cast<int4v_t*>(xsb)[t] = xr[i];                                                 \
        }                                                                                               \
        const int gl_ = tid / kMeta < ng_ ? tid / kMeta : ng_ - 1;                                      \
        if (tid < GC * kMeta) reinterpret_cast<int4v_t*>(msb)[gl_ * kMeta + tid % kMeta] = mr;         \
    } while (0)

    constexpr int NACC = ROWS4 ? 1 : 4;
    float acc[MT][NACC];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < NACC; r++) acc[mt][r] = 0.0f;

    IQ_LOAD_X(0);
    IQ_LOAD_W(wcur, 0);
    IQ_LOAD_W(wnxt, 1 < nchunk ? 1 : 0);
    IQ_STORE_X(0);
    __syncthreads();
    for (int c = 0; c < nchunk; c++) {
        if (c + 1 < nchunk) IQ_LOAD_X(c + 1);
        const int g0 = gbeg + c * GC;
        const int ng = gend - g0 < GC ? gend - g0 : GC;
#pragma unroll
        for (int gl = 0; gl < GC; gl++) {
            if (gl >= ng) break;
            const int g = g0 + gl;
            int4v_t b0, b1;
            weight_operands<KIND>(wcur[gl], b0, b1);
            const uint32_t sw = srow[g];  // bf16 scale (L1/L2 hit after the first tile)
            const float s = __uint_as_float(sw << 16);
            const int z = KIND == 1 ? int(zrow[g]) : 0;
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                if (ROWS4) {
                    const int mm = ln >> 2, L = ln & 3, m = mt * 4 + mm;
                    int4v_t a[2];
#pragma unroll
                    for (int st = 0; st < 2; st++) {
                        const int8_t* pa = (L < 3 && m < M) ? xsb + (gl * M + m) * kLimbRec + L * kGroup + st * 64 + kg * 16 : xzero;
                        a[st] = *reinterpret_cast<const int4v_t*>(pa);
                    }
                    int4v_t D = mfma_i8(a[0], b0, int4v_t{0, 0, 0, 0});
                    D = mfma_i8(a[1], b1, D);
                    const int mo = mt * 4 + kg;  // activation row of this lane's D
                    if (mo < M) acc[mt][0] = combine(acc[mt][0], D[0], D[1], D[2], z, msb[gl * kMeta + mo], s);
                } else {
                    const int m = mt * 16 + ln;
                    int4v_t D[3];
#pragma unroll
                    for (int L = 0; L < 3; L++) {
                        int4v_t a[2];
#pragma unroll
                        for (int st = 0; st < 2; st++) {
                            const int8_t* pa = m < M ? xsb + (gl * M + m) * kLimbRec + L * kGroup + st * 64 + kg * 16 : xzero;
                            a[st] = *reinterpret_cast<const int4v_t*>(pa);
                        }
                        D[L] = mfma_i8(a[0], b0, int4v_t{0, 0, 0, 0});
                        D[L] = mfma_i8(a[1], b1, D[L]);
                    }
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        const int mo = mt * 16 + 4 * kg + r;
                        if (mo < M) acc[mt][r] = combine(acc[mt][r], D[0][r], D[1][r], D[2][r], z, msb[gl * kMeta + mo], s);
                    }
                }
            }
        }
        if (c + 1 < nchunk) {
#pragma unroll
            for (int gl = 0; gl < GC; gl++)
#pragma unroll
                for (int h = 0; h < WPG; h++) wcur[gl][h] = wnxt[gl][h];
            IQ_LOAD_W(wnxt, c + 2 < nchunk ? c + 2 : c + 1);
            __syncthreads();  // every wave is done with chunk c in LDS
            IQ_STORE_X(c + 1);
            __syncthreads();
        }
    }

#undef IQ_LOAD_W
#undef IQ_LOAD_X
#undef IQ_STORE_X
    // Epilogue: this lane's outputs (row, activation row) pairs.
    if (row >= p.N) return;
    const float b = p.bias ? bf16_to_f32(p.bias[row]) : 0.0f;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int r = 0; r < NACC; r++) {
            const int mo = ROWS4 ? mt * 4 + kg : mt * 16 + 4 * kg + r;
            if (ROWS4 && ln >= 16) continue;
            if (mo >= M) continue;
            if (p.S == 1) p.y[int64_t(mo) * p.N + row] = acc[mt][r] + b;
            else p.part[(int64_t(ks) * M + mo) * p.N + row] = acc[mt][r];
        }
}

// y[m, n] = sum over slices s of part[s, m, n] (in slice order) + bias[n].
__global__ __launch_bounds__(256) void gemv_reduce_kernel(const float* __restrict__ part, int S, int M, int64_t N,
                                                          const uint16_t* __restrict__ bias, float* __restrict__ y) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(M) * N) return;
    float sum = 0.0f;
    for (int s = 0; s < S; s++) sum += part[int64_t(s) * M * N + i];
    y[i] = sum + (bias ? bf16_to_f32(bias[i % N]) : 0.0f);
}

template <int KIND, int TW, int KS, int GB>
void launch_gemv1_s(const GemvParams& p, int nb, int mode, unsigned grid, size_t lds, hipStream_t stream) {
#define IQ_G1(NB)                                                                                  \
    do {                                                                                           \
        if (mode == 2) gemv1_kernel<KIND, TW, KS, GB, NB, 2><<<grid, 64 * TW * KS, lds, stream>>>(p); \
        else if (mode == 1) gemv1_kernel<KIND, TW, KS, GB, NB, 1><<<grid, 64 * TW * KS, lds, stream>>>(p); \
        else gemv1_kernel<KIND, TW, KS, GB, NB, 0><<<grid, 64 * TW * KS, lds, stream>>>(p);        \
    } while (0)
    switch (nb) {
        case 1: IQ_G1(1); break;
        case 2: IQ_G1(2); break;
        case 3: IQ_G1(3); break;
        default: IQ_G1(4); break;
    }
#undef IQ_G1
}

// Instantiated workgroup shapes: one tile, KS = 4, 8 or 16 slices.
template <int KIND, int GB>
void launch_gemv1_t(const GemvParams& p, int KS, int vec, unsigned grid, hipStream_t stream) {
    const size_t lds = size_t(p.G) * kLimbRec + size_t(p.G + 1) * 16;
    const int nb = (p.gs + GB - 1) / GB;
    if (KS == 4) launch_gemv1_s<KIND, 1, 4, GB>(p, nb, vec, grid, lds, stream);
    else if (KS == 8) launch_gemv1_s<KIND, 1, 8, GB>(p, nb, vec, grid, lds, stream);
    else launch_gemv1_s<KIND, 1, 16, GB>(p, nb, vec, grid, lds, stream);
}

template <int KIND, int GC>
void launch_gemvb_t(const GemvParams& p, bool vec, unsigned grid, size_t lds, hipStream_t stream) {
    const int M = p.M;
#define IQ_GB(R4, MT)                                                                         \
    do {                                                                                      \
        if (vec) gemvb_kernel<KIND, R4, MT, GC, true><<<grid, 512, lds, stream>>>(p);         \
        else gemvb_kernel<KIND, R4, MT, GC, false><<<grid, 512, lds, stream>>>(p);            \
    } while (0)
    if (M <= 4) IQ_GB(true, 1);
    else if (M <= 8) IQ_GB(true, 2);
    else if (M <= 16) IQ_GB(false, 1);
    else IQ_GB(false, 2);
#undef IQ_GB
}

int env_int(const char* name, int dflt) {
    const char* v = getenv(name);
    return v ? atoi(v) : dflt;
}

// MODE of the 1-row kernel (see load_batch): 16-byte paths need K % 128 == 0
// and a 16-byte aligned activation row.
int gemv1_mode(int64_t K, int64_t G, const float* x) {
    if (K % kGroup || reinterpret_cast<uintptr_t>(x) % 16) return 0;
    return G % 4 ? 1 : 2;
}

// Workgroup K-slices of the 1-row kernel: the smallest of 4, 8, 16 whose
// slices fit 4 weight batches (measured on MI355X: 4 slices beat more,
// smaller workgroups whenever they fit); 0 when the kernel does not apply
// (the LDS copy of the converted row would exceed 96 KiB).
int gemv1_slices(int64_t G, int kind, int mode) {
    if (G * (kLimbRec + 16) > 96 * 1024) return 0;
    const int gb1 = kind == 1 ? 8 : 4;  // groups per batch (8 KiB of weights per wave)
    for (int ks : {4, 8, 16}) {
        int gs = int((G + ks - 1) / ks);
        if (mode == 2) gs = (gs + 3) / 4 * 4;
        if (gs <= 4 * gb1) return ks;
    }
    return 0;
}

// The 1-row kernel on n <= kMaxMulti matrices of one kind and width: one grid,
// matrix i owns the workgroups [tile0_i, tile0_i + ceil(N_i / 16)).
hipError_t launch_gemv1(const float* x, const QView* W, const uint16_t* const* bias, float* const* y, int n,
                        int KS, int mode, hipStream_t stream) {
    const int64_t K = W[0].cols, G = W[0].groups;
    GemvParams p{};
    int tiles = 0;
    for (int i = 0; i < n; i++) {
        p.mat[i] = MatRef{W[i].q, W[i].scales, W[i].zeros, bias[i], y[i], W[i].rows, tiles};
        tiles += int((W[i].rows + 15) / 16);
    }
    p.nmat = n;
    p.K = K; p.G = G;
    p.x = x;
    p.M = 1;
    p.gs = int((G + KS - 1) / KS);
    if (mode == 2) p.gs = (p.gs + 3) / 4 * 4;  // 4-group aligned slices: vector scale loads
    p.S = 1;
    if (W[0].kind == 1) launch_gemv1_t<1, 8>(p, KS, mode, unsigned(tiles), stream);
    else launch_gemv1_t<0, 4>(p, KS, mode, unsigned(tiles), stream);
    return hipGetLastError();
}

// Byte limbs + meta of x [M][K] into the workspace.
hipError_t launch_xprep_limbs(const float* x, int M, int64_t K, int kind, Workspace* ws, hipStream_t stream) {
    const int64_t G = (K + kGroup - 1) / kGroup;
    const int64_t quads = (G + 3) / 4;
    const int64_t waves = int64_t(M) * quads;
    const unsigned grid = unsigned((waves + 3) / 4);
    const bool vecx = (K % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    if (kind == 1) {
        if (vecx) xprep_kernel<true, true><<<grid, 256, 0, stream>>>(x, M, K, G, quads, ws->xq, ws->xmeta);
        else xprep_kernel<true, false><<<grid, 256, 0, stream>>>(x, M, K, G, quads, ws->xq, ws->xmeta);
    } else {
        if (vecx) xprep_kernel<false, true><<<grid, 256, 0, stream>>>(x, M, K, G, quads, ws->xq, ws->xmeta);
        else xprep_kernel<false, false><<<grid, 256, 0, stream>>>(x, M, K, G, quads, ws->xq, ws->xmeta);
    }
    return hipGetLastError();
}

// 2..32 rows (or a 1-row case the 1-row kernel does not cover), one matrix,
// on the limbs prepared in the workspace.
hipError_t launch_gemv_batched(const QView& W, const uint16_t* bias, int M, float* y, Workspace* ws,
                               hipStream_t stream) {
    const int64_t N = W.rows, K = W.cols, G = W.groups;
    const int kind = W.kind;
    GemvParams p{};
    p.q = W.q; p.scales = W.scales; p.zeros = W.zeros;
    p.N = N; p.K = K; p.G = G;
    p.xq = ws->xq; p.meta = ws->xmeta;
    p.bias = bias; p.y = y; p.part = ws->partials;
    p.M = M;
    const int gc = (kind == 1 && M <= 16) ? 8 : 4;  // groups per chunk (LDS: 2 * gc * M * 384 B max)
    static const int target = env_int("IQ_GEMV_WAVES", 2048);
    p.nrb = int((N + 127) / 128);
    const int64_t want_s = (int64_t(target) * device_cu_count() / 256 + int64_t(p.nrb) * 8 - 1) / (int64_t(p.nrb) * 8);
    int S = int(want_s < 1 ? 1 : want_s);
    if (S > (G + 1) / 2) S = int((G + 1) / 2);      // at least 2 groups per slice
    if (S < 1) S = 1;
    while (S > 1 && int64_t(S) * M * N > kPartialFloats) S--;
    p.gs = int((G + S - 1) / S);
    S = int((G + p.gs - 1) / p.gs);
    p.S = S;
    const unsigned grid = unsigned(int64_t(S) * p.nrb);
    const size_t lds = size_t(gc) * (size_t(M) * kLimbRec + kMeta * 16);
    const bool vec = (K % kGroup == 0);
    if (kind == 1) {
        if (gc == 8) launch_gemvb_t<1, 8>(p, vec, grid, lds, stream);
        else launch_gemvb_t<1, 4>(p, vec, grid, lds, stream);
    } else {
        launch_gemvb_t<0, 4>(p, vec, grid, lds, stream);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || S == 1) return e;
    const int64_t n = int64_t(M) * N;
    gemv_reduce_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(p.part, S, M, N, bias, y);
    return hipGetLastError();
}

hipError_t launch_batched_multi(const QView* W, const uint16_t* const* bias, float* const* y, int n, int M,
                                Workspace* ws, hipStream_t stream) {
    for (int i = 0; i < n; i++) {
        const hipError_t e = launch_gemv_batched(W[i], bias[i], M, y[i], ws, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

// A 1-row preparation that the 1-row kernel will consume is a copy of x
// (the kernel converts it itself); anything else is converted to limbs.
hipError_t launch_xprep(const float* x, int M, int64_t K, int kind, Workspace* ws, hipStream_t stream) {
    const int64_t G = (K + kGroup - 1) / kGroup;
    hipError_t e;
    if (M == 1 && gemv1_slices(G, kind, gemv1_mode(K, G, ws->xf)) > 0) {
        e = hipMemcpyAsync(ws->xf, x, sizeof(float) * size_t(K), hipMemcpyDeviceToDevice, stream);
        ws->prep_copy = true;
    } else {
        e = launch_xprep_limbs(x, M, K, kind, ws, stream);
        ws->prep_copy = false;
    }
    ws->prep_M = M;
    ws->prep_K = K;
    ws->prep_kind = kind;
    return e;
}

hipError_t launch_gemv_prepped_multi(const QView* W, const uint16_t* const* bias, float* const* y, int n,
                                     int M, Workspace* ws, hipStream_t stream) {
    if (ws->prep_copy) {
        const int64_t K = W[0].cols, G = W[0].groups;
        const int mode = gemv1_mode(K, G, ws->xf);
        return launch_gemv1(ws->xf, W, bias, y, n, gemv1_slices(G, W[0].kind, mode), mode, stream);
    }
    return launch_batched_multi(W, bias, y, n, M, ws, stream);
}

hipError_t launch_gemv_prepped(const QView& W, const uint16_t* bias, int M, float* y, Workspace* ws,
                               hipStream_t stream) {
    return launch_gemv_prepped_multi(&W, &bias, &y, 1, M, ws, stream);
}

hipError_t launch_gemv_multi(const float* x, const QView* W, const uint16_t* const* bias, float* const* y,
                             int n, int M, Workspace* ws, hipStream_t stream) {
    const int64_t K = W[0].cols, G = W[0].groups;
    if (M == 1) {
        const int mode = gemv1_mode(K, G, x);
        const int KS = gemv1_slices(G, W[0].kind, mode);
        if (KS > 0) return launch_gemv1(x, W, bias, y, n, KS, mode, stream);
    }
    hipError_t e = launch_xprep_limbs(x, M, K, W[0].kind, ws, stream);
    ws->prep_copy = false;
    ws->prep_M = M;
    ws->prep_K = K;
    ws->prep_kind = W[0].kind;
    if (e != hipSuccess) return e;
    return launch_batched_multi(W, bias, y, n, M, ws, stream);
}

hipError_t launch_gemv(const float* x, const QView& W, const uint16_t* bias, int M, float* y,
                       Workspace* ws, hipStream_t stream) {
    return launch_gemv_multi(x, &W, &bias, &y, 1, M, ws, stream);
}

}  // namespace iq

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
//   max|x| * 2^k in [2^30, 0x7F7F7F7F], X = rint(x * 2^k) (exact scaling,
//   one rounding: |x*2^k - X| <= 1/2, i.e. at most 2^-31 of the group's
//   max), and X is written as four signed byte limbs,
//   X = 2^24 X0 + 2^16 X1 + 2^8 X2 + X3.
// The GEMV then forms, per (row tile, group), four exact int32 sums
//   S_L = sum_k q_k * X_L,k        (L = 0..3; the four limbs of one
//                                   activation row are four rows of the
//                                   16-row MFMA tile)
// and for int4 subtracts the zero point exactly in integers,
//   T_L = S_L - z * sum_k X_L,k    (the limb sums come with the limbs),
// so the only floating-point steps are
//   acc += ldexp(s * (2^24 T_0 + 2^16 T_1 + 2^8 T_2 + T_3), -k)   (fp32).
// The int8 codes go to the MFMA untouched; int4 nibbles need one AND (even
// columns) or one shift + AND (odd columns) per 4 codes.
//
// Accuracy: the activation rounding is at most 2^-31 of the group's largest
// |x| per element, products and sums are exact integers, and the fp32
// combination adds a few ulps of each group's partial sum.  A group whose
// largest value is 10^5 x its typical one (an outlier channel of an LLM's
// residual stream) still keeps ~14 bits of its typical values, inside the
// reference's 5e-6 of the conditioning sum |w*x| (tests/test_ops_gpu.cu:
// 199-206).  Non-finite activations make the affected outputs NaN.
//
// Kernels:
//  * gemv1 (1 row, the decode step): workgroup = W waves on one tile of 16
//    output rows, the waves split K (reduced through LDS, deterministic; no
//    cross-workgroup traffic).  A wave requests all weight words, scales and
//    zero points of a batch of groups before it waits, stages the batch's
//    activation limbs in its own LDS slot and runs the MFMAs.
//  * gemvt / gemvb (2..16 rows): a workgroup stages the activation limbs of
//    one K range in LDS once and shares them over many 16-row tiles.  When a
//    matrix is too short to fill the GPU, K is split into ranges over
//    several workgroups; each writes fp32 partial sums to the workspace and
//    a separate reduce launch (gemvt_reduce_kernel / gemv_reduce_kernel)
//    adds them in range order, so the result is deterministic and no
//    counter has to be cleared between launches.
//  * gemvh (2..32 rows, f16 split activations): see gemvh_kernel.
//  * gemvs (7..16 rows on very wide calls, the same split operands shared
//    through LDS by 8 tiles): see gemvs_kernel.
//  * gemvr (5..16 rows on wide or long-K calls: a K range of up to 8 groups
//    requested at once, operands made from x in LDS): see gemvr_kernel.
//  * gemvq (9..16 rows on wide int4 calls, 17..32 rows on wide or long-K
//    calls: gemvr's scheme on 32-row tiles and the 32 x 32 matrix
//    instruction, up to two 16-row blocks): see gemvq_kernel.
#include <algorithm>
#include <cstdlib>

#include "iq_limbs.h"
#include "iq_plan.h"

namespace iq {

namespace {

// Columns [c0, c0 + 8) of an activation row, zero past K.  VECX: 0 scalar
// loads; 1 two 16-byte loads where the 8 columns lie inside K; 2 two 16-byte
// loads, the caller guarantees c0 + 8 <= K.
template <int VECX>
__device__ __forceinline__ void load_x8(const float* xr, int64_t c0, int64_t K, float (&v)[8]) {
    if (VECX == 2 || (VECX == 1 && c0 + 8 <= K)) {
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
    load_x8<VECX ? 1 : 0>(x + int64_t(m) * K, (gvalid ? g : 0) * kGroup + j * 8, gvalid ? K : 0, v);
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
    int ntiles;  // 1-row kernel: 16-row tiles over all matrices
    int th;      // 1-row kernel, one row: rows per tile (8..16; 0: 16)
    int kr, gr;  // 1-row kernel: K ranges (workgroups per tile) and groups per range;
                 // gemvq: kr consecutive K ranges per workgroup
    // Chain prologue (gemvr / gemvq instances with PRO): activation row m,
    // column c is x[m * xstride + c], or with gqa_span > 0 the value row of
    // c's key/value head, x[m * xstride + (c / gqa_span) * gqa_hd + c % gqa_hd];
    // with norm, RMSNorm'd: x * norm[c] is split into the operands and r_m =
    // 1 / sqrt(sum_b ssq[m][b] / K + eps), over the ssq_n partial sums of
    // squares of row m, multiplies the group factors.
    // to_part: K-range partial sums are written even when S == 1.
    int64_t xstride;
    int gqa_hd, gqa_span;
    const uint16_t* norm;
    const float* ssq;
    int ssq_n;
    float eps;
    int to_part;
    // gemvh epilogue (chain stages): y = res + (sum + bias) when res, and
    // the sum of squares of each 16-column tile of each output row into
    // ssq_out[m * ntiles + tile] when ssq_out
    const float* res;
    float* ssq_out;
};

// ------------------------------------------------------------------ chain prologue
// Byte offset of activation row m, columns [c, c + 8) (PRO instances).
__device__ __forceinline__ uint32_t pro_x_offset(const GemvParams& p, int m, int64_t c) {
    const int64_t src = p.gqa_span ? (c / p.gqa_span) * p.gqa_hd + c % p.gqa_hd : c;
    return uint32_t((int64_t(m) * p.xstride + src) * 4);
}

// The RMSNorm row factors r_m of a PRO launch into rsc[0 .. M): step 1
// requests this thread's partial sums of squares (thread t: row t / 16,
// partials t % 16, t % 16 + 16, ... of at most 256; issued before anything
// else), step 2 adds them in a fixed order (double) once they land.
struct ProScale {
    float sq[16];
    __device__ __forceinline__ void request(const GemvParams& p, int tid) {
        const rsrc_t r = make_rsrc(p.ssq, p.norm ? int64_t(p.M) * p.ssq_n * 4 : 0);
        const int m = tid >> 4, j = tid & 15;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int b = j + 16 * k;
            sq[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                  r, (m < p.M && b < p.ssq_n) ? uint32_t(m * p.ssq_n + b) * 4 : kOob, 0, 0));
        }
    }
    // every thread of the workgroup calls this (two barriers)
    __device__ __forceinline__ void finish(const GemvParams& p, int tid, double (*part)[16], float* rsc) {
        double v = 0.0;
#pragma unroll
        for (int k = 0; k < 16; k++) v += double(sq[k]);
        part[tid >> 4][tid & 15] = v;
        __syncthreads();
        if (tid < p.M) {
            double ss = 0.0;
#pragma unroll
            for (int j = 0; j < 16; j++) ss += part[tid][j];
            rsc[tid] = 1.0f / __builtin_sqrtf(float(ss / double(p.K)) + p.eps);
        }
        __syncthreads();
    }
};

// bf16 norm weights of columns [c, c + 8) applied to v (PRO with norm; the
// row factor r_m multiplies the group factors of the split operands
// instead, so the conversion need not wait for it).
__device__ __forceinline__ void pro_norm8(float (&v)[8], uint4 nw) {
    const uint32_t w4[4] = {nw.x, nw.y, nw.z, nw.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t h = w4[i >> 1];
        const float wn = __uint_as_float((i & 1) ? (h & 0xFFFF0000u) : (h << 16));
        v[i] = v[i] * wn;
    }
}

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

// ------------------------------------------------------------------ 1 row
// Weight words, scales and zero points of one wave's K slice of one tile.
template <int KIND, int NG>
struct Slice {
    static constexpr int WPG = KIND == 1 ? 1 : 2;
    int4v_t w[NG][WPG];
    uint32_t s[NG / 2];  // bf16 scales, two per word (group 2i in the low half)
    uint32_t z[NG / 4];  // int4 zero points, four per word (group 4i in the low byte)
};

// One tile's matrix, resolved from the tile index (wave-uniform).
struct TileSel {
    MatRef m;
    int64_t row0;
};

__device__ __forceinline__ TileSel select_tile(const GemvParams& p, int tile, int th = 16) {
    MatRef m = p.mat[0];
#pragma unroll
    for (int i = 1; i < kMaxMulti; i++)
        if (i < p.nmat && tile >= p.mat[i].tile0) m = p.mat[i];
    return TileSel{m, int64_t(tile - m.tile0) * th};
}

// The loads of one wave's slice [gbeg, gbeg + gs) of the tile at row0
// (lane: row row0 + ln, 16-byte column block kg of each 64-byte half group),
// in two calls: scales and zero points first, then the weight words, so the
// small metadata requests are not queued behind the weights.  Rows past N
// and slots past the slice read zero without touching memory (buffer range
// check), so every load is unconditional.
// MODE 0: rows not 16-byte aligned (byte loads, clamped); 1: one scale /
// zero-point load per group; 2: one 8-byte scale and one 4-byte zero-point
// load per 4 groups (G % 4 == 0, slices of whole 4-group blocks), unless the
// workgroup stages the tile's scales and zero points in LDS.
template <int KIND, int NG, int MODE>
__device__ __forceinline__ void load_meta(Slice<KIND, NG>& b, const GemvParams& p, const TileSel& ts, int gbeg,
                                          int gs, int ln, bool live = true) {
    const int G = int(p.G);
    const MatRef& mr = ts.m;
    const int64_t row = ts.row0 + ln;
    const rsrc_t rs = make_rsrc(mr.scales, mr.N * G * 2);
    const rsrc_t rz = make_rsrc(mr.zeros, KIND == 1 ? mr.N * G : 0);
    const int64_t rcs = MODE == 0 ? (row < mr.N ? row : mr.N - 1) : row;
    // (a 24-bit multiply, rows and G < 2^24: the compiler's 64-bit
    // multiply-add for a 32-bit product read an undefined high half from a
    // register that a pending load writes, and so waited for every earlier
    // load before these requests)
    const uint32_t vz = __umul24(uint32_t(rcs), uint32_t(G)) + uint32_t(gbeg);
    const uint32_t vs = vz * 2u;
    if (MODE == 2) {
#pragma unroll
        for (int q4 = 0; q4 < NG / 4; q4++) {
            const uint32_t ok = (4 * q4 < gs && live) ? 0u : kOob;
            const auto sv = __builtin_amdgcn_raw_buffer_load_b64(rs, vs + ok, q4 * 8, 0);
            b.s[2 * q4] = sv[0];
            b.s[2 * q4 + 1] = sv[1];
            b.z[q4] = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b32(rz, vz + ok, q4 * 4, 0) : 0u;
        }
    } else {
        uint32_t sh[NG], zb[NG];
#pragma unroll
        for (int gl = 0; gl < NG; gl++) {
            const uint32_t ok = (gl < gs && live) ? 0u : kOob;
            sh[gl] = __builtin_amdgcn_raw_buffer_load_b16(rs, vs + ok, gl * 2, 0);
            zb[gl] = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b8(rz, vz + ok, gl, 0) : 0u;
        }
#pragma unroll
        for (int i = 0; i < NG / 2; i++) b.s[i] = sh[2 * i] | (sh[2 * i + 1] << 16);
#pragma unroll
        for (int i = 0; i < NG / 4; i++)
            b.z[i] = zb[4 * i] | (zb[4 * i + 1] << 8) | (zb[4 * i + 2] << 16) | (zb[4 * i + 3] << 24);
    }
}

template <int KIND, int NG, int MODE>
__device__ __forceinline__ void load_weights(Slice<KIND, NG>& b, const GemvParams& p, const TileSel& ts, int gbeg,
                                             int gs, int ln, int kg, bool live = true) {
    constexpr int WPG = Slice<KIND, NG>::WPG;
    const int row_bytes = int(KIND == 1 ? p.K / 2 : p.K);
    const MatRef& mr = ts.m;
    const int64_t row = ts.row0 + ln;
    if (MODE == 0) {
        const int64_t rc = row < mr.N ? row : mr.N - 1;
        const uint8_t* qrow = mr.q + rc * row_bytes;
#pragma unroll
        for (int gl = 0; gl < NG; gl++) {
            const int g = gbeg + (gl < gs ? gl : gs - 1);
#pragma unroll
            for (int h = 0; h < WPG; h++) {
                const int off = KIND == 1 ? g * 64 + kg * 16 : g * 128 + h * 64 + kg * 16;
                const uint4 v = load16_slow(qrow, off, row_bytes);
                b.w[gl][h] = int4v_t{int(v.x), int(v.y), int(v.z), int(v.w)};
            }
        }
    } else {
        const rsrc_t rq = make_rsrc(mr.q, mr.N * row_bytes);
        const uint32_t vq = uint32_t(row * row_bytes) + uint32_t(gbeg * (KIND == 1 ? 64 : 128) + kg * 16);
#pragma unroll
        for (int gl = 0; gl < NG; gl++) {
            const uint32_t vo = vq + ((gl < gs && live) ? 0u : kOob);
#pragma unroll
            for (int h = 0; h < WPG; h++)
                b.w[gl][h] = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                             rq, vo, KIND == 1 ? gl * 64 : gl * 128 + h * 64, 0));
        }
    }
}

// Multiplies one tile's slice by the staged activation limbs.  R = 1: the A
// operand carries the four limbs as rows 0..3 of the 16-row MFMA tile
// (lanes l%16 = 0..3; the other lanes read a zero block), so two MFMAs per
// 128 columns give all four exact limb sums, in D rows 0..3 of lanes 0..15.
// R = 4: A row 4m + L = limb L of activation row m < M (rows of m >= M
// zero), so the same two MFMAs give row m's limb sums in D rows
// 4m .. 4m + 3, i.e. registers 0..3 of lanes 16m .. 16m + 15.  Returns the
// running sum of activation row l/16 (R = 4) or row 0 (R = 1, lanes 0..15).
// TP slices (TP 16-row tiles of one workgroup, R = 1 only) share each
// A operand read: acc[t] is tile t's sum.
template <int KIND, int NG, int R, int TP = 1>
__device__ __forceinline__ void slice_dot_tp(const Slice<KIND, NG> (&b)[TP], const int8_t* xs, const int4* ms,
                                             const int8_t* xzero, int RS, int glo, int M, int gbeg, int gs, int ln,
                                             int kg, float (&acc)[TP]) {
    // records of row m, group g at (m RS + g - glo) (RS records per row,
    // the first of them group glo)
#pragma unroll
    for (int t = 0; t < TP; t++) acc[t] = 0.0f;
    const int am = R == 1 ? 0 : ln >> 2, aL = R == 1 ? ln : ln & 3;  // A row of this lane
    const bool alive = am < M;
    const int xoff = (am * RS - glo) * kLimbRec + aL * kGroup + kg * 16;
    const int moff = (R == 1 ? 0 : (kg < R ? kg : 0)) * RS - glo;  // (lane groups past R: row 0, never stored)
    // blocks of 4 groups: an early exit over at most 8 iterations still
    // unrolls fully (so the slice stays in registers)
#pragma unroll
    for (int q4 = 0; q4 < NG / 4; q4++) {
        if (4 * q4 >= gs) break;  // wave-uniform
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int gl = 4 * q4 + e;
            const bool ok = gl < gs;
            const int g = gbeg + (ok ? gl : 0);
            int4v_t a0, a1;
            {
                const int8_t* pa = alive ? xs + (xoff + g * kLimbRec) : xzero;
                a0 = *reinterpret_cast<const int4v_t*>(pa);
                a1 = *reinterpret_cast<const int4v_t*>(pa + (alive ? 64 : 0));
            }
            const int4 md = ms[moff + g];
#pragma unroll
            for (int t = 0; t < TP; t++) {
                int4v_t b0, b1;
                if (KIND == 1) {
                    const int4v_t v = b[t].w[gl][0];
                    b0 = v & 0x0F0F0F0F;
                    b1 = (v >> 4) & 0x0F0F0F0F;
                } else {
                    b0 = b[t].w[gl][0];
                    b1 = b[t].w[gl][1];
                }
                int4v_t D = mfma_i8(a0, b0, int4v_t{0, 0, 0, 0});
                D = mfma_i8(a1, b1, D);
                const uint32_t sw = b[t].s[gl / 2];
                const float sc = __uint_as_float((gl & 1) ? (sw & 0xFFFF0000u) : (sw << 16));
                const int z = KIND == 1 ? int((b[t].z[gl / 4] >> (8 * (gl & 3))) & 0xFF) : 0;
                const float nacc = combine(acc[t], D[0], D[1], D[2], D[3], z, md, sc);
                acc[t] = ok ? nacc : acc[t];
            }
        }
    }
}

template <int KIND, int NG, int R>
__device__ __forceinline__ float slice_dot(const Slice<KIND, NG>& b, const int8_t* xs, const int4* ms,
                                           const int8_t* xzero, int RS, int glo, int M, int gbeg, int gs, int ln,
                                           int kg) {
    float acc[1];
    slice_dot_tp<KIND, NG, R, 1>(reinterpret_cast<const Slice<KIND, NG>(&)[1]>(b), xs, ms, xzero, RS, glo, M, gbeg,
                                 gs, ln, kg, acc);
    return acc[0];
}

// One activation row (the decode step).  Workgroup = KS waves (runtime,
// blockDim.x / 64) on one 16-row tile, wave w owning the K slice
// [w*gs, w*gs + gs).  Each wave converts its slice of the fp32 activations
// into byte limbs in LDS while its weights stream in.  With p.S == 2 (MODE
// 2) the workgroup stages the tile's scales and zero points (16 consecutive
// rows: one contiguous block each) in LDS with one 16-byte load per thread,
// instead of every wave fetching the same lines for its slice.  The slice partials are added
// through LDS by whichever wave finishes last (an LDS counter), in slice
// order, so the sum is deterministic and no wave waits for the others.
// TP = 2 (1 or 2 rows, staged metadata, G <= 32): the workgroup owns tiles
// 2b and 2b + 1 (wave t < 2 stages tile t's scales and zero points); each
// wave requests both tiles' slices and multiplies them by the same
// activation limbs, so one conversion of x and one LDS operand read serve
// 32 rows.
template <int KIND, int NG, int MODE, int MAXW, int R, bool KSPLIT, bool HALF = false, int TP = 1>
__global__ __launch_bounds__(64 * MAXW) void gemv1_kernel(const GemvParams p) {
    // dynamic LDS: limbs [RR][G][512], meta [R][G] int4, then (staged) the
    // tile's scales [16][G] bf16 and zero points [16][G] u8.  R = 8, and R =
    // 4 with HALF, run two blocks of R / 2 rows through the same limb
    // records (each wave reuses its own groups' records; the weights stay
    // in registers): half the LDS of one block of R rows.
    static_assert(!HALF || (R == 4 && !KSPLIT), "two 2-row blocks: the 4-row instance, one K range");
    static_assert(TP == 1 || (R <= 4 && !HALF && MODE == 2 && !KSPLIT), "two tiles: 1..4 rows, staged metadata");
    constexpr int RR = HALF ? R / 2 : (R < 4 ? R : 4);  // rows per block
    constexpr int RB = R / RR;                          // blocks
    extern __shared__ __attribute__((aligned(16))) int8_t xs1[];
    __shared__ __attribute__((aligned(16))) int8_t xzero[16];
    __shared__ float red[MAXW][RB * TP][16 * RR];
    __shared__ int arrived;
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, kg = lane >> 4, wave = tid >> 6;
    const int KS = int(blockDim.x) >> 6;
    const int G = int(p.G);
    // K range of this workgroup: groups [glo, ghi); RS = LDS records per row
    // (KSPLIT: several ranges per tile, 2..4 rows only)
    const int kr = KSPLIT ? p.kr : 1, range = KSPLIT ? int(blockIdx.x) % kr : 0;
    const int RS = KSPLIT ? p.gr : G, glo = range * RS, ghi = glo + RS < G ? glo + RS : G;
    const int gbeg = glo + wave * p.gs < ghi ? glo + wave * p.gs : ghi;
    const int gs = (gbeg + p.gs < ghi ? gbeg + p.gs : ghi) - gbeg;
    const int M = R == 1 ? 1 : p.M;  // activation rows (R = 4: 1..4, R = 8: 5..8)
    int4* ms1 = reinterpret_cast<int4*>(xs1 + RR * RS * kLimbRec);
    int8_t* tmeta = xs1 + (RR * kLimbRec + R * 16) * RS;
    const int tile = KSPLIT ? int(blockIdx.x) / kr : int(blockIdx.x) * TP;
    // rows per tile: th (1 row, one tile per workgroup, whole groups: p.th
    // when set, so that narrow matrices fill every CU), else 16; lanes
    // ln >= th read nothing and store nothing
    const int th = (R == 1 && TP == 1 && !KSPLIT && MODE >= 1 && p.th) ? p.th : 16;
    const bool live = ln < th;
    // (TP = 2, odd tile count: the last workgroup's second tile starts past
    // its matrix's rows, so its loads read zero and nothing is stored)
    TileSel tsv[TP];
#pragma unroll
    for (int t = 0; t < TP; t++) tsv[t] = select_tile(p, tile + t, th);
    const TileSel& ts = tsv[0];
    const bool staged = MODE == 2 && (TP > 1 || p.S == 2);  // (only with kr == 1)

    // 1. This wave's activations: pass t converts groups gbeg + 4t + kg,
    //    16 lanes (one DPP row) per group, 8 columns per lane.  Every wave
    //    requests them before any wave requests weights: the vector L1
    //    returns data in request order, so activations asked for behind the
    //    CU's weight misses would arrive only after them.
    //    The bias of the rows this lane may store goes first (lanes 0..15 of
    //    every wave: any wave may be the one that finishes the tile).
    uint32_t biasv[TP];
#pragma unroll
    for (int t = 0; t < TP; t++) {
        // (TP = 2: every lane takes row ln of both tiles)
        const rsrc_t rb = make_rsrc(tsv[t].m.bias, tsv[t].m.bias ? tsv[t].m.N * 2 : 0);
        const bool mine = (TP == 1 ? lane < 16 * (M < 4 ? M : 4) : true) && live;
        biasv[t] = __builtin_amdgcn_raw_buffer_load_b16(rb, mine ? uint32_t(tsv[t].row0 + ln) * 2 : kOob, 0, 0);
    }
    const uint32_t bias = biasv[0];
    constexpr int XP = NG / 4;
    float xv[R][XP][8];
#pragma unroll
    for (int m = 0; m < R; m++) {
        if (m >= M) break;  // uniform
#pragma unroll
        for (int t = 0; t < XP; t++) {
            const int g = 4 * t + kg < gs ? gbeg + 4 * t + kg : (gs > 0 ? gbeg + gs - 1 : 0);
            load_x8<MODE >= 1 ? 2 : 0>(p.x + int64_t(m) * p.K, int64_t(g) * kGroup + ln * 8, p.K, xv[m][t]);
        }
    }
    if (tid < 4) reinterpret_cast<uint32_t*>(xzero)[tid] = 0u;
    if (tid == 0) arrived = 0;
    __syncthreads();

    // 2. Staged: thread i requests 16 bytes of the tile's scale block
    //    (32 G bytes) and of its zero-point block (16 G bytes; rows past N
    //    read zero); otherwise each wave its own slice's.  Then every wave's
    //    weights, and the conversion while they stream in.
    //    The staged loads are unconditional (not staged, or threads past
    //    the block: an empty range, reading zero): under a branch the
    //    compiler waited for every earlier load before the weights went out.
    //    TP = 2: wave t < 2 stages tile t's blocks (2 G <= 64).
    int4v_t mv_s = {0, 0, 0, 0}, mv_z = {0, 0, 0, 0};
    if constexpr (MODE == 2) {
        const int wt = TP == 1 ? 0 : __builtin_amdgcn_readfirstlane(wave < TP ? wave : 0);
        const TileSel tw = (TP > 1 && wt) ? tsv[TP - 1] : tsv[0];
        int64_t trows = tw.m.N - tw.row0 < th ? tw.m.N - tw.row0 : th;
        trows = trows > 0 ? trows : 0;
        const int sl = TP == 1 ? tid : (wave < TP ? lane : 64);  // 16-byte chunk of this thread
        const rsrc_t rs = make_rsrc(tw.m.scales + tw.row0 * G, staged ? trows * G * 2 : 0);
        mv_s = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(
                                               rs, sl < 2 * G ? uint32_t(sl) * 16 : kOob, 0, 0));
        if (KIND == 1) {
            const rsrc_t rz = make_rsrc(tw.m.zeros + tw.row0 * G, staged ? trows * G : 0);
            mv_z = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                   rz, sl < G ? uint32_t(sl) * 16 : kOob, 0, 0));
        }
    }
    Slice<KIND, NG> bt[TP];
    Slice<KIND, NG>& b = bt[0];
    if (!staged) load_meta<KIND, NG, MODE>(b, p, ts, gbeg, gs, ln, live);
#pragma unroll
    for (int t = 0; t < TP; t++) load_weights<KIND, NG, MODE>(bt[t], p, tsv[t], gbeg, gs, ln, kg, live);
    // rows [m0, m0 + RR) into the limb records (row m at record row m - m0)
    auto convert_rows = [&](int m0) {
#pragma unroll
        for (int mm = 0; mm < RR; mm++) {
            const int m = m0 + mm;
            if (m >= M) break;  // uniform
#pragma unroll
            for (int t = 0; t < XP; t++) {
                if (4 * t >= gs) break;  // wave-uniform
                const int g = gbeg + 4 * t + kg;
                const bool st = 4 * t + kg < gs;
                const int4 md = convert_group<KIND == 1>(xv[m][t], ln, st,
                                                         xs1 + (mm * RS + (st ? g : gbeg) - glo) * kLimbRec);
                if (st && ln == 0) ms1[m * RS + g - glo] = md;
            }
        }
    };
    convert_rows(0);
    // (each wave reads only its own limb records; the zero block is shared)
    if (staged) {
        if (TP == 1) {
            if (wave * 64 < 2 * G) {
                if (tid < 2 * G) reinterpret_cast<int4v_t*>(tmeta)[tid] = mv_s;
                if (KIND == 1 && tid < G) reinterpret_cast<int4v_t*>(tmeta + 32 * G)[tid] = mv_z;
            }
        } else if (wave < TP) {
            int8_t* tm = tmeta + wave * 48 * G;
            if (lane < 2 * G) reinterpret_cast<int4v_t*>(tm)[lane] = mv_s;
            if (KIND == 1 && lane < G) reinterpret_cast<int4v_t*>(tm + 32 * G)[lane] = mv_z;
        }
        __syncthreads();
        // this wave's words: rows ln, groups gbeg .. gbeg + NG (gbeg % 4 == 0)
#pragma unroll
        for (int t = 0; t < TP; t++) {
            const int8_t* tm = tmeta + t * 48 * G;
#pragma unroll
            for (int q4 = 0; q4 < NG / 4; q4++) {
                const int g = 4 * q4 < gs ? gbeg + 4 * q4 : gbeg;
                const uint2 sv = *reinterpret_cast<const uint2*>(tm + (ln * G + g) * 2);
                bt[t].s[2 * q4] = sv.x;
                bt[t].s[2 * q4 + 1] = sv.y;
                bt[t].z[q4] = KIND == 1 ? *reinterpret_cast<const uint32_t*>(tm + 32 * G + ln * G + g) : 0u;
            }
        }
    }

    // 3. The slice as it lands; partials through LDS, the last wave to
    //    arrive adds them in slice order (rows k >= KS were never written).
    if constexpr (TP > 1) {
        float acc2[TP];
        slice_dot_tp<KIND, NG, RR, TP>(bt, xs1, ms1, xzero, RS, glo, M < RR ? M : RR, gbeg, gs, ln, kg, acc2);
#pragma unroll
        for (int t = 0; t < TP; t++)
            if (lane < 16 * RR) red[wave][t][lane] = acc2[t];
        int prior = 0;
        if (lane == 0) prior = __hip_atomic_fetch_add(&arrived, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
        prior = __builtin_amdgcn_readfirstlane(prior);
        if (prior != KS - 1) return;
        // (tile t, activation row m) pairs RR t + m = kg + 4 j
#pragma unroll
        for (int j = 0; j < (TP * RR + 3) / 4; j++) {
            const int pr = kg + 4 * j, tq = pr / RR, m = pr % RR;
            if (tq >= TP || m >= M) break;
            float sum = red[0][tq][16 * m + ln];
#pragma unroll
            for (int k = 1; k < MAXW; k++) {
                const float v = red[k][tq][16 * m + ln];
                sum += k < KS ? v : 0.0f;
            }
            const TileSel& tt = (TP > 1 && tq) ? tsv[TP - 1] : tsv[0];
            const uint32_t bv = (TP > 1 && tq) ? biasv[TP - 1] : biasv[0];
            if (tt.row0 + ln < tt.m.N) tt.m.y[int64_t(m) * tt.m.N + tt.row0 + ln] = sum + __uint_as_float(bv << 16);
        }
        return;
    }
    float acc = slice_dot<KIND, NG, RR>(b, xs1, ms1, xzero, RS, glo, M < RR ? M : RR, gbeg, gs, ln, kg);
    if (lane < 16 * RR) red[wave][0][lane] = acc;
    if constexpr (RB == 2) {
        // rows RR..2 RR - 1: the wave overwrites its own records (its reads
        // of them above come first in program order)
        if (M > RR) {  // uniform
            convert_rows(RR);
            acc = slice_dot<KIND, NG, RR>(b, xs1, ms1 + RR * RS, xzero, RS, glo, M - RR, gbeg, gs, ln, kg);
            if (lane < 16 * RR) red[wave][1][lane] = acc;
        }
    }
    int prior = 0;
    if (lane == 0) prior = __hip_atomic_fetch_add(&arrived, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    prior = __builtin_amdgcn_readfirstlane(prior);
    if (prior != KS - 1) return;
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        const int m = RR * rb + kg;  // lane group kg < RR of block rb: row m
        if (kg >= RR || m >= M) break;
        float sum = red[0][rb][lane];
#pragma unroll
        for (int k = 1; k < MAXW; k++) {
            const float v = red[k][rb][lane];
            sum += k < KS ? v : 0.0f;
        }
        if (ts.row0 + ln >= ts.m.N || !live) continue;
        if (kr == 1) ts.m.y[int64_t(m) * ts.m.N + ts.row0 + ln] = sum + __uint_as_float(bias << 16);
        else p.part[(int64_t(range) * M + m) * (int64_t(p.ntiles) * 16) + int64_t(tile) * 16 + ln] = sum;
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
//     (l%16 = n, l/16 = mm) ends with the 4 limb sums of one (row, n).
//   otherwise: A row i = activation row mt*16 + i, one MFMA per limb
//     (8 per 128 columns for 16 rows); D register r of limb L's MFMA holds
//     (row mt*16 + 4*(l/16) + r, n = l%16).
// With S > 1 slices (matrices too short to fill the GPU) each slice writes
// fp32 partial sums and gemv_reduce adds them in slice order (deterministic).
template <int KIND, bool ROWS4, int MT, int GC, bool VEC>
__global__ __launch_bounds__(512) void gemvb_kernel(const GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) int8_t xsb[];  // [GC][M][512] limbs, [GC][32] meta
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
            xr[i] = *reinterpret_cast<const int4v_t*>(p.xq + (int64_t(rem / (kLimbRec / 16)) * G + g0_ + gl) * kLimbRec + (rem % (kLimbRec / 16)) * 16); \
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
                        const int8_t* pa = m < M ? xsb + (gl * M + m) * kLimbRec + L * kGroup + st * 64 + kg * 16 : xzero;
                        a[st] = *reinterpret_cast<const int4v_t*>(pa);
                    }
                    int4v_t D = mfma_i8(a[0], b0, int4v_t{0, 0, 0, 0});
                    D = mfma_i8(a[1], b1, D);
                    const int mo = mt * 4 + kg;  // activation row of this lane's D
                    if (mo < M) acc[mt][0] = combine(acc[mt][0], D[0], D[1], D[2], D[3], z, msb[gl * kMeta + mo], s);
                } else {
                    const int m = mt * 16 + ln;
                    int4v_t D[kLimbs];
#pragma unroll
                    for (int L = 0; L < kLimbs; L++) {
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
                        if (mo < M) acc[mt][r] = combine(acc[mt][r], D[0][r], D[1][r], D[2][r], D[3][r], z, msb[gl * kMeta + mo], s);
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

// ------------------------------------------------------------------ 2..16 rows
// Several activation rows (M <= 16 per launch; more rows run in blocks of
// 16), K a multiple of 128.  Tile per wave: a workgroup copies the prepared
// activations (byte limbs, xprep) of one K range once into LDS, in MFMA
// operand order, then each wave runs over whole 16-row tiles on its own (no
// cross-wave reduction), tile after tile and group after group, two halves
// of D/2 groups of weights in flight (a half is multiplied while the other
// half's loads are outstanding).  Every weight byte is read once per
// launch.  The tile results go through LDS and are stored after the last
// tile (a store between prefetches would make the later waits count it).
// When the activations of all of K do not fit in LDS, K is split into S
// ranges: workgroup (u, s) writes its range's sums to part[s][m][16*tile + n]
// and gemvt_reduce_kernel adds the ranges of every matrix in one launch.
// A operand layouts: up to 12 rows, quad layout: A tile q row 4*mm + L =
// limb L of activation row 4q + mm, two MFMAs per 128 columns give the
// four limb sums of four rows, lane (n = l%16, mm = l/16) holding those of
// (row 4q + mm, output n).  13..16 rows, limb-major: A tile L = limb L of
// the 16 rows (eight MFMAs per group), lane (n, mm) holding rows 4*mm + i
// in D[i].
constexpr int kGtTmax = 8;     // tiles per wave
constexpr int kGtChunks = 16;  // staged 16-byte chunks per thread

template <int KIND, int MQ, int D>
__global__ __launch_bounds__(512) void gemvt_kernel(const GemvParams p) {
    extern __shared__ __attribute__((aligned(16))) int4 gsm4[];
    constexpr int WPG = KIND == 1 ? 1 : 2;
    constexpr bool LM = MQ == 4;       // limb-major A
    constexpr int NA = LM ? kLimbs : MQ;  // A tiles per 64 columns
    constexpr int NACC = LM ? 4 : MQ;  // running sums per lane
    constexpr int NM = MQ * 4;         // meta records per group
    constexpr int CH = kGtChunks;
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KW = int(blockDim.x) >> 6;
    const int G = int(p.G), M = p.M, S = p.S;
    const int range = int(blockIdx.x) % S, u = int(blockIdx.x) / S;
    const int NWu = int(gridDim.x) / S;
    const int g0 = range * p.gs;
    const int RG = (g0 + p.gs < G ? g0 + p.gs : G) - g0;  // groups of this range
    const int row_bytes = int(KIND == 1 ? p.K / 2 : p.K);
    int4* As = gsm4;                                      // [gs][NA][2][64]
    int4* ms = As + p.gs * NA * 2 * 64;                   // [gs][NM]
    float* outs = reinterpret_cast<float*>(ms + p.gs * NM);  // [KW][kGtTmax + 1][NACC][64]

    // this wave's tiles: u*KW + wave + k*NWu*KW
    const int tfirst = u * KW + wave, tstride = NWu * KW;
    const int ntw = tfirst < p.ntiles ? (p.ntiles - 1 - tfirst) / tstride + 1 : 0;

    // staging loads (A operands and meta records of the range)
    const int total = RG * NA * 2 * 64;
    int4 v[CH];
    int4 mrec;
    {
        const rsrc_t rx = make_rsrc(p.xq, int64_t(M) * G * kLimbRec);
        const rsrc_t rm = make_rsrc(p.meta, int64_t(G) * kMeta * 16);
#pragma unroll
        for (int i = 0; i < CH; i++) {
            const int c = tid + i * int(blockDim.x);
            const int blk = c >> 6, l = c & 63;
            const int gl = blk / (NA * 2), q = (blk >> 1) % NA, st = blk & 1;
            const int m = LM ? (l & 15) : 4 * q + ((l & 15) >> 2), L = LM ? q : l & 3, kgl = l >> 4;
            const bool ok = c < total && m < M;
            const uint32_t off = uint32_t(m * G + g0 + gl) * kLimbRec + uint32_t(L * kGroup + st * 64 + kgl * 16);
            v[i] = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(rx, ok ? off : kOob, 0, 0));
        }
        const int gl = tid / NM, mm = tid % NM;
        const bool ok = tid < RG * NM && mm < M;
        mrec = __builtin_bit_cast(int4, __builtin_amdgcn_raw_buffer_load_b128(
                                            rm, ok ? uint32_t((g0 + gl) * kMeta + mm) * 16 : kOob, 0, 0));
    }

    // loaded values are kept as loaded until their use (any operation on
    // them in flight would make the loop wait for every load)
    struct Buf {
        int4v_t w[WPG];
        uint32_t sc, zp;  // bf16 scale bits, zero point
    };
    // issue position: tile ordinal ik, group ig of the range (wave-uniform);
    // the buffers are based at the issue tile's first row (empty past the
    // wave's tiles) and refreshed when ik advances, so that the lane
    // offsets stay fixed and the loads straight-line
    int ik = 0, ig = 0;
    rsrc_t rq, rs, rz;
    const uint32_t vq = uint32_t(ln * row_bytes + kg * 16), vs = uint32_t(ln * G) * 2, vz = uint32_t(ln * G);
    auto set_tile = [&]() {
        const bool live = ik < ntw;
        const int tile = tfirst + (live ? ik : 0) * tstride;
        const TileSel ts = select_tile(p, tile < p.ntiles ? tile : p.ntiles - 1);
        const int64_t rows = live ? ts.m.N - ts.row0 : 0;
        rq = make_rsrc(ts.m.q + ts.row0 * row_bytes, rows * row_bytes);
        rs = make_rsrc(ts.m.scales + ts.row0 * G, rows * G * 2);
        rz = make_rsrc(ts.m.zeros ? ts.m.zeros + ts.row0 * G : nullptr, KIND == 1 ? rows * G : 0);
    };
    set_tile();
    auto issue = [&](Buf& bf) {
        const int g = g0 + ig;
#pragma unroll
        for (int h = 0; h < WPG; h++)
            bf.w[h] = __builtin_bit_cast(
                int4v_t, __builtin_amdgcn_raw_buffer_load_b128(rq, vq, KIND == 1 ? g * 64 : g * 128 + h * 64, 0));
        bf.sc = __builtin_amdgcn_raw_buffer_load_b16(rs, vs, g * 2, 0);
        bf.zp = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b8(rz, vz, g, 0) : 0u;
        if (++ig == RG) {
            ig = 0;
            ++ik;
            set_tile();
        }
    };

    // The first half of the weights is requested before the staged values
    // are written, the second after (when the staging registers are free).
    constexpr int H = D / 2;
    Buf buf[2][H];
#pragma unroll
    for (int i = 0; i < H; i++) issue(buf[0][i]);
#pragma unroll
    for (int i = 0; i < CH; i++) {
        const int c = tid + i * int(blockDim.x);
        if (c < total) As[c] = v[i];
    }
    if (tid < RG * NM) ms[tid] = mrec;
#pragma unroll
    for (int i = 0; i < H; i++) issue(buf[1][i]);
    __syncthreads();  // A operands and meta staged

    // H steps without branches (the scheduler interleaves them).  Steps past
    // the wave's last tile multiply zero weights and scales; every step
    // writes the running sums to an LDS slot, the tile's slot at its last
    // group of the range and a spare slot otherwise.
    float acc[NACC];
#pragma unroll
    for (int j = 0; j < NACC; j++) acc[j] = 0.0f;
    int ck = 0, cg = 0;
    auto compute_half = [&](const Buf (&hb)[H]) {
#pragma unroll
        for (int i = 0; i < H; i++) {
            const Buf& bf = hb[i];
            int4v_t b0, b1;
            if (KIND == 1) {
                b0 = bf.w[0] & 0x0F0F0F0F;
                b1 = (bf.w[0] >> 4) & 0x0F0F0F0F;
            } else {
                b0 = bf.w[0];
                b1 = bf.w[1];
            }
            const float sc = __uint_as_float(bf.sc << 16);
            const int z = int(bf.zp);
            const int4* ag = As + cg * (NA * 2 * 64) + lane;
            const int4* mg = ms + cg * NM;
            if (LM) {
                int4v_t Dv[kLimbs];
#pragma unroll
                for (int L = 0; L < kLimbs; L++) {
                    Dv[L] = mfma_i8(__builtin_bit_cast(int4v_t, ag[(2 * L) * 64]), b0, int4v_t{0, 0, 0, 0});
                    Dv[L] = mfma_i8(__builtin_bit_cast(int4v_t, ag[(2 * L + 1) * 64]), b1, Dv[L]);
                }
#pragma unroll
                for (int j = 0; j < 4; j++) acc[j] = combine(acc[j], Dv[0][j], Dv[1][j], Dv[2][j], Dv[3][j], z, mg[4 * kg + j], sc);
            } else {
#pragma unroll
                for (int q = 0; q < MQ; q++) {
                    int4v_t Dv = mfma_i8(__builtin_bit_cast(int4v_t, ag[(2 * q) * 64]), b0, int4v_t{0, 0, 0, 0});
                    Dv = mfma_i8(__builtin_bit_cast(int4v_t, ag[(2 * q + 1) * 64]), b1, Dv);
                    acc[q] = combine(acc[q], Dv[0], Dv[1], Dv[2], Dv[3], z, mg[4 * q + kg], sc);
                }
            }
            const bool flush = cg == RG - 1;
            const int slot = flush && ck < kGtTmax ? ck : kGtTmax;
#pragma unroll
            for (int j = 0; j < NACC; j++) {
                outs[((wave * (kGtTmax + 1) + slot) * NACC + j) * 64 + lane] = acc[j];
                acc[j] = flush ? 0.0f : acc[j];
            }
            cg = flush ? 0 : cg + 1;
            ck += flush ? 1 : 0;
        }
    };
    const int nsteps = ntw * RG;
    for (int s0 = 0; s0 < nsteps; s0 += 2 * H) {
        compute_half(buf[0]);
#pragma unroll
        for (int i = 0; i < H; i++) issue(buf[0][i]);
        compute_half(buf[1]);
#pragma unroll
        for (int i = 0; i < H; i++) issue(buf[1][i]);
    }

    // results of this wave's tiles (its own LDS region: no barrier needed)
    for (int k = 0; k < ntw; k++) {
        const int tile = tfirst + k * tstride;
        const TileSel ts = select_tile(p, tile);
        const int64_t row = ts.row0 + ln;
        const rsrc_t rb = make_rsrc(ts.m.bias, ts.m.bias ? ts.m.N * 2 : 0);
        const uint32_t bb =
            __builtin_amdgcn_raw_buffer_load_b16(rb, S == 1 && row < ts.m.N ? uint32_t(row) * 2 : kOob, 0, 0);
#pragma unroll
        for (int j = 0; j < NACC; j++) {
            const int m = LM ? 4 * kg + j : 4 * j + kg;
            const float val = outs[((wave * (kGtTmax + 1) + k) * NACC + j) * 64 + lane];
            if (m >= M || row >= ts.m.N) continue;
            if (S == 1) ts.m.y[int64_t(m) * ts.m.N + row] = val + __uint_as_float(bb << 16);
            else p.part[(int64_t(range) * M + m) * (int64_t(p.ntiles) * 16) + int64_t(tile) * 16 + ln] = val;
        }
    }
}

// y_i[m, n] = sum over ranges s of part[s][m][16*tile0_i + n] (in range
// order) + bias_i[n], for every matrix i of a gemvt launch in one grid
// (thread i covers (m, tile row) over all matrices' tiles).
__global__ __launch_bounds__(256) void gemvt_reduce_kernel(const GemvParams p) {
    const int64_t ld = int64_t(p.ntiles) * 16;
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(p.M) * ld) return;
    const int m = int(i / ld);
    const int64_t c = i - int64_t(m) * ld;
    const TileSel ts = select_tile(p, int(c >> 4));
    const int64_t row = ts.row0 + (c & 15);
    if (row >= ts.m.N) return;
    const float sum = sum_slices(p.part, p.S, int64_t(p.M) * ld, int64_t(m) * ld + c);
    ts.m.y[int64_t(m) * ts.m.N + row] = sum + (ts.m.bias ? bf16_to_f32(ts.m.bias[row]) : 0.0f);
}

// y[m, n] = sum over slices s of part[s, m, n] (in slice order) + bias[n].
__global__ __launch_bounds__(256) void gemv_reduce_kernel(const float* __restrict__ part, int S, int M, int64_t N,
                                                          const uint16_t* __restrict__ bias, float* __restrict__ y) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= int64_t(M) * N) return;
    const float sum = sum_slices(part, S, int64_t(M) * N, i);
    y[i] = sum + (bias ? bf16_to_f32(bias[i % N]) : 0.0f);
}

template <int KIND, int GC>
void launch_gemvb_t(const GemvParams& p, bool vec, unsigned grid, size_t lds, hipStream_t stream) {
    const int M = p.M;
#define IQ_GB(R4, MT)                                                                         \
    do {                                                                                      \
        if (vec) {                                                                            \
            allow_big_lds<gemvb_kernel<KIND, R4, MT, GC, true>>();                            \
            gemvb_kernel<KIND, R4, MT, GC, true><<<grid, 512, lds, stream>>>(p);              \
        } else {                                                                              \
            allow_big_lds<gemvb_kernel<KIND, R4, MT, GC, false>>();                           \
            gemvb_kernel<KIND, R4, MT, GC, false><<<grid, 512, lds, stream>>>(p);             \
        }                                                                                     \
    } while (0)
    if (M <= 4) IQ_GB(true, 1);
    else if (M <= 8) IQ_GB(true, 2);
    else if constexpr (GC <= 4) {
        // (8-group chunks of 9..32 rows would spill the staging registers)
        if (M <= 16) IQ_GB(false, 1);
        else IQ_GB(false, 2);
    }
#undef IQ_GB
}

// MODE of the 1-row kernel (see load_meta / load_weights); 16-byte paths also need a
// 16-byte aligned activation row.
int gemv1_mode(int64_t K, int64_t G, const float* x) {
    if (K % kGroup || reinterpret_cast<uintptr_t>(x) % 16) return 0;
    return G % 4 ? 1 : 2;
}

// Rows of the 1-row kernel instance for M activation rows, and its dynamic
// LDS (limbs of up to 4 rows, meta records of all).  2 rows have their own
// instance (A rows 0..7; 63-66 VGPRs against 79-82 for 4 rows, so 7-8
// waves per SIMD and half the limb LDS): 7B int4 step at 2 rows 1681 ->
// 1505 us (gate|up 25.5 -> 20.5, down 19.9 -> 18.0, lm_head int8 107.5 ->
// 94.7 us).
int gemv1_rows(int M) { return M > 4 ? 8 : (M > 2 ? 4 : M); }
// (half: the 4-row instance's two blocks of 2 rows)
size_t gemv1_lds(int64_t G, int R, bool half = false) {
    return size_t(G) * ((half ? R / 2 : (R < 4 ? R : 4)) * kLimbRec + R * 16);
}

// 1..4 rows always; 5..8 rows (two blocks of 4, the second converted after
// the first is multiplied) only on narrow launches, measured at 7B: o (224
// tiles) 10.1 -> 9.2 us at 8 rows and q|k|v (288) 12.2 -> 10.5 at 5, but
// q|k|v 12.2 -> 13.1 at 8 rows and gate|up 35 -> 41 / 53 us at 5 / 8.
bool gemv1_rows_preferred(int M, int tiles, int64_t G) {
    if (M <= 4) return true;
    if (M > 8) return false;
    const int cus = device_cu_count();
    // short rows convert fast: 1.5B gate (G = 12, 560 tiles) at 7 / 8 rows
    // 11.7 -> 10.1 / 11.8 -> 10.7 us (int8)
    return tiles <= cus || (tiles < 4 * cus && (M <= 6 || G <= 16));
}

// Shape of a 1-row launch: groups per wave slice (gs), waves per workgroup
// (ks), the slice capacity NG of the kernel instance (0: not applicable),
// the grid (kr workgroups per 16-row tile, each a K range of gr groups).
struct G1Plan {
    int gs, ks, ng, grid, kr, gr;
};

// Kernel instances: one 16-row tile per workgroup (measured faster than
// workgroups walking several tiles: the hardware dispatcher keeps every CU
// fed, and each wave requests its whole slice at once); slice capacity NG
// in {4, 8, 12} (int4, up to 16 waves) or {4, 8, 12, 20} (int8, up to 8
// waves): the smallest that holds the slice, since every slot past the
// slice would be an out-of-range request, and those still occupy the
// memory pipeline.  ng = 0 when the 1-row kernel does not apply (the
// slices would exceed the capacity, or the LDS copy of the converted row
// would exceed 64 KiB).
G1Plan gemv1_plan(int64_t G, int kind, int mode, int ntiles, int cus, int R) {
    (void)cus;
    G1Plan pl{0, 0, 0, 0, 1, int(G)};
    // 2..4 rows: the limbs of a long row split K into ranges (workgroups per
    // tile) whose records fit 64 KiB, multiples of 4 groups (7B down at 2
    // rows: int4 27.0 -> 18.0, int8 30.2 -> 23.8 us); 1 row, and 5..8 rows
    // (measured slower split: down 27 -> 32 us at 8 rows): one range
    if (R == 2 || R == 4) {
        while (gemv1_lds(pl.gr, R) > 64 * 1024 && pl.kr < 8) {
            pl.kr++;
            pl.gr = int((G + pl.kr - 1) / pl.kr + 3) / 4 * 4;
        }
        pl.kr = int((G + pl.gr - 1) / pl.gr);
        if (pl.kr > 1 && int64_t(pl.kr) * 8 * ntiles * 16 > kPartialFloats) return G1Plan{0, 0, 0, 0, 1, int(G)};
    }
    // (1 row: the converted row of up to 296 groups, 7B down's 148 in 78 KiB)
    if (gemv1_lds(pl.gr, R) > (R == 1 ? 156 : 64) * 1024) return pl;
    const int64_t GR = pl.gr;
    const int maxw = kind == 1 ? 16 : 8;
    pl.ng = kind == 1 ? 12 : 20;
    pl.gs = int((GR + maxw - 1) / maxw);
    if (mode == 2) pl.gs = (pl.gs + 3) / 4 * 4;
    for (int c : {4, 8, 12})
        if (pl.gs <= c && c < pl.ng) {
            pl.ng = c;
            break;
        }
    // 1 row with per-group metadata loads (MODE 1: G % 4 != 0): fill the
    // slice capacity, fewer waves with no dead slots (1.5B down 1536 x 8960,
    // int4: 14 waves of 5 groups in 8-group slots 9.7 -> 9 waves of 8 groups
    // 8.5 us; 6 groups 8.9, 12 groups 9.2-9.4 us; 1.5B set 23.9 -> 22.7 us;
    // int8 and other widths 2-20 % faster)
    if (mode == 1 && R == 1 && pl.gs < pl.ng) pl.gs = pl.ng;
    pl.grid = ntiles * pl.kr;
    if (pl.gs > GR) pl.gs = int(GR);
    pl.ks = int((GR + pl.gs - 1) / pl.gs);
    if (pl.gs > pl.ng || pl.ks > maxw) pl.ng = 0;
    // 2..8 rows: 16-byte aligned rows (MODE 2; 2..4 rows also MODE 1) and
    // at most 4 (int4, or 8 rows) / 8 (int8) groups per slice: the
    // activations of all rows stay in registers
    if (R > 1 && (mode == 0 || (R == 8 && mode != 2) || pl.ng > (kind == 1 || R == 8 ? 4 : 8))) pl.ng = 0;
    return pl;
}

template <int KIND, int NG, int MAXW>
void launch_gemv1_m(const GemvParams& p, int mode, int ks, unsigned grid, size_t lds, hipStream_t stream,
                    bool half = false, int tp = 1) {
#define IQ_G1X(MODE_, R_, KSPLIT_, HALF_, TP_)                                                          \
    do {                                                                                                \
        allow_big_lds<gemv1_kernel<KIND, NG, MODE_, MAXW, R_, KSPLIT_, HALF_, TP_>>();                  \
        gemv1_kernel<KIND, NG, MODE_, MAXW, R_, KSPLIT_, HALF_, TP_><<<grid, 64 * ks, lds, stream>>>(p); \
    } while (0)
#define IQ_G1H(MODE_, R_, KSPLIT_, HALF_) IQ_G1X(MODE_, R_, KSPLIT_, HALF_, 1)
#define IQ_G1(MODE_, R_, KSPLIT_) IQ_G1H(MODE_, R_, KSPLIT_, false)
    if (p.M > 4) {
        if constexpr (NG <= 4) IQ_G1(2, 8, false);
        return;
    }
    if (p.M == 2) {
        if constexpr (NG <= (KIND == 1 ? 4 : 8)) {
            if (mode == 2 && tp == 2) {
                if constexpr (NG == 4 && KIND == 1) IQ_G1X(2, 2, false, false, 2);
            } else if (mode == 2) {
                if (p.kr > 1) IQ_G1(2, 2, true);
                else IQ_G1(2, 2, false);
            } else {
                if (p.kr > 1) IQ_G1(1, 2, true);
                else IQ_G1(1, 2, false);
            }
        }
        return;
    }
    if (p.M > 1) {
        if constexpr (NG <= (KIND == 1 ? 4 : 8)) {
            if (KIND == 0 && half) {
                if constexpr (KIND == 0) {  // (int8 only)
                    if (mode == 2) IQ_G1H(2, 4, false, true);
                    else IQ_G1H(1, 4, false, true);
                }
            } else if (mode == 2 && tp == 2) {
                if constexpr (NG == 4 && KIND == 1) IQ_G1X(2, 4, false, false, 2);
            } else if (mode == 2) {
                if (p.kr > 1) IQ_G1(2, 4, true);
                else IQ_G1(2, 4, false);
            } else {
                if (p.kr > 1) IQ_G1(1, 4, true);
                else IQ_G1(1, 4, false);
            }
        }
        return;
    }
    if (mode == 2 && tp == 2) {
        if constexpr (NG == 4 && KIND == 1) IQ_G1X(2, 1, false, false, 2);
    } else if (mode == 2) IQ_G1(2, 1, false);
    else if (mode == 1) IQ_G1(1, 1, false);
    else IQ_G1(0, 1, false);
#undef IQ_G1
#undef IQ_G1H
#undef IQ_G1X
}

// The 1-row kernel on n <= kMaxMulti matrices of one kind and width.
// M = 1, or 2..8 rows (a plan made for gemv1_rows(M)) of x at stride K;
// part: the split-K partials (plans with kr > 1).
hipError_t launch_gemv1(const float* x, const QView* W, const uint16_t* const* bias, float* const* y, int n,
                        const G1Plan& pl, int mode, hipStream_t stream, int M = 1, float* part = nullptr,
                        bool reduce = true) {
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
    p.M = M;
    p.gs = pl.gs;
    p.ntiles = tiles;
    p.kr = pl.kr;
    p.gr = pl.gr;
    p.part = part;
    // int8, 3..4 rows on wide launches (at least 4 workgroups per CU), one
    // K range: two blocks of 2 rows through the limb records of 2 rows (7B
    // int8 at 3 rows: gate|up 33.2 -> 32.2, lm_head 130 -> 124.5 us, step
    // 2091 -> 2060 us; at 4 rows 2192 -> 2175 us).  Not int4 (gate|up at
    // 3 rows 28.0 -> 32.5 us): the instance's 82 VGPRs hold a CU to two
    // workgroups either way, and the second block's pass is then extra.
    const bool half = W[0].kind == 0 && gemv1_rows(M) == 4 && pl.kr == 1 && tiles >= 4 * device_cu_count();
    size_t lds = gemv1_lds(pl.gr, gemv1_rows(M), half);
    // Staged scales / zero points on wide launches (7B int4 gate|up 16.9 ->
    // 15.9 us); narrow ones (under 4 workgroups per CU) lose more to the
    // extra barrier than they save (o 4.8 -> 5.1 us).  Not where the 48 G
    // bytes would cut the workgroups a CU holds (160 KiB of LDS, 32 waves
    // at <= 64 VGPRs), or leave a staged word without a thread.
    const size_t cu_lds = 160 * 1024, staged = lds + size_t(G) * 48, wlim = size_t(32 / pl.ks);
    const size_t occ = std::min(cu_lds / lds, wlim), occ_staged = std::min(cu_lds / staged, wlim);
    p.S = 1;
    if (mode == 2 && pl.kr == 1 && tiles >= 4 * device_cu_count() && staged <= 64 * 1024 && occ_staged == occ &&
        2 * G <= 64 * pl.ks) {
        p.S = 2;
        lds = staged;
    }
    // int4, 1..4 rows, staged, 4-group slices, >= 6 waves: two tiles per
    // workgroup (TP = 2; 7B gate|up, 7 waves: 16.4 -> 15.7 us at 1 row,
    // 21.3 -> 17.9 at 2, 28.0 -> 21.4 at 3 rows; at 4 rows 22.8 us against
    // 27.5 on gemvr; steps at 2 / 3 / 4 rows 1488 / 1774 / 1835 -> 1439 /
    // 1630 / 1717 us; 1.5B gate|up, 3 waves, lost: 6.2 -> 6.7 us at 1 row).
    // Not int8 (lm_head 88 -> 92-98 us: two tiles' int8 words take the
    // instance to 97 VGPRs, five waves per SIMD)
    int tp = 1;
    if (W[0].kind == 1 && M <= 4 && !half && p.S == 2 && pl.ng == 4 && 2 * G <= 64 && pl.ks >= 6) {
        tp = 2;
        lds += size_t(G) * 48;
    }
    unsigned grid = unsigned(tp == 2 ? (pl.grid + 1) / 2 : pl.grid);
    // 1 row on fewer 16-row tiles than CUs (one tile per workgroup, whole
    // groups): the tallest tiles of 8..15 rows that give every CU one (7B
    // down and o, 224 tiles of 16 rows: 256 of 14; down 11.95 -> 11.78 us,
    // step 1188 -> 1179 us; 1.5B down, 96 tiles: 192 of 8, 8.5 -> 7.7 us)
    p.th = 0;
    if (M == 1 && tp == 1 && pl.kr == 1 && mode >= 1 && tiles < device_cu_count()) {
        int th = 15;
        auto count = [&](int h) {
            int t = 0;
            for (int i = 0; i < n; i++) t += int((W[i].rows + h - 1) / h);
            return t;
        };
        while (th > 8 && count(th) < device_cu_count()) th--;
        int t0 = 0;
        for (int i = 0; i < n; i++) {
            p.mat[i].tile0 = t0;
            t0 += int((W[i].rows + th - 1) / th);
        }
        p.th = th;
        grid = unsigned(t0);
    }
    if (W[0].kind == 1) {
        if (pl.ng == 4) launch_gemv1_m<1, 4, 16>(p, mode, pl.ks, grid, lds, stream, half, tp);
        else if (pl.ng == 8) launch_gemv1_m<1, 8, 16>(p, mode, pl.ks, grid, lds, stream, half);
        else launch_gemv1_m<1, 12, 16>(p, mode, pl.ks, grid, lds, stream, half);
    } else {
        if (pl.ng == 4) launch_gemv1_m<0, 4, 8>(p, mode, pl.ks, grid, lds, stream, half, tp);
        else if (pl.ng == 8) launch_gemv1_m<0, 8, 8>(p, mode, pl.ks, grid, lds, stream, half);
        else if (pl.ng == 12) launch_gemv1_m<0, 12, 8>(p, mode, pl.ks, grid, lds, stream, half);
        else launch_gemv1_m<0, 20, 8>(p, mode, pl.ks, grid, lds, stream, half);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pl.kr == 1 || !reduce) return e;
    // the K ranges' sums, in range order, + bias
    GemvParams pr = p;
    pr.S = pl.kr;
    const int64_t cnt = int64_t(M) * tiles * 16;
    gemvt_reduce_kernel<<<unsigned((cnt + 255) / 256), 256, 0, stream>>>(pr);
    return hipGetLastError();
}

int total_tiles(const QView* W, int n) {
    int t = 0;
    for (int i = 0; i < n; i++) t += int((W[i].rows + 15) / 16);
    return t;
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
    const int gc = (kind == 1 && M <= 8) ? 8 : 4;  // groups per chunk (LDS: gc * (M * 512 + 512) B)
    constexpr int target = 2048;  // waves per 256 CUs the slices aim for
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

// Plan of a gemvt launch (kw = 0: not applicable): K ranges of gs groups
// whose activations take at most 96 KiB of LDS, one workgroup per CU, the
// waves per workgroup that give the fewest idle tile slots.
struct GtPlan {
    int kw = 0, ks = 0, gs = 0, mq = 0, grid = 0;
    size_t lds = 0;
};

GtPlan gemvt_plan(int64_t G, int tiles, int M, int cus) {
    GtPlan pl;
    const int mq = (M + 3) / 4, na = mq == 4 ? kLimbs : mq, nacc = mq == 4 ? 4 : mq;
    const int rmax = 96 * 1024 / (na * 2048);
    const int ks = int((G + rmax - 1) / rmax);
    const int gs = int((G + ks - 1) / ks);
    const int nwu = cus / ks > 0 ? cus / ks : 1;
    const size_t fixed = size_t(gs) * na * 2048 + size_t(gs) * mq * 4 * 16;
    double best = 0;
    for (int kw = 2; kw <= 8; kw++) {
        const size_t lds = fixed + size_t(kw) * (kGtTmax + 1) * nacc * 256;
        if (lds > 160 * 1024) break;
        if (int64_t(gs) * na * 128 > int64_t(kGtChunks) * 64 * kw || gs * mq * 4 > 64 * kw) continue;
        const int waves = nwu * kw;
        const int rounds = (tiles + waves - 1) / waves;
        if (rounds > kGtTmax) continue;
        const double eff = double(tiles) / (double(waves) * rounds);
        if (eff > best + 1e-9) {
            best = eff;
            pl.kw = kw;
            pl.lds = lds;
        }
    }
    if (!pl.kw) return pl;
    pl.ks = ks;
    pl.gs = gs;
    pl.mq = mq;
    pl.grid = nwu * ks;
    return pl;
}

template <int KIND>
void launch_gemvt_k(const GemvParams& p, const GtPlan& pl, hipStream_t stream) {
    constexpr int D = KIND == 1 ? 16 : 10;  // ~100 VGPRs of weights in flight
    allow_big_lds<gemvt_kernel<KIND, 1, D>>();
    allow_big_lds<gemvt_kernel<KIND, 2, D>>();
    allow_big_lds<gemvt_kernel<KIND, 3, D>>();
    allow_big_lds<gemvt_kernel<KIND, 4, D>>();
    switch (pl.mq) {
        case 1: gemvt_kernel<KIND, 1, D><<<pl.grid, 64 * pl.kw, pl.lds, stream>>>(p); break;
        case 2: gemvt_kernel<KIND, 2, D><<<pl.grid, 64 * pl.kw, pl.lds, stream>>>(p); break;
        case 3: gemvt_kernel<KIND, 3, D><<<pl.grid, 64 * pl.kw, pl.lds, stream>>>(p); break;
        default: gemvt_kernel<KIND, 4, D><<<pl.grid, 64 * pl.kw, pl.lds, stream>>>(p); break;
    }
}

// Batched GEMV with gemvt on n matrices sharing K (false: shape not covered).
bool launch_gemvt(const QView* W, const uint16_t* const* bias, float* const* y, int n, int M, Workspace* ws,
                  hipStream_t stream, hipError_t* err) {
    const int64_t K = W[0].cols, G = W[0].groups;
    if (K % kGroup) return false;
    const int tiles = total_tiles(W, n);
    const int cus = device_cu_count();
    for (int r0 = 0; r0 < M; r0 += 16) {
        const int mb = M - r0 < 16 ? M - r0 : 16;
        const GtPlan pl = gemvt_plan(G, tiles, mb, cus);
        if (!pl.kw || (pl.ks > 1 && int64_t(pl.ks) * mb * tiles * 16 > kPartialFloats)) {
            if (r0 == 0) return false;
            *err = hipErrorInvalidValue;  // a block after the first cannot fall back
            return true;
        }
        GemvParams p{};
        int t0 = 0;
        for (int i = 0; i < n; i++) {
            p.mat[i] = MatRef{W[i].q, W[i].scales, W[i].zeros, bias[i], y[i] + int64_t(r0) * W[i].rows,
                              W[i].rows, t0};
            t0 += int((W[i].rows + 15) / 16);
        }
        p.nmat = n;
        p.K = K;
        p.G = G;
        p.xq = ws->xq + int64_t(r0) * G * kLimbRec;
        p.meta = ws->xmeta + r0;
        p.part = ws->partials;
        p.M = mb;
        p.S = pl.ks;
        p.gs = pl.gs;
        p.ntiles = tiles;
        if (W[0].kind == 1) launch_gemvt_k<1>(p, pl, stream);
        else launch_gemvt_k<0>(p, pl, stream);
        if (pl.ks > 1) {
            const int64_t cnt = int64_t(mb) * tiles * 16;
            gemvt_reduce_kernel<<<unsigned((cnt + 255) / 256), 256, 0, stream>>>(p);
        }
        *err = hipGetLastError();
        if (*err != hipSuccess) return true;
    }
    return true;
}

// ------------------------------------------------------------------ 2..32 rows, f16 split
// Activations as two f16 terms, weights as exact f16 integers, on
// v_mfma_f32_16x16x32_f16.  Per (activation row m, 128-column group g):
// 2^k with max|x| 2^k in [2^14, 2^15), v = x 2^k (exact), hi = f16(v),
// lo = f16(v - hi); |v - hi - lo| <= 2^-22 max|v| (hi has 11 significant
// bits, v - hi is exact in fp32 and lo keeps 11 more), so the error per
// value is within 2^-22 of the group maximum, as with the byte limbs.  The
// weights enter as q (int8) or q - z (int4), integers f16 holds exactly, so
// every product is exact and the matrix core accumulates in fp32; per group
// the kernel adds D * (s * 2^-k) to the running sums.
//
// Prepared layout (xhprep): per block of 16 rows b and group g, 8 KiB =
// [MFMA k-chunk j = 0..3][term hi, lo][lane 0..63][8 f16], lane l = (row
// i = l % 16, q = l / 16) holding x[16 b + i][128 g + 32 q + 8 j + c(e)] for
// its 8 slots e, c(e) = perm8(e) for int4 weights (the order in which
// dq_int4_x8 leaves the nibbles) and e for int8; and per (b, g) the 16
// factors 2^-k (NaN when the group holds a non-finite value, so the outputs
// it reaches are NaN).  Every A operand is then one contiguous 1 KiB load.
constexpr int kHGroupBytes = 4 * 2 * 64 * 16;  // prepared bytes per (block, group)

// The f16 split of one lane's 8 values of a (row, group): all 16 lanes of a
// DPP row hold the group's 128 values (the group maximum is taken across
// them).  ho / lo: the hi and lo terms in operand slot order (perm8 for int4
// weights); fac: 2^-k, or NaN when the group holds a non-finite value.
template <bool PERM>
__device__ __forceinline__ void xh_split8(const float (&v)[8], half8_t& ho, half8_t& lo, float& fac) {
    // largest |x| bits over the 16 lanes; a NaN or an infinity has larger
    // bits (>= 0x7F800000) than any finite value, so one test of the
    // maximum finds any of them
    uint32_t am = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t a = __float_as_uint(v[i]) & 0x7FFFFFFFu;
        am = a > am ? a : am;
    }
    am = row16_max_u32(am);
    const bool fin = am < 0x7F800000u;
    // amax = f 2^E, f in [0.5, 1): k = 15 - E puts amax 2^k in [2^14, 2^15)
    const int k = (am > 0 && fin) ? 15 - __builtin_amdgcn_frexp_expf(__uint_as_float(am)) : 0;
    // operand dword j: values (j, j + 4) with PERM, else (2j, 2j + 1).
    // (A group with a non-finite value keeps its values: fac is NaN, so its
    // row's outputs are NaN whatever the operand holds, and an MFMA output
    // row reads only its own operand row.)
    u32x4_t hw, lw;
#pragma unroll
    for (int j = 0; j < 4; j++) {
        const int e0 = PERM ? j : 2 * j, e1 = PERM ? j + 4 : 2 * j + 1;
        const float s0 = __builtin_amdgcn_ldexpf(v[e0], k);
        const float s1 = __builtin_amdgcn_ldexpf(v[e1], k);
        half2_t h, l;
        h[0] = _Float16(s0);
        h[1] = _Float16(s1);
        const uint32_t hb = h2_bits(h);
        const float b0 = float(__builtin_bit_cast(_Float16, uint16_t(hb)));
        const float b1 = float(__builtin_bit_cast(_Float16, uint16_t(hb >> 16)));
        l[0] = _Float16(s0 - b0);
        l[1] = _Float16(s1 - b1);
        hw[j] = hb;
        lw[j] = h2_bits(l);
    }
    ho = __builtin_bit_cast(half8_t, hw);
    lo = __builtin_bit_cast(half8_t, lw);
    fac = fin ? __builtin_amdgcn_ldexpf(1.0f, -k) : __builtin_nanf("");
}

// PK (M <= 8): one A operand per k-chunk holds both terms, rows 0..7 the hi
// and rows 8..15 the lo terms of the 8 activation rows (4 KiB per group,
// half the operand bytes and MFMAs); the kernel adds the two halves of each
// output at the end.
template <bool PERM, bool PK>
__global__ __launch_bounds__(256) void xhprep_kernel(const float* __restrict__ x, int M, int64_t K, int64_t G,
                                                     int64_t quads, int nb, _Float16* __restrict__ xh,
                                                     float* __restrict__ xfx) {
    const int lane = threadIdx.x & 63, j16 = lane & 15;
    const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (wave >= int64_t(nb) * 16 * quads) return;
    const int m = int(wave / quads);  // 0 .. 16 nb - 1 (rows past M are written as zeros)
    const int64_t g = (wave % quads) * 4 + (lane >> 4);
    const bool gvalid = g < G;
    float v[8];
    load_x8<1>(x + int64_t(m < M ? m : 0) * K, (gvalid && m < M ? g : 0) * kGroup + j16 * 8,
               (gvalid && m < M) ? K : 0, v);
    half8_t ho, lo2;
    float fac;
    xh_split8<PERM>(v, ho, lo2, fac);
    if (!gvalid) return;
    const int b = m >> 4, i = m & 15, q = j16 >> 2, jj = j16 & 3;
    if (PK) {
        if (m >= 8) return;
        _Float16* base = xh + (g * (kHGroupBytes / 2)) / 2;
        *reinterpret_cast<half8_t*>(base + (jj * 64 + i + 16 * q) * 8) = ho;
        *reinterpret_cast<half8_t*>(base + (jj * 64 + i + 8 + 16 * q) * 8) = lo2;
    } else {
        _Float16* base = xh + ((int64_t(b) * G + g) * kHGroupBytes) / 2;
        const int l = i + 16 * q;
        *reinterpret_cast<half8_t*>(base + ((jj * 2 + 0) * 64 + l) * 8) = ho;
        *reinterpret_cast<half8_t*>(base + ((jj * 2 + 1) * 64 + l) * 8) = lo2;
    }
    if (j16 == 0) xfx[(int64_t(b) * G + g) * 16 + i] = fac;
}

// xhprep_kernel's output (16-row blocks, not packed) from a chain stage's
// input: activation row m read through the prologue's gather and RMSNorm
// (pro_x_offset, pro_norm8).  Each wave takes one (row, 4 groups) and
// computes its row's factor r_m itself, in ProScale's order (lane j < 16
// adds partials j, j + 16, ... in double, then the 16 sums in order), and
// multiplies the group factor by it after the split, so the operands and
// factors equal those the prologue instances make.
template <bool PERM>
__global__ __launch_bounds__(256) void xhprep_pro_kernel(const GemvParams p, int64_t quads, int nb,
                                                         _Float16* __restrict__ xh, float* __restrict__ xfx) {
    const int lane = threadIdx.x & 63, j16 = lane & 15;
    const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (wave >= int64_t(nb) * 16 * quads) return;
    const int M = p.M;
    const int64_t G = p.G;
    const int m = int(wave / quads);  // rows past M are written as zeros
    const int64_t g = (wave % quads) * 4 + (lane >> 4);
    const bool ok = g < G && m < M;
    const int64_t c = (ok ? g : 0) * kGroup + j16 * 8;
    const rsrc_t rx = make_rsrc(p.x, int64_t(M) * p.xstride * 4);
    const uint32_t o = ok ? pro_x_offset(p, m, c) : kOob;
    const float4_t a = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 0, 0));
    const float4_t bq = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, o, 16, 0));
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
        v[e] = a[e];
        v[4 + e] = bq[e];
    }
    float r = 1.0f;
    if (p.norm) {  // uniform
        const rsrc_t rn = make_rsrc(p.norm, p.K * 2);
        const uint4 nw = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rn, ok ? uint32_t(c) * 2 : kOob, 0, 0));
        const rsrc_t rq = make_rsrc(p.ssq, int64_t(M) * p.ssq_n * 4);
        double part = 0.0;
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int bb = lane + 16 * k;
            const float sq = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                           rq, (lane < 16 && m < M && bb < p.ssq_n) ? uint32_t(m * p.ssq_n + bb) * 4 : kOob, 0, 0));
            part += double(sq);
        }
        // the operands split x w; r_m joins the group factor after the split
        pro_norm8(v, nw);
        double ss = 0.0;
#pragma unroll
        for (int j = 0; j < 16; j++) ss += __shfl(part, j, 64);
        r = 1.0f / __builtin_sqrtf(float(ss / double(p.K)) + p.eps);
    }
    half8_t ho, lo2;
    float fac;
    xh_split8<PERM>(v, ho, lo2, fac);
    fac *= r;
    if (g >= G) return;
    const int b = m >> 4, i = m & 15, q = j16 >> 2, jj = j16 & 3;
    _Float16* base = xh + ((int64_t(b) * G + g) * kHGroupBytes) / 2;
    const int l = i + 16 * q;
    *reinterpret_cast<half8_t*>(base + ((jj * 2 + 0) * 64 + l) * 8) = ho;
    *reinterpret_cast<half8_t*>(base + ((jj * 2 + 1) * 64 + l) * 8) = lo2;
    if (j16 == 0) xfx[(int64_t(b) * G + g) * 16 + i] = fac;
}

// Workgroup = T consecutive 16-row tiles (of any of the call's matrices) x
// KS waves, wave w taking groups [w gs, w gs + gs) of every tile; per group a
// wave loads the 8 prepared A operands once (contiguous 1 KiB each, from
// L2) and applies them to its T tiles' weights, with the next group's loads
// in flight.  Slice sums are added through LDS in wave order
// (deterministic).  p.M <= 16 rows of the block; p.xq / p.meta point at the
// block's prepared operands and factors.
template <int KIND, int T, bool PK, bool D3 = false>
__global__ __launch_bounds__(T == 1 ? 1024 : 512) void gemvh_kernel(const GemvParams p) {
    extern __shared__ float hred[];  // [T][KS][4][64]
    constexpr int WPG = KIND == 1 ? 1 : 2;
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int KS = int(blockDim.x) >> 6;
    const int G = int(p.G);
    const int g0 = wave * p.gs < G ? wave * p.gs : G;
    const int g1 = g0 + p.gs < G ? g0 + p.gs : G;
    const int tb = int(blockIdx.x) * T;
    const int row_bytes = int(KIND == 1 ? p.K / 2 : p.K);

    rsrc_t rq[T], rs[T], rz[T];
#pragma unroll
    for (int t = 0; t < T; t++) {
        const bool ok = tb + t < p.ntiles;
        const TileSel ts = select_tile(p, ok ? tb + t : p.ntiles - 1);
        const int64_t left = ts.m.N - ts.row0;
        const int64_t rows = ok ? (left < 16 ? left : 16) : 0;
        rq[t] = make_rsrc_wave(ts.m.q + ts.row0 * row_bytes, rows * row_bytes);
        rs[t] = make_rsrc_wave(ts.m.scales + ts.row0 * G, rows * G * 2);
        rz[t] = make_rsrc_wave(KIND == 1 ? ts.m.zeros + ts.row0 * G : nullptr, KIND == 1 ? rows * G : 0);
    }
    constexpr int NA = PK ? 4 : 8;  // A operands per group
    const rsrc_t ra = make_rsrc(p.xq, int64_t(G) * NA * 1024);
    const rsrc_t rf = make_rsrc(p.meta, int64_t(G) * 64);
    const uint32_t vq = uint32_t(ln * row_bytes + q * (KIND == 1 ? 16 : 32));
    const uint32_t vs = uint32_t(ln * G) * 2, vz = uint32_t(ln * G);

    struct GB {
        int4v_t a[NA];      // [j][term], or [j] with both terms (PK)
        float4_t fx;        // 2^-k of activation rows 4q .. 4q + 3
        int4v_t w[T][WPG];
        // raw bits: widening a loaded value right after the request would
        // wait for every request made before it
        uint16_t s[T];
        uint8_t z[T];
    };
    auto load = [&](int g, GB& b) {
#pragma unroll
        for (int c = 0; c < NA; c++)
            b.a[c] = __builtin_bit_cast(int4v_t,
                                        __builtin_amdgcn_raw_buffer_load_b128(ra, uint32_t(lane * 16), g * NA * 1024 + c * 1024, 0));
        // factors of this lane's activation rows (PK: rows 4q .. 4q + 3 mod 8)
        b.fx = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rf, uint32_t((PK ? q & 1 : q) * 16), g * 64, 0));
#pragma unroll
        for (int t = 0; t < T; t++) {
#pragma unroll
            for (int h = 0; h < WPG; h++)
                b.w[t][h] = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                            rq[t], vq, g * (KIND == 1 ? 64 : 128) + h * 16, 0));
            b.s[t] = __builtin_amdgcn_raw_buffer_load_b16(rs[t], vs, g * 2, 0);
            b.z[t] = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b8(rz[t], vz, g, 0) : 0u;
        }
    };
    float acc[T][4];
#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) acc[t][r] = 0.0f;
    auto compute = [&](const GB& b) {
#pragma unroll
        for (int t = 0; t < T; t++) {
            half8_t B[4];
            if (KIND == 1) {
                const uint32_t zb = zpair_1024(b.z[t]), zc = zpair_64(b.z[t]);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    uint32_t o0, o1, o2, o3;
                    dq_int4_x8(uint32_t(b.w[t][0][j]), zb, zc, o0, o1, o2, o3);
                    B[j] = pack_h8(o0, o1, o2, o3);
                }
            } else {
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    uint32_t l0, h0, l1, h1;
                    const int4v_t& wv = b.w[t][j >> 1];
                    dq_int8_x4(uint32_t(wv[2 * (j & 1)]), l0, h0);
                    dq_int8_x4(uint32_t(wv[2 * (j & 1) + 1]), l1, h1);
                    B[j] = pack_h8(l0, h0, l1, h1);
                }
            }
            float4_t D = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; j++) {
                if (PK) {
                    D = mfma16(__builtin_bit_cast(half8_t, b.a[j]), B[j], D);
                } else {
                    D = mfma16(__builtin_bit_cast(half8_t, b.a[2 * j]), B[j], D);
                    D = mfma16(__builtin_bit_cast(half8_t, b.a[2 * j + 1]), B[j], D);
                }
            }
            const float s = __uint_as_float(uint32_t(b.s[t]) << 16);
#pragma unroll
            for (int r = 0; r < 4; r++) acc[t][r] = __builtin_fmaf(D[r], s * b.fx[r], acc[t][r]);
        }
    };
    if constexpr (D3) {
        // two groups in flight while one is multiplied
        GB b0, b1, b2;
        if (g0 < g1) load(g0, b0);
        if (g0 + 1 < g1) load(g0 + 1, b1);
        for (int g = g0; g < g1; g += 3) {
            if (g + 2 < g1) load(g + 2, b2);
            compute(b0);
            if (g + 1 >= g1) break;
            if (g + 3 < g1) load(g + 3, b0);
            compute(b1);
            if (g + 2 >= g1) break;
            if (g + 4 < g1) load(g + 4, b1);
            compute(b2);
        }
    } else {
        GB b0, b1;
        if (g0 < g1) load(g0, b0);
        for (int g = g0; g < g1; g += 2) {
            if (g + 1 < g1) load(g + 1, b1);
            compute(b0);
            if (g + 1 >= g1) break;
            if (g + 2 < g1) load(g + 2, b0);
            compute(b1);
        }
    }

#pragma unroll
    for (int t = 0; t < T; t++)
#pragma unroll
        for (int r = 0; r < 4; r++) hred[((t * KS + wave) * 4 + r) * 64 + lane] = acc[t][r];
    __syncthreads();
    for (int o = tid; o < T * 256; o += int(blockDim.x)) {
        const int t = o >> 8, r = (o >> 6) & 3, l = o & 63;
        const int m = 4 * (l >> 4) + r, n = l & 15;
        if (m >= p.M || tb + t >= p.ntiles) continue;
        float sum = 0.0f;
        for (int w = 0; w < KS; w++) sum += hred[((t * KS + w) * 4 + r) * 64 + l];
        if (PK) {
            // rows 8..15 of the operand carried the lo terms: lane l + 32
            float lo = 0.0f;
            for (int w = 0; w < KS; w++) lo += hred[((t * KS + w) * 4 + r) * 64 + l + 32];
            sum += lo;
        }
        const TileSel ts = select_tile(p, tb + t);
        const int64_t row = ts.row0 + n;
        float v = sum + (ts.m.bias && row < ts.m.N ? bf16_to_f32(ts.m.bias[row]) : 0.0f);
        if (p.res && row < ts.m.N) v = p.res[int64_t(m) * ts.m.N + row] + v;
        if (row < ts.m.N) ts.m.y[int64_t(m) * ts.m.N + row] = v;
        if (p.ssq_out) {
            // (the 16 lanes n of (t, m) are one DPP row and take this branch
            // together: m and t are the same for all of them)
            float sq = row < ts.m.N ? v * v : 0.0f;
            sq += __int_as_float(row_ror<8>(__float_as_int(sq)));
            sq += __int_as_float(row_ror<4>(__float_as_int(sq)));
            sq += __int_as_float(row_ror<2>(__float_as_int(sq)));
            sq += __int_as_float(row_ror<1>(__float_as_int(sq)));
            if (n == 0) p.ssq_out[int64_t(m) * p.ntiles + tb + t] = sq;
        }
    }
}

// 7..16 rows on the prepared f16 split operands (16-row blocks), shared
// through LDS: workgroup = 8 waves on 8 consecutive 16-row tiles (wave w:
// tile 8 b + w, over every matrix of the call) and one K range of groups
// [g0, g1).  Per group the workgroup copies the group's 8 KiB of A operands
// (4 k-chunks x hi, lo) into LDS once (one 16-byte load per thread, the next
// group's in registers), and every wave multiplies them by its own tile's
// weights, which stream D groups ahead in registers.  A operand bytes read
// from L2 per weight byte: 1 (int4) / 0.5 (int8) instead of the 8 / 4 of a
// wave that loads the operands for its tile alone.  S > 1 ranges write fp32
// partial sums that gemvt_reduce_kernel adds in range order.
template <int KIND>
__global__ __launch_bounds__(512, 2) void gemvs_kernel(const GemvParams p) {
    constexpr int D = 4;  // weight groups in flight per wave
    constexpr int WPG = KIND == 1 ? 1 : 2;
    __shared__ __attribute__((aligned(16))) int4v_t As[2][512];
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = int(p.G);
    const int nrb = (p.ntiles + 7) / 8;
    const int rb = int(blockIdx.x) % nrb, range = int(blockIdx.x) / nrb;
    const int g0 = range * p.gs, g1 = g0 + p.gs < G ? g0 + p.gs : G;
    const int tile = rb * 8 + wave;
    const bool tok = tile < p.ntiles;
    const TileSel ts = select_tile(p, tok ? tile : p.ntiles - 1);
    const int row_bytes = int(KIND == 1 ? p.K / 2 : p.K);
    const int64_t left = ts.m.N - ts.row0;
    const int64_t rows = tok ? (left < 16 ? left : 16) : 0;
    const rsrc_t rq = make_rsrc_wave(ts.m.q + ts.row0 * row_bytes, rows * row_bytes);
    const rsrc_t rs = make_rsrc_wave(ts.m.scales + ts.row0 * G, rows * G * 2);
    const rsrc_t rz = make_rsrc_wave(KIND == 1 ? ts.m.zeros + ts.row0 * G : nullptr, KIND == 1 ? rows * G : 0);
    const rsrc_t ra = make_rsrc(p.xq, int64_t(G) * kHGroupBytes);
    const rsrc_t rf = make_rsrc(p.meta, int64_t(G) * 64);
    const uint32_t vq = uint32_t(ln * row_bytes + q * (KIND == 1 ? 16 : 32));
    const uint32_t vs = uint32_t(ln * G) * 2, vz = uint32_t(ln * G);

    // Everything a group needs (its A operand share, this wave's weights,
    // scale, zero point and row factors) is requested together, D groups
    // ahead, into one of D register slots: the memory counter completes in
    // request order, so a wait for one group's data never waits for a
    // request made later than D - 1 groups before it.
    struct Slot {
        int4v_t a;
        int4v_t w[WPG];
        uint16_t s;  // raw bits (see gemvh_kernel)
        uint8_t z;
        float4_t fx;
    };
    auto load = [&](int g, Slot& b) {
        const uint32_t off = g < g1 ? 0u : kOob;
        b.a = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(ra, uint32_t(tid * 16) + off,
                                                                                 g * kHGroupBytes, 0));
#pragma unroll
        for (int h = 0; h < WPG; h++)
            b.w[h] = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                     rq, vq + off, g * (KIND == 1 ? 64 : 128) + h * 16, 0));
        b.s = __builtin_amdgcn_raw_buffer_load_b16(rs, vs + off, g * 2, 0);
        b.z = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b8(rz, vz + off, g, 0) : 0u;
        b.fx = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rf, uint32_t(q * 16) + off, g * 64, 0));
    };
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](const Slot& b, int buf) {
        half8_t B[4];
        if (KIND == 1) {
            const uint32_t zb = zpair_1024(b.z), zc = zpair_64(b.z);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t o0, o1, o2, o3;
                dq_int4_x8(uint32_t(b.w[0][j]), zb, zc, o0, o1, o2, o3);
                B[j] = pack_h8(o0, o1, o2, o3);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t l0, h0, l1, h1;
                const int4v_t& wv = b.w[j >> 1];
                dq_int8_x4(uint32_t(wv[2 * (j & 1)]), l0, h0);
                dq_int8_x4(uint32_t(wv[2 * (j & 1) + 1]), l1, h1);
                B[j] = pack_h8(l0, h0, l1, h1);
            }
        }
        float4_t Dv = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; j++) {
            Dv = mfma16(__builtin_bit_cast(half8_t, As[buf][(2 * j) * 64 + lane]), B[j], Dv);
            Dv = mfma16(__builtin_bit_cast(half8_t, As[buf][(2 * j + 1) * 64 + lane]), B[j], Dv);
        }
        const float sc = __uint_as_float(uint32_t(b.s) << 16);
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(Dv[r], sc * b.fx[r], acc[r]);
    };

    Slot s0, s1, s2, s3;
    load(g0, s0);
    load(g0 + 1, s1);
    load(g0 + 2, s2);
    load(g0 + 3, s3);
    As[0][tid] = s0.a;
    // group g: operands in As[(g - g0) & 1] (stored at the previous step),
    // weights in slot (g - g0) % D; the slot is refilled with group g + D
    auto iter = [&](int g, Slot& cur, const Slot& next) {
        __syncthreads();
        const int par = (g - g0) & 1;
        if (g + 1 < g1) As[par ^ 1][tid] = next.a;
        compute(cur, par);
        load(g + D, cur);
    };
    for (int g = g0; g < g1; g += D) {
        iter(g, s0, s1);
        if (g + 1 >= g1) break;
        iter(g + 1, s1, s2);
        if (g + 2 >= g1) break;
        iter(g + 2, s2, s3);
        if (g + 3 >= g1) break;
        iter(g + 3, s3, s0);
    }
    if (!tok) return;
    const int64_t ld = int64_t(p.ntiles) * 16;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = 4 * q + r;
        if (m >= p.M || ln >= rows) continue;
        if (p.S == 1) {
            const int64_t row = ts.row0 + ln;
            ts.m.y[int64_t(m) * ts.m.N + row] = acc[r] + (ts.m.bias ? bf16_to_f32(ts.m.bias[row]) : 0.0f);
        } else {
            p.part[(int64_t(range) * p.M + m) * ld + int64_t(tile) * 16 + ln] = acc[r];
        }
    }
}

// 5..16 rows, a K range of at most 8 groups per workgroup, everything
// requested at once: workgroup = 8 waves on 8 consecutive 16-row tiles;
// each thread requests its share of the range's activations (fp32, 16 rows
// x 8 groups, no preparation launch) and each lane its row's scales, zero
// points and weights for the whole range (64 contiguous bytes of one row
// per group, 8 groups in flight per wave), like the 1-row kernel.  While
// the weights are in flight the workgroup makes the range's f16 split
// operands and row factors in LDS exactly as xhprep_kernel makes them
// (xh_split8; PK: the packed form), one barrier, and every wave multiplies
// its weights by the range's operands group by group as they land.  S > 1
// ranges write fp32 partial sums (gemvt_reduce_kernel).
template <int KIND, bool PK, int NG, bool PRO = false>
// (the second bound is the minimum waves per SIMD: 4 caps the registers at
// 128, two 8-wave workgroups per CU; the prologue's instances rose to 132
// under a bound of 2, one workgroup per CU.  Not the int8 prologue
// instance, which would spill.)
__global__ __launch_bounds__(512, NG > 8 ? 1 : ((PRO && KIND == 0 && !PK) ? 2 : 4)) void gemvr_kernel(const GemvParams p) {
    constexpr int WPG = KIND == 1 ? 1 : 2;
    // operand chunks of a group 65 16-byte slots apart (not 64): a row's
    // 16-byte stores from the conversion spread over the bank groups
    // instead of hitting one; the MFMA's reads stay contiguous
    constexpr int CS = 65;
    constexpr int GB = (PK ? 4 : 8) * CS * 16;  // operand bytes per group
    __shared__ __attribute__((aligned(16))) int8_t As[NG][GB];
    __shared__ __attribute__((aligned(16))) float4_t Fs[NG][4];
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = int(p.G);
    const int nrb = (p.ntiles + 7) / 8;
    const int rb = int(blockIdx.x) % nrb, range = int(blockIdx.x) / nrb;
    const int g0 = range * p.gs, gs = (g0 + p.gs < G ? g0 + p.gs : G) - g0;
    const int tile = rb * 8 + wave;
    const bool tok = tile < p.ntiles;
    const TileSel ts = select_tile(p, tok ? tile : p.ntiles - 1);
    const int row_bytes = int(KIND == 1 ? p.K / 2 : p.K);
    const int64_t left = ts.m.N - ts.row0;
    const int64_t rows = tok ? (left < 16 ? left : 16) : 0;
    const rsrc_t rq = make_rsrc_wave(ts.m.q + ts.row0 * row_bytes, rows * row_bytes);
    const rsrc_t rs = make_rsrc_wave(ts.m.scales + ts.row0 * G, rows * G * 2);
    const rsrc_t rz = make_rsrc_wave(KIND == 1 ? ts.m.zeros + ts.row0 * G : nullptr, KIND == 1 ? rows * G : 0);
    const uint32_t vq = uint32_t(ln * row_bytes + q * (KIND == 1 ? 16 : 32));
    const uint32_t vs = uint32_t(ln * G) * 2, vz = uint32_t(ln * G);

    // 1. the range's activations, then this lane's scales, zero points and
    //    weights; slots past the range (and rows past M) read zero without
    //    a memory access (buffer range check).  Activation task t = tid +
    //    512 u is lane t % 16 of (row m, group i), 8 values.
    constexpr int NX = (PK ? 8 : 16) * NG * 16 / 512;
    static_assert(NX * 512 == (PK ? 8 : 16) * NG * 16, "whole DPP rows per task set");
    float xv[NX][8];
    uint4 nwv[PRO ? NX : 1];
    ProScale psc;
    if constexpr (PRO) psc.request(p, tid);
    {
        const rsrc_t rxx = make_rsrc(p.x, int64_t(p.M) * (PRO ? p.xstride : p.K) * 4);
        const rsrc_t rn = make_rsrc(PRO ? p.norm : nullptr, PRO && p.norm ? p.K * 2 : 0);
#pragma unroll
        for (int u = 0; u < NX; u++) {
            const int t = tid + 512 * u, j16 = t & 15, pr = t >> 4;
            const int m = PK ? pr & 7 : pr & 15, i = PK ? pr >> 3 : pr >> 4;
            const int64_t c = int64_t(g0 + i) * kGroup + j16 * 8;
            const bool ok = i < gs && m < p.M;
            const uint32_t o = !ok ? kOob : (PRO ? pro_x_offset(p, m, c) : uint32_t((int64_t(m) * p.K + c) * 4));
            const float4_t a = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rxx, o, 0, 0));
            const float4_t b = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rxx, o, 16, 0));
            if constexpr (PRO)
                nwv[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rn, ok ? uint32_t(c) * 2 : kOob, 0, 0));
#pragma unroll
            for (int e = 0; e < 4; e++) {
                xv[u][e] = a[e];
                xv[u][4 + e] = b[e];
            }
        }
    }
    uint16_t sv[NG];
    uint8_t zv[NG];
    int4v_t wv[NG][WPG];
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const uint32_t o = i < gs ? 0u : kOob;
        sv[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, vs + o, (g0 + i) * 2, 0);
        zv[i] = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b8(rz, vz + o, g0 + i, 0) : 0u;
    }
#pragma unroll
    for (int i = 0; i < NG; i++) {
        const uint32_t o = i < gs ? 0u : kOob;
#pragma unroll
        for (int h = 0; h < WPG; h++)
            wv[i][h] = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rq, vq + o, (g0 + i) * (KIND == 1 ? 64 : 128) + h * 16, 0));
    }
    // 2. the operands and factors of the range (all 16 lanes of each
    //    (row, group) together), then one barrier
    //    (with RMSNorm: the operands split x w, and the row factor r_m joins
    //    the group factor once the producer's sums of squares are added)
    __shared__ double rsp[PRO ? kMaxRowsGemv : 1][16];
    __shared__ float rsc[PRO ? kMaxRowsGemv : 1];
#pragma unroll
    for (int u = 0; u < NX; u++) {
        const int t = tid + 512 * u, j16 = t & 15, pr = t >> 4;
        const int m = PK ? pr & 7 : pr & 15, i = PK ? pr >> 3 : pr >> 4;
        const int qq = j16 >> 2, jj = j16 & 3;
        if constexpr (PRO) {
            if (p.norm) pro_norm8(xv[u], nwv[u]);
        }
        half8_t ho, lo;
        float fac;
        xh_split8<KIND == 1>(xv[u], ho, lo, fac);
        half8_t* dst = reinterpret_cast<half8_t*>(As[i]);
        if (PK) {
            dst[jj * CS + m + 16 * qq] = ho;
            dst[jj * CS + m + 8 + 16 * qq] = lo;
        } else {
            dst[(jj * 2) * CS + m + 16 * qq] = ho;
            dst[(jj * 2 + 1) * CS + m + 16 * qq] = lo;
        }
        if (j16 == 0) reinterpret_cast<float*>(Fs[i])[m] = fac;
    }
    if constexpr (PRO) {
        if (p.norm) {  // workgroup-uniform
            psc.finish(p, tid, rsp, rsc);
            // (each factor rescaled by the thread that stored it)
#pragma unroll
            for (int u = 0; u < NX; u++) {
                const int t = tid + 512 * u, j16 = t & 15, pr = t >> 4;
                const int m = PK ? pr & 7 : pr & 15, i = PK ? pr >> 3 : pr >> 4;
                if (j16 == 0) reinterpret_cast<float*>(Fs[i])[m] *= rsc[m < p.M ? m : 0];
            }
        }
    }
    __syncthreads();

    // 3. the groups in order, each as its weights land
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int i = 0; i < NG; i++) {
        if (i >= gs) continue;  // workgroup-uniform
        half8_t B[4];
        if (KIND == 1) {
            const uint32_t zb = zpair_1024(zv[i]), zc = zpair_64(zv[i]);
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t o0, o1, o2, o3;
                dq_int4_x8(uint32_t(wv[i][0][j]), zb, zc, o0, o1, o2, o3);
                B[j] = pack_h8(o0, o1, o2, o3);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                uint32_t l0, h0, l1, h1;
                const int4v_t& w = wv[i][j >> 1];
                dq_int8_x4(uint32_t(w[2 * (j & 1)]), l0, h0);
                dq_int8_x4(uint32_t(w[2 * (j & 1) + 1]), l1, h1);
                B[j] = pack_h8(l0, h0, l1, h1);
            }
        }
        float4_t Dv = {0.0f, 0.0f, 0.0f, 0.0f};
        const int4v_t* Ai = reinterpret_cast<const int4v_t*>(As[i]);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            if (PK) {
                // one operand per k-chunk: A rows 0..7 the hi, 8..15 the lo terms
                Dv = mfma16(__builtin_bit_cast(half8_t, Ai[j * CS + lane]), B[j], Dv);
            } else {
                Dv = mfma16(__builtin_bit_cast(half8_t, Ai[(2 * j) * CS + lane]), B[j], Dv);
                Dv = mfma16(__builtin_bit_cast(half8_t, Ai[(2 * j + 1) * CS + lane]), B[j], Dv);
            }
        }
        const float sc = __uint_as_float(uint32_t(sv[i]) << 16);
        // (PK: lanes of D rows 8..15 hold the lo terms of rows 0..7)
        const float4_t fx = Fs[i][PK ? q & 1 : q];
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] = __builtin_fmaf(Dv[r], sc * fx[r], acc[r]);
    }
    if (PK) {
        // row m's lo-term sums sit 32 lanes above its hi-term sums
#pragma unroll
        for (int r = 0; r < 4; r++) acc[r] += __shfl_down(acc[r], 32, 64);
    }
    if (!tok || (PK && q >= 2)) return;
    const int64_t ld = int64_t(p.ntiles) * 16;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = 4 * q + r;
        if (m >= p.M || ln >= rows) continue;
        if (p.S == 1 && !(PRO && p.to_part)) {
            const int64_t row = ts.row0 + ln;
            ts.m.y[int64_t(m) * ts.m.N + row] = acc[r] + (ts.m.bias ? bf16_to_f32(ts.m.bias[row]) : 0.0f);
        } else {
            p.part[(int64_t(range) * p.M + m) * ld + int64_t(tile) * 16 + ln] = acc[r];
        }
    }
}

// 9..16 rows on v_mfma_f32_32x32x16_f16: like gemvr (a K range of at most
// NG groups per workgroup, every request made at once, operands made from x
// in LDS while the weights are in flight), but each wave takes 32 weight
// rows (a 32-row tile of one matrix), and one A operand holds both terms of
// all 16 activation rows (A rows 0..15 the hi, 16..31 the lo terms), so each
// 1 KiB operand read from LDS feeds 32 weight rows instead of 16.  K order
// inside a group: lane half h = l / 32 of chunk c (16 columns per MFMA)
// covers columns 64 h + 8 c .. + 8 (int4 slots in perm8 order), so a lane's
// weights of a group are 32 (int4) or 64 (int8) contiguous bytes of its
// row.  D lane l, register r: A row 8 (r / 4) + 4 h + r % 4, weight row
// l % 32; registers r and r + 8 hold the two terms of one activation row.
// S > 1 ranges write fp32 partial sums in the 16-row tile order of the
// other kernels (gemvt_reduce_kernel adds them).  MB = 2 (17..32 rows):
// MB blocks of 16 activation rows, each group's dequantised weights (one
// chunk at a time) multiplied by every block's operand before the next
// chunk, so the weights are read and converted once for all the rows.
template <int KIND, int NG, int MB, bool LOOP, bool PRO = false>
// (bounds as gemvr_kernel's; the looped and int8 two-block prologue
// instances keep 2, where 4 would spill)
__global__ __launch_bounds__(512, (PRO && (LOOP || (KIND == 0 && MB == 2))) ? 2 : 4) void gemvq_kernel(const GemvParams p) {
    constexpr int NW = KIND == 1 ? 2 : 4;  // 16-byte weight loads per lane and group
    // [block][group][chunk][lane], chunks 65 slots apart: the conversion's
    // 16-byte stores of one row's 8 chunks then fall in 8 different bank
    // groups (64 apart they all hit one), the MFMA's reads stay contiguous
    __shared__ __attribute__((aligned(16))) half8_t Aq[MB][NG][8][65];
    __shared__ __attribute__((aligned(16))) float Fq[MB][NG][16];
    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int G = int(p.G);
    const int rb = int(blockIdx.x) % p.nrb, range = int(blockIdx.x) / p.nrb;
    // this wave's 32-row tile: matrix i holds tiles [t0, t0 + ceil(N / 32))
    const int tile = rb * 8 + wave;
    MatRef mr = p.mat[0];
    int t0 = 0, tot = 0;
#pragma unroll
    for (int i = 0; i < kMaxMulti; i++) {
        if (i < p.nmat) {
            if (tile >= tot) {
                mr = p.mat[i];
                t0 = tot;
            }
            tot += int((p.mat[i].N + 31) / 32);
        }
    }
    const bool tok = tile < tot;
    const int row_bytes = int(KIND == 1 ? p.K / 2 : p.K);
    const int64_t row0 = int64_t(tok ? tile - t0 : 0) * 32;
    const int64_t left = mr.N - row0;
    const int64_t rows = tok ? (left < 32 ? left : 32) : 0;
    const rsrc_t rq = make_rsrc_wave(mr.q + row0 * row_bytes, rows * row_bytes);
    const rsrc_t rs = make_rsrc_wave(mr.scales + row0 * G, rows * G * 2);
    const rsrc_t rz = make_rsrc_wave(KIND == 1 ? mr.zeros + row0 * G : nullptr, KIND == 1 ? rows * G : 0);
    const uint32_t vq = uint32_t(l32 * row_bytes + h * NW * 16);
    const uint32_t vs = uint32_t(l32 * G) * 2, vz = uint32_t(l32 * G);

    __shared__ double rsp[PRO ? kMaxRowsGemv : 1][16];
    __shared__ float rsc[PRO ? kMaxRowsGemv : 1];
    float acc[MB][8];
#pragma unroll
    for (int b = 0; b < MB; b++)
#pragma unroll
        for (int r = 0; r < 8; r++) acc[b][r] = 0.0f;
    // LOOP: p.kr consecutive K ranges per workgroup (when the partial sums
    // of one range per workgroup would not fit), accumulated in registers
    const int nit = LOOP ? p.kr : 1;
    for (int it = 0; it < nit; it++) {
        const int g0 = (range * nit + it) * p.gs;
        const int gs = g0 >= G ? 0 : (g0 + p.gs < G ? g0 + p.gs : G) - g0;
        if (it > 0) __syncthreads();  // the previous range's operands are read
        // 1. the range's activations (task t = tid + 512 u: lane t % 16 of
        //    (row 16 b + m, group i), 8 values, b = (t / 256) / NG, i = (t /
        //    256) % NG), then this lane's scales, zero points and weights;
        //    slots past the range and rows past M read zero without a memory
        //    access (buffer range check)
        constexpr int NX = MB * 16 * NG * 16 / 512;
        static_assert(NX * 512 == MB * 16 * NG * 16, "whole DPP rows per task set");
        float xv[NX][8];
        uint4 nwv[PRO ? NX : 1];
        ProScale psc;
        if constexpr (PRO) {
            if (it == 0) psc.request(p, tid);
        }
        {
            const rsrc_t rxx = make_rsrc(p.x, int64_t(p.M) * (PRO ? p.xstride : p.K) * 4);
            const rsrc_t rn = make_rsrc(PRO ? p.norm : nullptr, PRO && p.norm ? p.K * 2 : 0);
#pragma unroll
            for (int u = 0; u < NX; u++) {
                const int t = tid + 512 * u, j16 = t & 15, m = (t >> 4) & 15, i = (t >> 8) % NG;
                const int row = 16 * ((t >> 8) / NG) + m;
                const int64_t c = int64_t(g0 + i) * kGroup + j16 * 8;
                const bool ok = i < gs && row < p.M;
                const uint32_t o = !ok ? kOob : (PRO ? pro_x_offset(p, row, c) : uint32_t((int64_t(row) * p.K + c) * 4));
                const float4_t a = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rxx, o, 0, 0));
                const float4_t b = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rxx, o, 16, 0));
                if constexpr (PRO)
                    nwv[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rn, ok ? uint32_t(c) * 2 : kOob, 0, 0));
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    xv[u][e] = a[e];
                    xv[u][4 + e] = b[e];
                }
            }
        }
        uint16_t sv[NG];
        uint8_t zv[NG];
        int4v_t wv[NG][NW];
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const uint32_t o = i < gs ? 0u : kOob;
            sv[i] = __builtin_amdgcn_raw_buffer_load_b16(rs, vs + o, (g0 + i) * 2, 0);
            zv[i] = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b8(rz, vz + o, g0 + i, 0) : 0u;
        }
#pragma unroll
        for (int i = 0; i < NG; i++) {
            const uint32_t o = i < gs ? 0u : kOob;
#pragma unroll
            for (int c = 0; c < NW; c++)
                wv[i][c] = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                           rq, vq + o, (g0 + i) * (KIND == 1 ? 64 : 128) + c * 16, 0));
        }

        // 2. the range's operands and factors (16 lanes per (row, group)):
        //    octet j16 = 8 h' + c of row m goes to chunk c, lanes m + 32 h'
        //    (hi) and m + 16 + 32 h' (lo); then one barrier.  With RMSNorm
        //    the operands split x w and the row factor r_m joins the group
        //    factor afterwards, so the conversion does not wait for the
        //    producer's sums of squares.
#pragma unroll
        for (int u = 0; u < NX; u++) {
            const int t = tid + 512 * u, j16 = t & 15, m = (t >> 4) & 15, i = (t >> 8) % NG, b = (t >> 8) / NG;
            if constexpr (PRO) {
                if (p.norm) pro_norm8(xv[u], nwv[u]);
            }
            half8_t ho, lo;
            float fac;
            xh_split8<KIND == 1>(xv[u], ho, lo, fac);
            Aq[b][i][j16 & 7][m + 32 * (j16 >> 3)] = ho;
            Aq[b][i][j16 & 7][m + 16 + 32 * (j16 >> 3)] = lo;
            if (j16 == 0) Fq[b][i][m] = fac;
        }
        if constexpr (PRO) {
            if (p.norm) {  // workgroup-uniform
                if (it == 0) psc.finish(p, tid, rsp, rsc);
                // (each factor rescaled by the thread that stored it)
#pragma unroll
                for (int u = 0; u < NX; u++) {
                    const int t = tid + 512 * u, j16 = t & 15, m = (t >> 4) & 15, i = (t >> 8) % NG, b = (t >> 8) / NG;
                    const int row = 16 * b + m;
                    if (j16 == 0) Fq[b][i][m] *= rsc[row < p.M ? row : 0];
                }
            }
        }
        __syncthreads();

        // 3. the groups in order, each as its weights land
#pragma unroll
        for (int i = 0; i < NG; i++) {
            if (i >= gs) continue;  // workgroup-uniform
            float16_t D[MB];
#pragma unroll
            for (int b = 0; b < MB; b++) D[b] = float16_t{};
            const uint32_t zb = zpair_1024(zv[i]), zc = zpair_64(zv[i]);
#pragma unroll
            for (int c = 0; c < 8; c++) {
                half8_t B;
                if (KIND == 1) {
                    uint32_t o0, o1, o2, o3;
                    dq_int4_x8(uint32_t(wv[i][c >> 2][c & 3]), zb, zc, o0, o1, o2, o3);
                    B = pack_h8(o0, o1, o2, o3);
                } else {
                    uint32_t l0, h0, l1, h1;
                    const int4v_t& w = wv[i][c >> 1];
                    dq_int8_x4(uint32_t(w[2 * (c & 1)]), l0, h0);
                    dq_int8_x4(uint32_t(w[2 * (c & 1) + 1]), l1, h1);
                    B = pack_h8(l0, h0, l1, h1);
                }
#pragma unroll
                for (int b = 0; b < MB; b++) D[b] = __builtin_amdgcn_mfma_f32_32x32x16_f16(Aq[b][i][c][lane], B, D[b], 0, 0, 0);
            }
            const float sc = __uint_as_float(uint32_t(sv[i]) << 16);
#pragma unroll
            for (int b = 0; b < MB; b++) {
                const float4_t f0 = *reinterpret_cast<const float4_t*>(&Fq[b][i][4 * h]);
                const float4_t f1 = *reinterpret_cast<const float4_t*>(&Fq[b][i][8 + 4 * h]);
#pragma unroll
                for (int r = 0; r < 8; r++)
                    acc[b][r] = __builtin_fmaf(D[b][r] + D[b][r + 8], sc * (r < 4 ? f0[r] : f1[r - 4]), acc[b][r]);
            }
        }
    }
    if (!tok || l32 >= rows) return;
    const int64_t ld = int64_t(p.ntiles) * 16;
    const int64_t row = row0 + l32;
#pragma unroll
    for (int b = 0; b < MB; b++) {
#pragma unroll
        for (int r = 0; r < 8; r++) {
            const int m = 16 * b + 8 * (r >> 2) + 4 * h + (r & 3);
            if (m >= p.M) continue;
            if (p.S == 1 && !(PRO && p.to_part))
                mr.y[int64_t(m) * mr.N + row] = acc[b][r] + (mr.bias ? bf16_to_f32(mr.bias[row]) : 0.0f);
            else
                p.part[(int64_t(range) * p.M + m) * ld + int64_t(mr.tile0) * 16 + row] = acc[b][r];
        }
    }
}

// gemvr on n matrices, M in 5..16, straight from x (false: the partial sums
// would not fit).
bool launch_gemvr(const float* x, const QView* W, const uint16_t* const* bias, float* const* y, int n, int M, Workspace* ws,
                  hipStream_t stream, hipError_t* err) {
    const int64_t K = W[0].cols, G = W[0].groups;
    GemvParams p{};
    int tiles = 0;
    for (int i = 0; i < n; i++) {
        p.mat[i] = MatRef{W[i].q, W[i].scales, W[i].zeros, bias[i], y[i], W[i].rows, tiles};
        tiles += int((W[i].rows + 15) / 16);
    }
    const int nrb = (tiles + 7) / 8;
    // ranges of at most 8 groups (16: one workgroup per CU, 7B gate|up at
    // 16 rows 38.5 -> 53.9 us), and enough workgroups for two per CU
    constexpr int ngr = 8;
    const int want = 2 * device_cu_count();
    int S = int((G + ngr - 1) / ngr);
    S = std::max<int>(S, std::min<int>((want + nrb - 1) / nrb, int(G)));
    const int gs = int((G + S - 1) / S);
    S = int((G + gs - 1) / gs);
    if (S > 1 && int64_t(S) * M * tiles * 16 > kPartialFloats) return false;
    p.nmat = n;
    p.K = K;
    p.G = G;
    p.x = x;
    p.M = M;
    p.gs = gs;
    p.S = S;
    p.ntiles = tiles;
    p.part = ws->partials;
    const unsigned grid = unsigned(nrb * S);
    if (M <= 8) {
        if (W[0].kind == 1) gemvr_kernel<1, true, 8><<<grid, 512, 0, stream>>>(p);
        else gemvr_kernel<0, true, 8><<<grid, 512, 0, stream>>>(p);
    } else {
        if (W[0].kind == 1) gemvr_kernel<1, false, 8><<<grid, 512, 0, stream>>>(p);
        else gemvr_kernel<0, false, 8><<<grid, 512, 0, stream>>>(p);
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && S > 1) {
        const int64_t outs = int64_t(M) * tiles * 16;
        gemvt_reduce_kernel<<<unsigned((outs + 255) / 256), 256, 0, stream>>>(p);
        e = hipGetLastError();
    }
    *err = e;
    return true;
}

// 17..32 rows on gemvq's two 16-row blocks instead of the GEMM's 64-row
// tiles, for calls of >= 224 16-row tiles (N >= 3584), long rows or several
// matrices (7B, fp32 activations, int8 / int4 at 17 / 32 rows: gate 18944 x
// 3584 43.9 -> 29.9 / 48.7 -> 34.7 us, down 3584 x 18944 43.3 -> 35.8 / 46.3
// -> 38.1 us, o 3584 x 3584 20.2 -> 17.3 / 21.2 -> 19.8 (int4 20.4 -> 16.5
// / 22.1 -> 19.6), 1.5B gate 8960 x 1536 19.5 -> 16.9 / 21.4 -> 20.0, 3584
// x 2048 15.5 -> 12.5 / 17.4 -> 14.0 us; q|k|v as one call, which the GEMM
// takes one launch sequence per matrix, 59 / 63 -> 24 / 25 us at 24 / 32
// rows); narrower calls with shorter rows stay on the GEMM (1.5B o 1536 x
// 1536 at 17 rows 8.8 against 10.0, 2048 x 1536 8.4 against 9.4 us), and so
// do 33..64 rows (ranges of 2 groups: their partial sums cost more than the
// tiles save, 7B gate at 48 rows 50.0 -> 51.3 us).
bool gemvq_rows_preferred(int64_t M, int tiles, int64_t K, int n) {
    return M >= 17 && M <= 32 && K % kGroup == 0 && (tiles >= 224 || K / kGroup >= 128 || n > 1);
}

// gemvq on n matrices, M in 7..32, straight from x (false: M out of range;
// partial sums beyond the workspace are avoided by looping over K ranges,
// gemvq_plan in iq_plan.h).
bool launch_gemvq(const float* x, const QView* W, const uint16_t* const* bias, float* const* y, int n, int M,
                  Workspace* ws, hipStream_t stream, hipError_t* err) {
    const int64_t K = W[0].cols, G = W[0].groups;
    GemvParams p{};
    int tiles = 0, t32 = 0;
    for (int i = 0; i < n; i++) {
        p.mat[i] = MatRef{W[i].q, W[i].scales, W[i].zeros, bias[i], y[i], W[i].rows, tiles};
        tiles += int((W[i].rows + 15) / 16);
        t32 += int((W[i].rows + 31) / 32);
    }
    const GqPlan pl = gemvq_plan(G, M, tiles, t32, W[0].kind, device_cu_count(), ws->part_floats);
    if (!pl.ok) return false;
    const int S = pl.S, L = pl.L, gs = pl.gs, nrb = pl.nrb, mb = pl.mb;
    p.nmat = n;
    p.K = K;
    p.G = G;
    p.x = x;
    p.M = M;
    p.gs = gs;
    p.S = S;
    p.kr = L;
    p.nrb = nrb;
    p.ntiles = tiles;
    p.part = ws->partials;
    const unsigned grid = unsigned(nrb * S);
    if (mb == 1) {
        if (W[0].kind == 1) {
            if (L > 1) gemvq_kernel<1, 6, 1, true><<<grid, 512, 0, stream>>>(p);
            else gemvq_kernel<1, 6, 1, false><<<grid, 512, 0, stream>>>(p);
        } else {
            if (L > 1) gemvq_kernel<0, 4, 1, true><<<grid, 512, 0, stream>>>(p);
            else gemvq_kernel<0, 4, 1, false><<<grid, 512, 0, stream>>>(p);
        }
    } else {
        if (W[0].kind == 1) {
            if (L > 1) gemvq_kernel<1, 4, 2, true><<<grid, 512, 0, stream>>>(p);
            else gemvq_kernel<1, 4, 2, false><<<grid, 512, 0, stream>>>(p);
        } else {
            if (L > 1) gemvq_kernel<0, 2, 2, true><<<grid, 512, 0, stream>>>(p);
            else gemvq_kernel<0, 4, 2, false><<<grid, 512, 0, stream>>>(p);
        }
    }
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && S > 1) {
        const int64_t outs = int64_t(M) * tiles * 16;
        gemvt_reduce_kernel<<<unsigned((outs + 255) / 256), 256, 0, stream>>>(p);
        e = hipGetLastError();
    }
    *err = e;
    return true;
}

// gemvs on n matrices, M in 9..16, on the prepared split operands (false:
// the split-K partials would not fit).
bool launch_gemvs(const QView* W, const uint16_t* const* bias, float* const* y, int n, int M, Workspace* ws,
                  hipStream_t stream, hipError_t* err) {
    const int64_t K = W[0].cols, G = W[0].groups;
    GemvParams p{};
    int tiles = 0;
    for (int i = 0; i < n; i++) {
        p.mat[i] = MatRef{W[i].q, W[i].scales, W[i].zeros, bias[i], y[i], W[i].rows, tiles};
        tiles += int((W[i].rows + 15) / 16);
    }
    const int nrb = (tiles + 7) / 8;
    // K ranges: enough workgroups for two per CU, at least 4 groups each
    const int want = 2 * device_cu_count();
    int S = (want + nrb - 1) / nrb;
    S = std::max(1, std::min<int>(S, int(G / 4)));
    int gs = int((G + S - 1) / S);
    S = int((G + gs - 1) / gs);
    if (S > 1 && int64_t(S) * M * tiles * 16 > kPartialFloats) return false;
    p.nmat = n;
    p.K = K;
    p.G = G;
    p.xq = ws->xq;
    p.meta = ws->xmeta;
    p.M = M;
    p.gs = gs;
    p.S = S;
    p.ntiles = tiles;
    p.part = ws->partials;
    const unsigned grid = unsigned(nrb * S);
    if (W[0].kind == 1) gemvs_kernel<1><<<grid, 512, 0, stream>>>(p);
    else gemvs_kernel<0><<<grid, 512, 0, stream>>>(p);
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && S > 1) {
        const int64_t outs = int64_t(M) * tiles * 16;
        gemvt_reduce_kernel<<<unsigned((outs + 255) / 256), 256, 0, stream>>>(p);
        e = hipGetLastError();
    }
    *err = e;
    return true;
}

// f16 split preparation of x [M][K] (M <= kMaxRowsGemv, K % 128 == 0).
// pk: the packed form up to 8 rows (false: 16-row blocks at any M, the form
// gemvs reads).
hipError_t launch_xhprep(const float* x, int M, int64_t K, int kind, Workspace* ws, hipStream_t stream,
                         bool pk = true) {
    const int64_t G = K / kGroup, quads = (G + 3) / 4;
    const int nb = (M + 15) / 16;
    const int64_t waves = int64_t(nb) * 16 * quads;
    const unsigned grid = unsigned((waves + 3) / 4);
    _Float16* xh = reinterpret_cast<_Float16*>(ws->xq);
    float* xfx = reinterpret_cast<float*>(ws->xmeta);
    if (M <= 8 && pk) {
        if (kind == 1) xhprep_kernel<true, true><<<grid, 256, 0, stream>>>(x, M, K, G, quads, nb, xh, xfx);
        else xhprep_kernel<false, true><<<grid, 256, 0, stream>>>(x, M, K, G, quads, nb, xh, xfx);
    } else {
        if (kind == 1) xhprep_kernel<true, false><<<grid, 256, 0, stream>>>(x, M, K, G, quads, nb, xh, xfx);
        else xhprep_kernel<false, false><<<grid, 256, 0, stream>>>(x, M, K, G, quads, nb, xh, xfx);
    }
    return hipGetLastError();
}

bool gemvh_applies(int64_t K, int M) {
    return M >= 2 && M <= kMaxRowsGemv && K % kGroup == 0;
}

// Direct calls (x given with the matrices) pick per shape, from 7B and
// 1.5B measurements at 2..16 rows: gemvh for narrow calls (< 512 tiles: 7B
// q|k|v 13.7 against 16 us, o 10.8 against 16); gemvt, whose workgroups share
// one LDS copy of the activations over many tiles and pack 4 rows x 4 limbs
// per MFMA up to 8 rows, for wider calls up to 8 rows and for 1024..4095-tile
// calls with short K (7B gate|up: 27..38 against 47..48 us); gemvh otherwise
// (lm_head at 12..16 rows: 173 against 184 us).
bool gemvh_preferred(int64_t K, int M, int tiles, int kind) {
    if (!gemvh_applies(K, M)) return false;
    // int8 with long K: gemvt (7B down int8, K = 18944, at 16 / 8 rows:
    // 38.3 -> 32.6 / 30.5 -> 29.3 us; not at K = 8960: 1.5B down 17 -> 24
    // us; int4 stays on gemvh: 33.5 against 36.7 / 27.0 against 32.3)
    if (kind == 0 && K / kGroup > 128) return false;
    if (tiles < 512) return true;
    if (M <= 8) return false;
    return !(tiles >= 1024 && tiles < 4096 && K / kGroup <= 64);
}

template <int KIND, int T>
void launch_gemvh_t(const GemvParams& p, int ks, hipStream_t stream) {
    const unsigned grid = unsigned((p.ntiles + T - 1) / T);
    const size_t lds = size_t(T) * ks * 4 * 64 * 4;
    // (T = 2, 9..16 rows: two groups in flight per wave, 183 / 199 VGPRs on
    // 8-wave workgroups; 7B q|k|v at 16 rows 13.8 -> 13.2 us with its
    // preparation.  The 16-wave T = 1 instance would spill at 128.)
    if (p.M <= 8 && p.S == 0) gemvh_kernel<KIND, T, true><<<grid, 64 * ks, lds, stream>>>(p);
    else if constexpr (T == 2) gemvh_kernel<KIND, T, false, true><<<grid, 64 * ks, lds, stream>>>(p);
    else gemvh_kernel<KIND, T, false><<<grid, 64 * ks, lds, stream>>>(p);
}

// The n matrices (one kind and width) on the prepared f16 split activations.
// gemvh over the prepared operands at xq / xmeta (16-row blocks), with the
// chain epilogue's residual and per-tile sums of squares (res: one matrix,
// [M][N]; ssq_out: [M][tiles]) when given.
hipError_t launch_gemvh_on(const QView* W, const uint16_t* const* bias, float* const* y, int n, int M,
                           const int8_t* xq, const float* xmeta, const float* res, float* ssq_out,
                           hipStream_t stream, bool packed = true) {
    const int64_t K = W[0].cols, G = W[0].groups;
    const int tiles = total_tiles(W, n);
    // tiles per workgroup (measured, 7B shapes at 16 rows): the prepared
    // operands of a group are read from L2 once per workgroup and group, so
    // wide calls share them over more tiles (lm_head: 174 us at 4 against
    // 280 at 1); narrow ones keep enough workgroups to fill the GPU (o: 10.8
    // us at 1 against 13.8 at 2; q|k|v: 13.8 at 2 against 16.2 at 1)
    const int T = tiles >= 4096 ? 4 : ((tiles >= 256 && G <= 64) ? 2 : 1);
    const int maxw = T == 1 ? 16 : 8;  // the kernel's launch bound
    int gs = int((G + maxw - 1) / maxw);
    const int ks = int((G + gs - 1) / gs);
    for (int r0 = 0; r0 < M; r0 += 16) {
        GemvParams p{};
        int t0 = 0;
        for (int i = 0; i < n; i++) {
            p.mat[i] = MatRef{W[i].q, W[i].scales, W[i].zeros, bias[i], y[i] + int64_t(r0) * W[i].rows, W[i].rows, t0};
            t0 += int((W[i].rows + 15) / 16);
        }
        p.nmat = n;
        p.K = K;
        p.G = G;
        p.xq = xq + int64_t(r0 / 16) * G * kHGroupBytes;
        p.meta = reinterpret_cast<const int4*>(xmeta + int64_t(r0 / 16) * G * 16);
        p.res = res ? res + int64_t(r0) * W[0].rows : nullptr;
        p.ssq_out = ssq_out ? ssq_out + int64_t(r0) * tiles : nullptr;
        p.M = M - r0 < 16 ? M - r0 : 16;
        p.gs = gs;
        p.S = M <= 8 && packed ? 0 : 1;  // 0: the packed (M <= 8) preparation
        p.ntiles = tiles;
        if (W[0].kind == 1) {
            if (T == 4) launch_gemvh_t<1, 4>(p, ks, stream);
            else if (T == 2) launch_gemvh_t<1, 2>(p, ks, stream);
            else launch_gemvh_t<1, 1>(p, ks, stream);
        } else {
            if (T == 4) launch_gemvh_t<0, 4>(p, ks, stream);
            else if (T == 2) launch_gemvh_t<0, 2>(p, ks, stream);
            else launch_gemvh_t<0, 1>(p, ks, stream);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t launch_gemvh(const QView* W, const uint16_t* const* bias, float* const* y, int n, int M, Workspace* ws,
                        hipStream_t stream) {
    return launch_gemvh_on(W, bias, y, n, M, ws->xq, reinterpret_cast<const float*>(ws->xmeta), nullptr, nullptr,
                           stream);
}

hipError_t launch_batched_multi(const QView* W, const uint16_t* const* bias, float* const* y, int n, int M,
                                Workspace* ws, hipStream_t stream) {
    hipError_t e = hipSuccess;
    if (launch_gemvt(W, bias, y, n, M, ws, stream, &e)) return e;
    for (int i = 0; i < n; i++) {
        const hipError_t e = launch_gemv_batched(W[i], bias[i], M, y[i], ws, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

// A preparation of 1..4 rows that the 1-row kernel will consume is a copy
// of x (the kernel converts it itself); anything else is converted (f16
// split or limbs).
hipError_t launch_xprep(const float* x, int M, int64_t K, int kind, Workspace* ws, hipStream_t stream) {
    const int64_t G = (K + kGroup - 1) / kGroup;
    hipError_t e;
    if (M <= 4 && gemv1_plan(G, kind, gemv1_mode(K, G, ws->xf), 1, device_cu_count(), gemv1_rows(M)).ng > 0) {
        e = hipMemcpyAsync(ws->xf, x, sizeof(float) * size_t(M) * size_t(K), hipMemcpyDeviceToDevice, stream);
        ws->prep_copy = true;
        ws->prep_h = false;
    } else if (gemvh_applies(K, M)) {
        e = launch_xhprep(x, M, K, kind, ws, stream);
        ws->prep_copy = false;
        ws->prep_h = true;
    } else {
        e = launch_xprep_limbs(x, M, K, kind, ws, stream);
        ws->prep_copy = false;
        ws->prep_h = false;
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
        const G1Plan pl = gemv1_plan(G, W[0].kind, mode, total_tiles(W, n), device_cu_count(), gemv1_rows(M));
        if (pl.ng > 0) return launch_gemv1(ws->xf, W, bias, y, n, pl, mode, stream, M, ws->partials);
        // (too many tiles for the split-K partials of this width): the
        // general path on the copy, the preparation left as it was
        const int keep_M = ws->prep_M, keep_kind = ws->prep_kind;
        const int64_t keep_K = ws->prep_K;
        const hipError_t e = launch_gemv_multi(ws->xf, W, bias, y, n, M, ws, stream);
        ws->prep_M = keep_M;
        ws->prep_K = keep_K;
        ws->prep_kind = keep_kind;
        ws->prep_copy = true;
        ws->prep_h = false;
        return e;
    }
    if (ws->prep_h) return launch_gemvh(W, bias, y, n, M, ws, stream);
    return launch_batched_multi(W, bias, y, n, M, ws, stream);
}

hipError_t launch_gemv_prepped(const QView& W, const uint16_t* bias, int M, float* y, Workspace* ws,
                               hipStream_t stream) {
    return launch_gemv_prepped_multi(&W, &bias, &y, 1, M, ws, stream);
}

hipError_t launch_gemv_multi(const float* x, const QView* W, const uint16_t* const* bias, float* const* y,
                             int n, int M, Workspace* ws, hipStream_t stream) {
    const int64_t K = W[0].cols, G = W[0].groups;
    if (gemvq_rows_preferred(M, total_tiles(W, n), K, n)) {
        hipError_t e = hipSuccess;
        if (launch_gemvq(x, W, bias, y, n, M, ws, stream, &e)) return e;
    }
    if (M > 16) {
        // 17..32 rows: the prefill GEMM's 64-row tiles beat two 16-row GEMV
        // blocks (1.5B gate 8960 x 1536 at 32 rows: 23.0 -> 16.2 us int8;
        // 7B down 3584 x 18944 at 24 / 32 rows: 50.1 / 54.0 -> 37.4 / 38.4
        // us int8, gate 18944 x 3584 int4: 47.5 / 53.0 -> 44.7 / 46.7)
        for (int i = 0; i < n; i++) {
            const hipError_t e = launch_gemm(x, nullptr, W[i], bias[i], M, y[i], ws, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // 5..8 rows on wide or long-K calls: gemvr on the packed hi/lo operands
    // (7B int4 at 5 / 8 rows: gate|up 34.5 -> 28.7 / 35.1 -> 29.2, down
    // 27.6 -> 24.0 / 27.4 -> 25.0 us against gemvt / gemvh; lm_head 152064 x
    // 3584 int8: 166 -> 121 / 166 -> 155 us; at 2..4 rows the 1-row
    // kernel's 4-row instance is far faster; not at G = 70: 1.5B down
    // 1536 x 8960 at 5 / 8 rows 13.2 / 13.1 us elsewhere against 18.5 /
    // 20.2 on gemvr, and 15.4 against 21.3 at 16 rows)
    // 7..8 rows on very wide calls (the lm_head): gemvs on the 16-row
    // operand blocks (7B lm_head int8 at 7 / 8 rows: 163 -> 135 / 163 -> 138
    // us; at 5 / 6 rows gemvr stays ahead, 121 / 124 against 137 / 138)
    // ... and before them, for int4, gemvq straight from x, rows past 8 of
    // its 16-row block reading zero (7 / 8 rows: lm_head int4 109 / 109 ->
    // 90 / 91 us; at 5 / 6 rows gemvr stays ahead; int8, whose launch alone
    // measured 141 -> 136 us, made the 7B step at 8 rows 2094 -> 2117 us)
    if (W[0].kind == 1 && M >= 7 && M <= 8 && K % kGroup == 0 && total_tiles(W, n) >= 4096) {
        hipError_t e = hipSuccess;
        if (launch_gemvq(x, W, bias, y, n, M, ws, stream, &e)) return e;
    }
    if (M >= 7 && M <= 8 && K % kGroup == 0 && total_tiles(W, n) >= 4096) {
        if (!ws->prep_copy) ws->invalidate_prep();
        hipError_t e = launch_xhprep(x, M, K, W[0].kind, ws, stream, false);
        if (e != hipSuccess) return e;
        if (launch_gemvs(W, bias, y, n, M, ws, stream, &e)) return e;
    }
    // (and from 3 rows on long rows, G >= 128, which the 1-row kernel's
    // 4-row instance splits over K ranges: 7B down 3584 x 18944 int8 at 3 /
    // 4 rows 27.3 / 30.6 -> 24.1 / 24.2 us, int4 at 3 / 4 rows 22.5 / 22.1
    // -> 19.9 / 20.8 (int4 step at 3 rows 1807 -> 1761 us); at 2 rows the
    // 2-row instance stays ahead, int4 17.8 against 19.4)
    // ... and, since the cheaper int4 dequantisation and activation split,
    // from 4 rows on wide int4 calls and very wide calls of either kind
    // (7B at 4 rows: int4 gate|up 32.5 -> 27.3, lm_head int4 137 -> 118,
    // int8 138 -> 127 us; int4 step 1922 -> 1825 us; the 4-row instance's
    // limb records of 4 rows hold a CU to two workgroups); at 3 rows the
    // step measured the same either way, at 2 the 4-row instance is far
    // ahead
    const int tiles_all = total_tiles(W, n);
    int m_lo = G >= 128 ? 3 : 5;
    if (tiles_all >= 4096 || (W[0].kind == 1 && tiles_all >= 1024)) m_lo = m_lo < 4 ? m_lo : 4;
    // ... except wide int4 calls whose rows the 1-row kernel's 4-row
    // instance takes two tiles per workgroup (6..8 waves of 4 groups: 7B
    // gate|up at 4 rows 27.5 -> 22.8 us)
    if (W[0].kind == 1 && tiles_all < 4096 && G >= 21 && G <= 32 && G % 4 == 0) m_lo = 5;
    if (M >= m_lo && M <= 8 && K % kGroup == 0 && (total_tiles(W, n) >= 1024 || G >= 128)) {
        hipError_t e = hipSuccess;
        if (launch_gemvr(x, W, bias, y, n, M, ws, stream, &e)) return e;
        if (!ws->prep_copy) ws->invalidate_prep();
        e = launch_xhprep(x, M, K, W[0].kind, ws, stream);
        if (e != hipSuccess) return e;
        return launch_gemvh(W, bias, y, n, M, ws, stream);
    }
    if (gemv1_rows_preferred(M, total_tiles(W, n), G)) {
        // the 1-row kernel converts x itself; 2..8 rows share each weight
        // operand (no preparation launch, and the workspace's preparation
        // stays as it was)
        const int mode = gemv1_mode(K, G, x);
        const G1Plan pl = gemv1_plan(G, W[0].kind, mode, total_tiles(W, n), device_cu_count(), gemv1_rows(M));
        if (pl.ng > 0) return launch_gemv1(x, W, bias, y, n, pl, mode, stream, M, ws->partials);
    }
    // The conversion below overwrites xq / xmeta: a preparation held there
    // (not a copy in xf) is gone, so iq_gemv_prepped must refuse to run on it.
    if (!ws->prep_copy) ws->invalidate_prep();
    // 9..16 rows on very wide calls (the lm_head): gemvs, whose workgroups
    // share each group's operands over 8 tiles through LDS (7B lm_head
    // 152064 x 3584 int8 at 16 rows: 176 -> 139 us; on the layer shapes it
    // measured no better than gemvh / gemvt: gate|up 41.7 -> 42.8, down
    // 33.6 -> 34.5 us at its best K split)
    // ... except int4, on gemvq straight from x (7B lm_head int4 at 9 / 12 /
    // 16 rows 109 / 109 / 110 -> 93 / 99 / 104 us; int8 at 9 / 16 rows 153 /
    // 143 against 142 / 160 for the launch alone, and no faster in the 7B
    // step at 9 / 10 rows)
    if (W[0].kind == 1 && M > 8 && M <= 16 && K % kGroup == 0 && total_tiles(W, n) >= 4096) {
        hipError_t e = hipSuccess;
        if (launch_gemvq(x, W, bias, y, n, M, ws, stream, &e)) return e;
    }
    if (M > 8 && M <= 16 && K % kGroup == 0 && total_tiles(W, n) >= 4096) {
        hipError_t e = launch_xhprep(x, M, K, W[0].kind, ws, stream);
        if (e != hipSuccess) return e;
        if (launch_gemvs(W, bias, y, n, M, ws, stream, &e)) return e;
        return launch_gemvh(W, bias, y, n, M, ws, stream);
    }
    // 9..16 rows on wide or long-K layer calls (7B gate|up 2368 tiles, down
    // G = 148): gemvr, every request of a K range made at once (int4 at 16
    // rows: gate|up 41.5 -> 38.3, down 34.3 -> 28.6 us; narrow short-K
    // calls such as q|k|v and o lose: 13.7 -> 18.9, 10.7 -> 18.4 us; the
    // lm_head stays on gemvs above: 138 against 180 us), and on wide calls
    // gemvq, half the operand reads per weight (int4 gate|up at 12 / 16
    // rows: 36.0 -> 31.2 / 38.3 -> 33.7 us; int8 stays on gemvr: 40.2
    // against 39.9 at 9 rows, 44.1 against 45.3 at 16;
    // down loses with its shorter K ranges: 28.8 -> 34.2)
    if (M > 8 && M <= 16 && K % kGroup == 0 && (total_tiles(W, n) >= 1024 || G >= 128)) {
        hipError_t e = hipSuccess;
        if (W[0].kind == 1 && total_tiles(W, n) >= 1024 && launch_gemvq(x, W, bias, y, n, M, ws, stream, &e))
            return e;
        if (launch_gemvr(x, W, bias, y, n, M, ws, stream, &e)) return e;
        e = launch_xhprep(x, M, K, W[0].kind, ws, stream);
        if (e != hipSuccess) return e;
        return launch_gemvh(W, bias, y, n, M, ws, stream);
    }
    if (gemvh_preferred(K, M, total_tiles(W, n), W[0].kind)) {
        const hipError_t e = launch_xhprep(x, M, K, W[0].kind, ws, stream);
        if (e != hipSuccess) return e;
        return launch_gemvh(W, bias, y, n, M, ws, stream);
    }
    hipError_t e = launch_xprep_limbs(x, M, K, W[0].kind, ws, stream);
    if (e != hipSuccess) return e;
    return launch_batched_multi(W, bias, y, n, M, ws, stream);
}

bool launch_gemm_rows(const float* x, const QView& W, const uint16_t* bias, int64_t T, float* y, Workspace* ws,
                      hipStream_t stream, hipError_t* err) {
    if (!gemvq_rows_preferred(T, int((W.rows + 15) / 16), W.cols, 1)) return false;
    return launch_gemvq(x, &W, &bias, &y, 1, int(T), ws, stream, err);
}

hipError_t launch_gemv(const float* x, const QView& W, const uint16_t* bias, int M, float* y,
                       Workspace* ws, hipStream_t stream) {
    return launch_gemv_multi(x, &W, &bias, &y, 1, M, ws, stream);
}

// ------------------------------------------------------------------ B-row chain stages
namespace {

// The kernel and K ranges of a B-row chain stage (the rows GEMV of
// launch_gemv_multi: gemvr, or gemvq from 17 rows and for wide int4 calls
// from 9), every range's sums written to part [S][M][tiles * 16].
struct RowsSetup {
    GemvParams p{};
    bool q = false;  // gemvq (else gemvr)
    int S = 0;
    unsigned grid = 0;
    bool ok = false;
};

RowsSetup rows_setup(const QView* W, int n, int M, int64_t part_floats) {
    RowsSetup r;
    const int64_t K = W[0].cols, G = W[0].groups;
    int tiles = 0, t32 = 0;
    for (int i = 0; i < n; i++) {
        r.p.mat[i] = MatRef{W[i].q, W[i].scales, W[i].zeros, nullptr, nullptr, W[i].rows, tiles};
        tiles += int((W[i].rows + 15) / 16);
        t32 += int((W[i].rows + 31) / 32);
    }
    if (M < 1 || M > kMaxRowsGemv || K % kGroup) return r;
    r.p.nmat = n;
    r.p.K = K;
    r.p.G = G;
    r.p.M = M;
    r.p.ntiles = tiles;
    r.p.to_part = 1;
    const int cus = device_cu_count();
    const bool use_q = M >= 17 || (M >= 9 && W[0].kind == 1 && tiles >= 1024);
    if (!use_q) {
        // launch_gemvr's ranges
        const int nrb = (tiles + 7) / 8;
        constexpr int ngr = 8;
        int S = int((G + ngr - 1) / ngr);
        S = std::max<int>(S, std::min<int>((2 * cus + nrb - 1) / nrb, int(G)));
        const int gs = int((G + S - 1) / S);
        S = int((G + gs - 1) / gs);
        if (int64_t(S) * M * tiles * 16 <= part_floats) {
            r.p.gs = gs;
            r.p.S = S;
            r.S = S;
            r.grid = unsigned(nrb * S);
            r.ok = true;
            return r;
        }
        if (M < 7) return r;
    }
    const GqPlan pl = gemvq_plan(G, M, tiles, t32, W[0].kind, cus, part_floats);
    if (!pl.ok) return r;
    r.q = true;
    r.p.gs = pl.gs;
    r.p.S = pl.S;
    r.p.kr = pl.L;
    r.p.nrb = pl.nrb;
    r.S = pl.S;
    r.grid = unsigned(pl.nrb * pl.S);
    r.ok = true;
    return r;
}

}  // namespace

int64_t chain_rows_partials(const QView* W, int n, int M, int64_t cap) {
    const RowsSetup r = rows_setup(W, n, M, cap);
    return r.ok ? int64_t(r.S) * M * r.p.ntiles * 16 : -1;
}

hipError_t launch_chain_rows(const QView* W, int n, int M, const RowsIn& in, float* part, int64_t part_floats,
                             int* S, hipStream_t stream) {
    // 2 rows of a plain input (no RMSNorm, no gather: the down stage) on
    // long rows: the 1-row kernel's K-split 2-row instance, its range sums
    // into `part` for the epilogue (7B int4 decode chain at 2 sequences
    // 1629 -> 1529 us; at 3 / 4 the 4-row instance lost to gemvr, 1900 /
    // 2031 -> 1908 / 2105 us)
    if (M == 2 && !in.norm && in.gqa_hd == 0 && in.xstride == W[0].cols) {
        const int64_t K = W[0].cols, G = W[0].groups;
        const int tiles = total_tiles(W, n);
        const int mode = gemv1_mode(K, G, in.x);
        const G1Plan pl = gemv1_plan(G, W[0].kind, mode, tiles, device_cu_count(), gemv1_rows(M));
        if (pl.ng > 0 && pl.kr > 1 && int64_t(pl.kr) * M * tiles * 16 <= part_floats) {
            const uint16_t* nb[kMaxMulti] = {};
            float* ny[kMaxMulti] = {};
            *S = pl.kr;
            return launch_gemv1(in.x, W, nb, ny, n, pl, mode, stream, M, part, false);
        }
    }
    RowsSetup r = rows_setup(W, n, M, part_floats);
    if (!r.ok) return hipErrorInvalidValue;
    GemvParams& p = r.p;
    p.x = in.x;
    p.xstride = in.xstride;
    p.gqa_hd = in.gqa_hd;
    p.gqa_span = in.gqa_span;
    p.norm = in.norm;
    p.ssq = in.ssq;
    p.ssq_n = in.ssq_n;
    p.eps = in.eps;
    p.part = part;
    *S = r.S;
    const int kind = W[0].kind;
    if (!r.q) {
        if (M <= 8) {
            if (kind == 1) gemvr_kernel<1, true, 8, true><<<r.grid, 512, 0, stream>>>(p);
            else gemvr_kernel<0, true, 8, true><<<r.grid, 512, 0, stream>>>(p);
        } else {
            if (kind == 1) gemvr_kernel<1, false, 8, true><<<r.grid, 512, 0, stream>>>(p);
            else gemvr_kernel<0, false, 8, true><<<r.grid, 512, 0, stream>>>(p);
        }
    } else if (M <= 16) {
        if (kind == 1) {
            if (p.kr > 1) gemvq_kernel<1, 6, 1, true, true><<<r.grid, 512, 0, stream>>>(p);
            else gemvq_kernel<1, 6, 1, false, true><<<r.grid, 512, 0, stream>>>(p);
        } else {
            if (p.kr > 1) gemvq_kernel<0, 4, 1, true, true><<<r.grid, 512, 0, stream>>>(p);
            else gemvq_kernel<0, 4, 1, false, true><<<r.grid, 512, 0, stream>>>(p);
        }
    } else {
        if (kind == 1) {
            if (p.kr > 1) gemvq_kernel<1, 4, 2, true, true><<<r.grid, 512, 0, stream>>>(p);
            else gemvq_kernel<1, 4, 2, false, true><<<r.grid, 512, 0, stream>>>(p);
        } else {
            if (p.kr > 1) gemvq_kernel<0, 2, 2, true, true><<<r.grid, 512, 0, stream>>>(p);
            else gemvq_kernel<0, 4, 2, false, true><<<r.grid, 512, 0, stream>>>(p);
        }
    }
    return hipGetLastError();
}

void chain_h_bytes(int64_t G, int M, size_t* xq_bytes, size_t* meta_floats) {
    const int64_t nb = (M + 15) / 16;
    *xq_bytes = size_t(nb * G * kHGroupBytes);
    *meta_floats = size_t(nb * G * 16);
}

bool chain_h_applies(const QView* W, int n, int M) {
    return M >= 5 && M <= 16 && W[0].cols % kGroup == 0 && total_tiles(W, n) < 1024 && W[0].groups < 128;
}

hipError_t launch_chain_h(const QView* W, int n, int M, const RowsIn& in, const uint16_t* const* bias,
                          float* const* y, const float* res, float* ssq_out, int8_t* xq, float* xmeta,
                          hipStream_t stream) {
    if (!chain_h_applies(W, n, M)) return hipErrorInvalidValue;
    const int64_t K = W[0].cols, G = W[0].groups, quads = (G + 3) / 4;
    const int nb = (M + 15) / 16;
    GemvParams pp{};
    pp.x = in.x;
    pp.xstride = in.xstride;
    pp.gqa_hd = in.gqa_hd;
    pp.gqa_span = in.gqa_span;
    pp.norm = in.norm;
    pp.ssq = in.ssq;
    pp.ssq_n = in.ssq_n;
    pp.eps = in.eps;
    pp.M = M;
    pp.K = K;
    pp.G = G;
    const unsigned grid = unsigned((int64_t(nb) * 16 * quads + 3) / 4);
    _Float16* xh = reinterpret_cast<_Float16*>(xq);
    if (W[0].kind == 1) xhprep_pro_kernel<true><<<grid, 256, 0, stream>>>(pp, quads, nb, xh, xmeta);
    else xhprep_pro_kernel<false><<<grid, 256, 0, stream>>>(pp, quads, nb, xh, xmeta);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // (the unpacked operand form at 5..8 rows too: rows 8..15 of each block
    // are zero)
    return launch_gemvh_on(W, bias, y, n, M, xq, xmeta, res, ssq_out, stream, false);
}

}  // namespace iq

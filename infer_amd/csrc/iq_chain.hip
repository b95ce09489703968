// iq_chain.hip -- a chain of dependent 1-row quantised GEMV stages: the
// quantised part of the reference's decode step
// (GpuBatch::Impl::launch_sequence, kernels/batch_gpu.cu:186-215) as a
// program, each stage one linear call site (q|k|v, o, gate|up, down, the
// LM head) whose input is the output of an earlier stage, with the
// elementwise work around it fused in:
//   prologue  RMSNorm of the input (launch_rmsnorm, src/forward.cpp:21-31),
//             or the single-key attention output (value row of each query
//             head's key/value head);
//   epilogue  bias, residual add (launch_residual_add), or SwiGLU of a
//             gate / up tile pair (launch_swiglu, kernels/ops/elementwise.cu:6-11).
// One launch per stage, stream-ordered (the caller captures a run in a HIP
// graph); the reference needs 3-5 launches per stage for the same work.
//
// The stage kernel is the 1-row GEMV's arithmetic (iq_limbs.h): a workgroup
// owns one 16-row output tile (or a gate tile with the up tile of the same
// rows); its waves split K into slices of whole 128-column groups, each
// wave requests its activations first, then its scales, zero points and
// weights (16-byte loads), converts its activation slice into byte limbs
// in LDS while the weights stream in, and multiplies codes by limbs on
// v_mfma_i32_16x16x64_i8 (exact int32 sums); combine() applies scale, zero
// point and the activation exponent in fp32.  The slice sums are added in
// wave order through LDS by the wave that finishes last (deterministic).
//
// RMSNorm needs the sum of squares of the whole input vector.  When the
// input is the output of an earlier stage of the same chain (the residual
// stream after o and down), that stage writes one partial sum of squares
// per 16-row output tile as it stores the tile, and the consumer adds the
// producer's partials in tile order (in double) before its slices' scale is
// known: no extra pass over the vector.  Otherwise (the chain's first
// input) every thread of the workgroup loads a part of the vector (16-byte
// loads, issued before the weights), the sum of squares is reduced in
// double through LDS in a fixed order, and the raw vector stays in LDS for
// the waves' slices.
//
// A persistent variant (one cooperative launch for the whole program, grid
// barriers between stages, next-stage weights requested before each
// barrier) was built and measured slower: 2.75 ms against 1.16 ms for the
// 7B step, because the barrier's atomics, the write-through stores and the
// next input's loads wait in the same memory queues as the megabytes of
// weights in flight (2-4 us each), and the stage's loop of dependent
// slices kept too few bytes in flight per CU.
#include <algorithm>
#include <cstring>
#include <vector>

#include "../../include/iq.h"
#include "iq_limbs.h"

namespace iq {

namespace {

constexpr int kMaxStageMats = 3;
constexpr int kMaxWaves = 16;

struct CMat {
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
    const uint16_t* bias;
    float* y;
    int32_t N;
    int32_t tile0;  // first tile of this matrix in the stage's tile numbering
};

// One stage as the kernel sees it (a kernel argument: read through the
// scalar cache).
struct CStage {
    CMat mat[kMaxStageMats];
    const float* x;
    const uint16_t* norm;
    const float* res;
    float eps;
    int32_t in_op, out_op, nmat;
    int32_t K, G;
    int32_t units;    // workgroups: tiles, or gate / up tile pairs
    int32_t tpu;      // tiles per unit (2: SwiGLU pair)
    int32_t ks;       // waves per tile
    int32_t gs;       // groups per wave slice (even; the last slice may be shorter)
    int32_t gqa_hd, gqa_span;  // IQ_IN_GQA: head_dim, head_dim * group
    // RMSNorm input: per-16-row-tile sums of squares of x written by the
    // stage that produced x (ssq_n of them), or null (then the kernel sums
    // the whole input itself)
    const float* ssq_in;
    int32_t ssq_n;
    // per-tile sums of squares of this stage's output (for a later RMSNorm), or null
    float* ssq_out;
    // activation rows (R-row instances: 1..R; row m of x at m * xlen, of
    // residual and y at m * N); per-row sums of squares: ssq_in [rows][ssq_n]
    // and ssq_out [rows][tiles]
    int32_t rows;
};

// Output side of a B-row stage (epi_kernel): the K-range sums of the rows
// GEMV, bias, then store / residual add / SwiGLU, and (when a later
// RMSNorm stage reads the output) the sums of squares of each row's
// 256-column blocks.
struct CEpi {
    float* y[kMaxStageMats];
    const uint16_t* bias[kMaxStageMats];
    int32_t N[kMaxStageMats];
    int32_t tile0[kMaxStageMats];
    int32_t nmat;
    const float* part;
    int32_t S, M;
    int64_t ld;        // partial-sum row length: 16 x tiles of all matrices
    int32_t swiglu;
    const float* res;
    float* ssq_out;    // [M][ssq_n] or null
    int32_t ssq_n;
    int32_t ncols;     // columns of the grid: N_0 (SwiGLU) or ld
};

// Host record of a stage: the kernel argument and its launch shape.
struct HostStage {
    CStage st;
    int kind;
    int ng;  // slice capacity of the kernel instance
    size_t lds;
    // B-row stages (rows > 1)
    int rows = 1;
    int fused_r = 1;  // > 1: one stage_kernel launch of the R-row instance (rows <= R)
    bool hroute = false;  // B rows on a narrow stage: operand preparation + gemvh (no epilogue launch)
    QView W[kMaxStageMats];
    RowsIn in{};
    CEpi epi{};
    // RMSNorm input no earlier stage of the chain produces: its sums of
    // squares come from ssq_kernel before the GEMV
    bool own_ssq = false;
    float* ssq = nullptr;  // [rows][ssq_n] (own or the producer's)
};

__device__ __forceinline__ CMat stage_mat(const CStage& st, int m) {
    return m == 0 ? st.mat[0] : (m == 1 ? st.mat[1] : st.mat[2]);
}

// Columns [k0, k0 + 8) of the stage input (IQ_IN_GQA: the value row of the
// query head's key/value head).
__device__ __forceinline__ void load_input8(const CStage& st, int k0, float (&v)[8]) {
    const float* src = st.x + k0;
    if (st.in_op == IQ_IN_GQA) src = st.x + (k0 / st.gqa_span) * st.gqa_hd + (k0 % st.gqa_hd);
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 c = *reinterpret_cast<const float4*>(src + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
}

__device__ __forceinline__ double wave_sum(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// Sum over the 16 lanes of a DPP row (every lane of the row active).
__device__ __forceinline__ float row16_fsum(float v) {
    v += __int_as_float(row_ror<8>(__float_as_int(v)));
    v += __int_as_float(row_ror<4>(__float_as_int(v)));
    v += __int_as_float(row_ror<2>(__float_as_int(v)));
    v += __int_as_float(row_ror<1>(__float_as_int(v)));
    return v;
}

// Workgroup = ks waves on one unit: TP = 1 one 16-row tile, TP = 2 the gate
// and up tiles of the same rows (each wave holds both tiles' weights of its
// slice and multiplies both by the same activation operand).  Wave w owns
// the K slice [w gs, w gs + gs).  NG = slice capacity in groups (a multiple
// of 4).  Dynamic LDS: limb records [G][512] | meta [G] int4 | (RMSNorm
// without producer partials) the raw input [K] fp32.
// R = 2 or 4: up to R activation rows per launch (st.rows), the limb records
// [R][G][512] and meta [R][G]; A row 4m + L = limb L of activation row m (as
// in the 1-row GEMV's 4-row instance), lane group m of D holding row m's
// sums; RMSNorm only from per-row partial sums of squares (NORM 1: st.ssq_n
// <= 256 per row), slices of at most 4 groups.
template <int KIND, int NG, int TP, int NORM, int R>
__global__ __launch_bounds__(KIND == 1 ? 64 * kMaxWaves : 32 * kMaxWaves) void stage_kernel(const CStage st) {
    static_assert(R == 1 || (NG == 4 && NORM != 2), "R-row stages: 4-group slices, producer sums of squares");
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    __shared__ float red[kMaxWaves][TP][16 * R];
    __shared__ double ssq[kMaxWaves];
    __shared__ int arrived;
    constexpr int WPG = KIND == 1 ? 1 : 2;  // 16-byte weight loads per group
    constexpr int XP = NG / 4;              // conversion passes (4 groups each)
    const int tid = threadIdx.x, lane = tid & 63, ln = lane & 15, kg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nw = int(blockDim.x) >> 6;
    const int G = st.G, K = st.K;
    const int g0 = wave * st.gs < G ? wave * st.gs : G;
    const int gs = (g0 + st.gs < G ? g0 + st.gs : G) - g0;
    const int M = R == 1 ? 1 : st.rows;
    int4* ms = reinterpret_cast<int4*>(lds + R * G * kLimbRec);
    float* xraw = reinterpret_cast<float*>(lds + G * (kLimbRec + 16));

    // the unit's tiles and their matrices
    const int u = blockIdx.x;
    int m0 = 0, tile = u;
    if (TP == 1) {
        if (st.nmat > 1 && u >= st.mat[1].tile0) m0 = 1;
        if (st.nmat > 2 && u >= st.mat[2].tile0) m0 = 2;
        m0 = __builtin_amdgcn_readfirstlane(m0);
        tile = u - stage_mat(st, m0).tile0;
    }
    CMat Ms[TP];
    Ms[0] = stage_mat(st, m0);
    if (TP == 2) Ms[TP - 1] = st.mat[1];
    const int64_t row0 = int64_t(tile) * 16, N = Ms[0].N;

    // 1. Activations first (the vector L1 returns data in request order),
    //    then bias / residual, scales, zero points and weights.  Every load
    //    is a buffer load whose out-of-range offset reads zero, and no loaded
    //    value is used before all loads are issued (a use waits for every
    //    load issued before it).
    // NORM: 0 no RMSNorm; 1 from the producer's per-tile sums of squares
    // (<= 256 tiles: one 16-byte load per lane); 2 from the whole input
    constexpr bool norm = NORM != 0;
    constexpr bool full = NORM == 2;
    constexpr int kMaxChunks = NORM == 2 ? 4 : 1;  // 16-byte chunks per thread
    const int xlen = st.in_op == IQ_IN_GQA ? K / (st.gqa_span / st.gqa_hd) : K;
    const rsrc_t rx = make_rsrc(st.x, int64_t(M) * xlen * 4);
    u32x4_t xc[R == 1 ? kMaxChunks : R], xw[R][XP][2], nwv[norm ? XP : 1];
    if constexpr (full) {
        const int nchunk = K / 4, nthr = nw * 64;
#pragma unroll
        for (int i = 0; i < kMaxChunks; i++) {
            const int c = tid + i * nthr;
            xc[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, c < nchunk ? uint32_t(c) * 16 : kOob, 0, 0));
        }
    } else {
        if constexpr (norm) {
            // the producer's sums of squares, 4 per lane (row m: ssq_n of
            // them at m * ssq_n)
            const rsrc_t rp = make_rsrc(st.ssq_in, int64_t(M) * st.ssq_n * 4);
#pragma unroll
            for (int m = 0; m < (R == 1 ? 1 : R); m++) {
                const uint32_t o = (m < M && 4 * lane < st.ssq_n) ? uint32_t(m * st.ssq_n + 4 * lane) * 4 : kOob;
                xc[m] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                        rp, R == 1 ? uint32_t(lane) * 16 : o, 0, 0));
            }
        }
#pragma unroll
        for (int m = 0; m < R; m++) {
#pragma unroll
            for (int t = 0; t < XP; t++) {
                const int g = g0 + 4 * t + kg;
                int k0 = g * kGroup + ln * 8;
                if (st.in_op == IQ_IN_GQA) k0 = (k0 / st.gqa_span) * st.gqa_hd + (k0 % st.gqa_hd);
                const uint32_t off = (4 * t + kg < gs && m < M) ? uint32_t(m * xlen + k0) * 4 : kOob;
                xw[m][t][0] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
                xw[m][t][1] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 16, 0));
            }
        }
    }
    if constexpr (norm) {
        const rsrc_t rn = make_rsrc(st.norm, int64_t(K) * 2);
#pragma unroll
        for (int t = 0; t < XP; t++) {
            const int g = g0 + 4 * t + kg;
            nwv[t] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                     rn, 4 * t + kg < gs ? uint32_t(g * kGroup + ln * 8) * 2 : kOob, 0, 0));
        }
    }
    // bias (and residual) of the rows this lane may store (lane group m <
    // M of every wave, activation row m: the last wave to finish stores);
    // rows past N read zero
    uint32_t addb[TP], resb = 0;
    {
        const bool st_lane = lane < 16 * M;
        const uint32_t ro = st_lane ? uint32_t(row0 + ln) : 0x20000000u;
#pragma unroll
        for (int t = 0; t < TP; t++) {
            const rsrc_t rb = make_rsrc(Ms[t].bias, Ms[t].bias ? N * 2 : 0);
            addb[t] = __builtin_amdgcn_raw_buffer_load_b16(rb, ro * 2, 0, 0);
        }
        if (TP == 1 && st.out_op == IQ_OUT_RESIDUAL) {
            const rsrc_t rr = make_rsrc(st.res, int64_t(M) * N * 4);
            resb = __builtin_amdgcn_raw_buffer_load_b32(rr, st_lane ? uint32_t(kg * N + row0 + ln) * 4 : kOob, 0, 0);
        }
    }
    if (tid == 0) arrived = 0;
    // Every wave's activation requests go out before any wave's weight
    // requests (the barrier waits for no load); this also publishes the
    // cleared arrival counter before any wave can arrive.
    __syncthreads();

    const int64_t rb = KIND == 1 ? K / 2 : K;
    const int64_t rows = N - row0 < 16 ? N - row0 : 16;
    uint32_t sw[TP][NG / 2], zw[TP][NG / 2];
    int4v_t w[TP][NG][WPG];
#pragma unroll
    for (int t = 0; t < TP; t++) {
        const rsrc_t rs = make_rsrc(Ms[t].scales + row0 * G, rows * G * 2);
        const rsrc_t rz = make_rsrc(KIND == 1 ? Ms[t].zeros + row0 * G : nullptr, KIND == 1 ? rows * G : 0);
        const uint32_t vs = uint32_t((ln * G + g0) * 2), vz = uint32_t(ln * G + g0);
        if (G % 4 == 0) {
            // slices start on 4-group boundaries: one 8-byte scale load and
            // one 4-byte zero-point load per 4 groups
#pragma unroll
            for (int i = 0; i < NG / 4; i++) {
                const uint32_t ok = 4 * i < gs ? 0u : kOob;
                const auto sv = __builtin_amdgcn_raw_buffer_load_b64(rs, vs + ok, 8 * i, 0);
                sw[t][2 * i] = sv[0];
                sw[t][2 * i + 1] = sv[1];
                zw[t][2 * i] = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b32(rz, vz + ok, 4 * i, 0) : 0u;
            }
        } else {
#pragma unroll
            for (int i = 0; i < NG / 2; i++) {
                const uint32_t ok = 2 * i < gs ? 0u : kOob;
                sw[t][i] = __builtin_amdgcn_raw_buffer_load_b32(rs, vs + ok, 4 * i, 0);
                zw[t][i] = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b16(rz, vz + ok, 2 * i, 0) : 0u;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TP; t++) {
        const rsrc_t rq = make_rsrc(Ms[t].q + row0 * rb, rows * rb);
        const uint32_t vq = uint32_t(ln * rb) + uint32_t(g0 * (KIND == 1 ? 64 : 128) + kg * 16);
#pragma unroll
        for (int gl = 0; gl < NG; gl++)
#pragma unroll
            for (int h = 0; h < WPG; h++)
                w[t][gl][h] = __builtin_bit_cast(int4v_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                              rq, vq + (gl < gs ? 0u : kOob), KIND == 1 ? gl * 64 : gl * 128 + h * 64, 0));
    }

    // 2. The slice's activations.  RMSNorm (src/forward.cpp:21-31):
    //    x / sqrt(mean(x^2) + eps) * w, the sum of squares in double in a
    //    fixed order: from the producer's per-tile sums (every wave adds
    //    them itself), or from the whole input (reduced through LDS, the raw
    //    input kept in LDS for the slices).
    float xv[R][XP][8];
    float scale[R];
#pragma unroll
    for (int m = 0; m < R; m++) scale[m] = 1.0f;
    if constexpr (full) {
        double part = 0.0;
#pragma unroll
        for (int i = 0; i < kMaxChunks; i++)
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const double v = double(__uint_as_float(xc[i][j]));
                part += v * v;
            }
        const int nchunk = K / 4, nthr = nw * 64;
#pragma unroll
        for (int i = 0; i < kMaxChunks; i++) {
            const int c = tid + i * nthr;
            if (c < nchunk) reinterpret_cast<u32x4_t*>(xraw)[c] = xc[i];
        }
        part = wave_sum(part);
        if (lane == 0) ssq[wave] = part;
        __syncthreads();
        double ss = 0.0;
        for (int i = 0; i < nw; i++) ss += ssq[i];
        scale[0] = 1.0f / __builtin_sqrtf(float(ss / double(K)) + st.eps);
#pragma unroll
        for (int t = 0; t < XP; t++) {
            if (4 * t >= gs) continue;
            const int g = 4 * t + kg < gs ? g0 + 4 * t + kg : g0;
            const u32x4_t a = reinterpret_cast<const u32x4_t*>(xraw + g * kGroup + ln * 8)[0];
            const u32x4_t c = reinterpret_cast<const u32x4_t*>(xraw + g * kGroup + ln * 8)[1];
            xw[0][t][0] = a;
            xw[0][t][1] = c;
        }
    }
    // (from the producer's sums, NORM 1, the factor r_m multiplies the
    // output sums at the end instead: the limbs are made from x * w, so
    // the conversion does not wait for the sums of squares to land and be
    // added; (W (x w)) r and W ((x r) w) differ by fp32 rounding only)
#pragma unroll
    for (int m = 0; m < R; m++)
#pragma unroll
        for (int t = 0; t < XP; t++)
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const float r = __uint_as_float(xw[m][t][i >> 2][i & 3]);
                if constexpr (norm) {
                    const uint32_t nv = nwv[t][i >> 1];
                    const float wn = __uint_as_float((i & 1) ? (nv & 0xFFFF0000u) : (nv << 16));
                    xv[m][t][i] = (r * scale[m]) * wn;
                } else {
                    xv[m][t][i] = r;
                }
            }

    // 3. This wave's slice into limb records (row m: records m * G + g).
#pragma unroll
    for (int m = 0; m < R; m++) {
        if (m >= M) break;  // uniform
#pragma unroll
        for (int t = 0; t < XP; t++) {
            if (4 * t >= gs) continue;  // wave-uniform
            const int g = g0 + 4 * t + kg;
            const bool ok = 4 * t + kg < gs;
            const int4 md = convert_group<KIND == 1>(xv[m][t], ln, ok, lds + (m * G + (ok ? g : g0)) * kLimbRec);
            if (ok && ln == 0) ms[m * G + g] = md;
        }
    }

    // 4. Codes x limbs: A rows 0..3 = limbs 0..3 (lanes 0..15 hold the four
    //    sums of row ln in D[0..3]); the wave reads only its own records.
    //    (Fully unrolled with a wave-uniform guard: a loop the compiler does
    //    not unroll indexes the weight registers dynamically, which moves
    //    them to scratch memory.)
    float acc[TP];
#pragma unroll
    for (int t = 0; t < TP; t++) acc[t] = 0.0f;
    // A row of this lane: limb ln (R = 1) or limb ln % 4 of activation row
    // ln / 4 (R > 1); D lane group kg holds activation row kg's sums (R > 1)
    const int am = R == 1 ? 0 : ln >> 2, aL = R == 1 ? ln : ln & 3;
    const bool alive = R == 1 ? ln < kLimbs : am < M;
    const int mrow = R == 1 ? 0 : (kg < M ? kg : 0);
#pragma unroll
    for (int gl = 0; gl < NG; gl++) {
        if (gl >= gs) continue;  // wave-uniform
        const int g = g0 + gl;
        int4v_t a0 = {0, 0, 0, 0}, a1 = {0, 0, 0, 0};
        if (alive) {
            const int8_t* pa = lds + (am * G + g) * kLimbRec + aL * kGroup + kg * 16;
            a0 = *reinterpret_cast<const int4v_t*>(pa);
            a1 = *reinterpret_cast<const int4v_t*>(pa + 64);
        }
        const int4 md = ms[mrow * G + g];
#pragma unroll
        for (int t = 0; t < TP; t++) {
            int4v_t b0, b1;
            if (KIND == 1) {
                b0 = w[t][gl][0] & 0x0F0F0F0F;
                b1 = (w[t][gl][0] >> 4) & 0x0F0F0F0F;
            } else {
                b0 = w[t][gl][0];
                b1 = w[t][gl][WPG - 1];
            }
            int4v_t D = mfma_i8(a0, b0, int4v_t{0, 0, 0, 0});
            D = mfma_i8(a1, b1, D);
            const uint32_t s2 = sw[t][gl >> 1];
            const float sc = __uint_as_float((gl & 1) ? (s2 & 0xFFFF0000u) : (s2 << 16));
            const int z = KIND != 1 ? 0
                          : (G % 4 == 0 ? int((zw[t][(gl >> 2) * 2] >> (8 * (gl & 3))) & 0xFF)
                                        : int((zw[t][gl >> 1] >> (8 * (gl & 1))) & 0xFF));
            acc[t] = combine(acc[t], D[0], D[1], D[2], D[3], z, md, sc);
        }
    }

    // RMSNorm factors from the producer's per-tile sums (NORM 1), in double
    // in a fixed order, every wave (wave_sum needs all 64 lanes)
    if constexpr (NORM == 1) {
#pragma unroll
        for (int m = 0; m < R; m++) {
            double part = 0.0;
#pragma unroll
            for (int j = 0; j < 4; j++)
                part += (R == 1 || 4 * lane + j < st.ssq_n) ? double(__uint_as_float(xc[m][j])) : 0.0;
            const double ss = wave_sum(part);
            scale[m] = 1.0f / __builtin_sqrtf(float(ss / double(K)) + st.eps);
        }
    }

    // 5. Partials through LDS; the last wave adds them in wave order and
    //    applies the epilogue (and the per-tile sum of squares of the output
    //    for a consumer's RMSNorm).
    //    (R > 1: lane group m = activation row m.)
    if (lane < 16 * R) {
#pragma unroll
        for (int t = 0; t < TP; t++) red[wave][t][lane] = acc[t];
    }
    int prior = 0;
    if (lane == 0) prior = __hip_atomic_fetch_add(&arrived, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_WORKGROUP);
    prior = __builtin_amdgcn_readfirstlane(prior);
    if (prior != nw - 1 || lane >= 16 * M) return;
    float sum[TP];
#pragma unroll
    for (int t = 0; t < TP; t++) {
        sum[t] = 0.0f;
        for (int i = 0; i < nw; i++) sum[t] += red[i][t][lane];
    }
    const int64_t row = row0 + ln;
    if constexpr (NORM == 1) {
        // this lane's row: 0, or lane group kg (R > 1); no dynamic index
        float rsc = scale[0];
#pragma unroll
        for (int m = 1; m < R; m++) rsc = kg == m ? scale[m] : rsc;
#pragma unroll
        for (int t = 0; t < TP; t++) sum[t] *= rsc;
    }
    float v = sum[0] + __uint_as_float(addb[0] << 16);
    if (TP == 2) {
        // silu(g) * u  (kernels/ops/elementwise.cu:6-11)
        const float up = sum[TP - 1] + __uint_as_float(addb[TP - 1] << 16);
        v = v / (1.0f + expf(-v)) * up;
    } else if (st.out_op == IQ_OUT_RESIDUAL) {
        v = __uint_as_float(resb) + v;
    }
    if (row < N) Ms[0].y[int64_t(kg) * N + row] = v;
    if (st.ssq_out) {
        // (the 16 lanes of row kg together: M is a whole number of groups)
        const float sq = row16_fsum(row < N ? v * v : 0.0f);
        if (ln == 0) st.ssq_out[R == 1 ? tile : kg * ((N + 15) / 16) + tile] = sq;
    }
}

// Sum over the 256 threads of a block, in a fixed order (shuffle tree per
// wave, then the four wave sums in order); the result in thread 0.
__device__ __forceinline__ float block256_sum(float v, float* red4) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) red4[threadIdx.x >> 6] = v;
    __syncthreads();
    return ((red4[0] + red4[1]) + red4[2]) + red4[3];
}

// Output side of a B-row stage: thread (column c, row m = blockIdx.y).
__global__ __launch_bounds__(256) void epi_kernel(const CEpi e) {
    __shared__ float red4[4];
    const int m = blockIdx.y;
    const int c = int(blockIdx.x) * 256 + int(threadIdx.x);
    const int64_t stride = int64_t(e.M) * e.ld, base = int64_t(m) * e.ld;
    float v = 0.0f;
    bool valid = false;
    if (c < e.ncols) {
        if (e.swiglu) {
            // silu(g) * u  (kernels/ops/elementwise.cu:6-11)
            const float g = sum_slices(e.part, e.S, stride, base + c) + (e.bias[0] ? bf16_to_f32(e.bias[0][c]) : 0.0f);
            const float u = sum_slices(e.part, e.S, stride, base + int64_t(e.tile0[1]) * 16 + c) +
                            (e.bias[1] ? bf16_to_f32(e.bias[1][c]) : 0.0f);
            v = g / (1.0f + expf(-g)) * u;
            e.y[0][int64_t(m) * e.N[0] + c] = v;
            valid = true;
        } else {
            int i = 0;
            for (int k = 1; k < e.nmat; k++)
                if (c >= e.tile0[k] * 16) i = k;
            const int col = c - e.tile0[i] * 16;
            if (col < e.N[i]) {
                v = sum_slices(e.part, e.S, stride, base + c) + (e.bias[i] ? bf16_to_f32(e.bias[i][col]) : 0.0f);
                if (e.res) v = e.res[int64_t(m) * e.N[0] + col] + v;
                e.y[i][int64_t(m) * e.N[i] + col] = v;
                valid = true;
            }
        }
    }
    if (e.ssq_out) {
        const float sq = block256_sum(valid ? v * v : 0.0f, red4);
        if (threadIdx.x == 0) e.ssq_out[int64_t(m) * e.ssq_n + blockIdx.x] = sq;
    }
}

// Sums of squares of the 256-column blocks of each row of x [M][K] (row
// stride K), for an RMSNorm input that no earlier stage produced.
__global__ __launch_bounds__(256) void ssq_kernel(const float* __restrict__ x, int K, int ssq_n,
                                                  float* __restrict__ ssq) {
    __shared__ float red4[4];
    const int m = blockIdx.y;
    const int c = int(blockIdx.x) * 256 + int(threadIdx.x);
    const float v = c < K ? x[int64_t(m) * K + c] : 0.0f;
    const float sq = block256_sum(v * v, red4);
    if (threadIdx.x == 0) ssq[int64_t(m) * ssq_n + blockIdx.x] = sq;
}

hipError_t run_rows_stage(const HostStage& h, float* part, int64_t part_floats, hipStream_t stream) {
    if (h.own_ssq) {
        const int K = int(h.W[0].cols);
        ssq_kernel<<<dim3(unsigned(h.in.ssq_n), unsigned(h.rows)), 256, 0, stream>>>(h.in.x, K, h.in.ssq_n, h.ssq);
    }
    int S = 0;
    hipError_t e = launch_chain_rows(h.W, h.st.nmat, h.rows, h.in, part, part_floats, &S, stream);
    if (e != hipSuccess) return e;
    CEpi ep = h.epi;
    ep.part = part;
    ep.S = S;
    epi_kernel<<<dim3(unsigned((ep.ncols + 255) / 256), unsigned(h.rows)), 256, 0, stream>>>(ep);
    return hipGetLastError();
}

template <int KIND>
hipError_t launch_stage_k(const HostStage& h, hipStream_t stream) {
    const dim3 grid(unsigned(h.st.units)), block(unsigned(64 * h.st.ks));
    const int norm = h.st.in_op != IQ_IN_RMSNORM ? 0 : (h.st.ssq_in ? 1 : 2);
#define IQ_STAGE1(NG_, TP_, N_, R_)                                                         \
    do {                                                                                    \
        allow_big_lds<stage_kernel<KIND, NG_, TP_, N_, R_>>();                              \
        stage_kernel<KIND, NG_, TP_, N_, R_><<<grid, block, h.lds, stream>>>(h.st);         \
    } while (0)
#define IQ_STAGE(NG_, TP_)                                                                  \
    do {                                                                                    \
        if (norm == 1) IQ_STAGE1(NG_, TP_, 1, 1);                                           \
        else if (norm == 2) IQ_STAGE1(NG_, TP_, 2, 1);                                      \
        else IQ_STAGE1(NG_, TP_, 0, 1);                                                     \
    } while (0)
#define IQ_STAGER(TP_, R_)                                                                  \
    do {                                                                                    \
        if (norm == 1) IQ_STAGE1(4, TP_, 1, R_);                                            \
        else IQ_STAGE1(4, TP_, 0, R_);                                                      \
    } while (0)
    if (h.fused_r > 1) {
        // (norm == 2 never reaches an R-row stage: chain_create gives its
        // input per-row sums of squares)
        if (h.fused_r == 2) {
            if (h.st.tpu == 2) IQ_STAGER(2, 2);
            else IQ_STAGER(1, 2);
        } else {
            if (h.st.tpu == 2) IQ_STAGER(2, 4);
            else IQ_STAGER(1, 4);
        }
    } else if (h.st.tpu == 2) {
        if (h.ng == 4) IQ_STAGE(4, 2);
        else IQ_STAGE(8, 2);
    } else {
        switch (h.ng) {
            case 4: IQ_STAGE(4, 1); break;
            case 8: IQ_STAGE(8, 1); break;
            case 12: IQ_STAGE(12, 1); break;
            default:
                if constexpr (KIND == 0) IQ_STAGE(20, 1);
                break;
        }
    }
#undef IQ_STAGE
#undef IQ_STAGE1
#undef IQ_STAGER
    return hipGetLastError();
}

struct Range {
    uintptr_t lo, hi;
};
bool overlaps(const Range& a, const Range& b) { return a.lo < b.hi && b.lo < a.hi; }

}  // namespace

// Host side of a chain: the validated stages and their launch shapes.
struct Chain {
    int device = 0;
    std::vector<HostStage> stages;
    float* partials = nullptr;  // per-tile sums of squares passed between stages
    // B-row stages: K-range sums (one buffer, the stages run in order) and
    // the per-row block sums of squares
    float* rpart = nullptr;
    int64_t rpart_floats = 0;
    float* rssq = nullptr;
    // narrow B-row stages: their prepared f16 operands (one stage at a time)
    int8_t* hxq = nullptr;
    float* hxmeta = nullptr;
};

int chain_create(const iq_stage* stages, int n, Chain** out) {
    if (!stages || !out) return IQ_ENULL;
    *out = nullptr;
    if (n < 1) return IQ_ESHAPE;
    std::vector<HostStage> prog(static_cast<size_t>(n));
    for (int s = 0; s < n; s++) {
        const iq_stage& a = stages[s];
        HostStage& hs = prog[size_t(s)];
        CStage& c = hs.st;
        std::memset(&c, 0, sizeof(c));
        if (a.n < 1 || a.n > kMaxStageMats) return IQ_ESHAPE;
        const int rows = a.rows == 0 ? 1 : a.rows;
        if (rows < 1 || rows > kMaxRowsGemv) return IQ_ESHAPE;
        hs.rows = rows;
        if (a.in_op < IQ_IN_PLAIN || a.in_op > IQ_IN_GQA) return IQ_ESHAPE;
        if (a.out_op < IQ_OUT_STORE || a.out_op > IQ_OUT_SWIGLU) return IQ_ESHAPE;
        const iq_view& W0 = a.W[0];
        if (W0.kind != IQ_INT8 && W0.kind != IQ_INT4) return IQ_EKIND;
        const int64_t K = W0.cols, G = (K + kGroup - 1) / kGroup;
        // whole groups and an even group count (paired scale loads)
        if (K <= 0 || K % (2 * kGroup)) return IQ_ESHAPE;
        int tiles = 0;
        for (int i = 0; i < a.n; i++) {
            const iq_view& Wi = a.W[i];
            if (Wi.kind != W0.kind) return IQ_EKIND;
            if (Wi.cols != K || Wi.groups != G || Wi.rows <= 0 || Wi.rows > (int64_t(1) << 30)) return IQ_ESHAPE;
            if (!Wi.q || !Wi.scales || (Wi.kind == IQ_INT4 && !Wi.zeros)) return IQ_ENULL;
            const int64_t rb = Wi.kind == IQ_INT4 ? K / 2 : K;
            if (16 * rb >= (int64_t(1) << 31)) return IQ_ETOOLARGE;
            c.mat[i] = CMat{Wi.q, Wi.scales, Wi.kind == IQ_INT4 ? Wi.zeros : nullptr, a.bias[i], a.y[i],
                            int32_t(Wi.rows), tiles};
            tiles += int((Wi.rows + 15) / 16);
        }
        const bool pair = a.out_op == IQ_OUT_SWIGLU;
        if (pair && (a.n != 2 || a.W[1].rows != W0.rows)) return IQ_ESHAPE;
        if (a.out_op == IQ_OUT_RESIDUAL && a.n != 1) return IQ_ESHAPE;
        std::vector<Range> reads, writes;
        const int nout = pair ? 1 : a.n;
        for (int i = 0; i < nout; i++) {
            if (!a.y[i]) return IQ_ENULL;
            writes.push_back({reinterpret_cast<uintptr_t>(a.y[i]),
                              reinterpret_cast<uintptr_t>(a.y[i] + int64_t(rows) * a.W[i].rows)});
        }
        if (!a.x) return IQ_ENULL;
        if (reinterpret_cast<uintptr_t>(a.x) % 16) return IQ_ESHAPE;
        int64_t xlen = K;
        if (a.in_op == IQ_IN_GQA) {
            const int64_t hd = a.gqa_head_dim, grp = a.gqa_group;
            if (hd <= 0 || hd % 8 || grp <= 0 || K % (hd * grp)) return IQ_ESHAPE;
            c.gqa_hd = int32_t(hd);
            c.gqa_span = int32_t(hd * grp);
            xlen = K / grp;
        }
        reads.push_back({reinterpret_cast<uintptr_t>(a.x), reinterpret_cast<uintptr_t>(a.x + int64_t(rows) * xlen)});
        if (a.in_op == IQ_IN_RMSNORM) {
            if (!a.norm) return IQ_ENULL;
            if (reinterpret_cast<uintptr_t>(a.norm) % 16) return IQ_ESHAPE;
            if (!(a.eps >= 0.0f)) return IQ_ESHAPE;
            if (K > 16384) return IQ_ETOOLARGE;  // the raw input is kept in LDS
        }
        if (a.out_op == IQ_OUT_RESIDUAL) {
            if (!a.residual) return IQ_ENULL;
            reads.push_back({reinterpret_cast<uintptr_t>(a.residual),
                             reinterpret_cast<uintptr_t>(a.residual + int64_t(rows) * W0.rows)});
        }
        // a stage's workgroups read its inputs while others store: no output
        // may overlap an input or another output of the same stage
        for (size_t i = 0; i < writes.size(); i++) {
            for (const Range& r : reads)
                if (overlaps(writes[i], r)) return IQ_EALIAS;
            for (size_t j = 0; j < i; j++)
                if (overlaps(writes[i], writes[j])) return IQ_EALIAS;
        }
        c.x = a.x;
        c.norm = a.norm;
        c.res = a.residual;
        c.eps = a.eps;
        c.in_op = a.in_op;
        c.out_op = a.out_op;
        c.nmat = a.n;
        c.K = int32_t(K);
        c.G = int32_t(G);
        c.tpu = pair ? 2 : 1;
        c.units = pair ? int((W0.rows + 15) / 16) : tiles;
        hs.kind = W0.kind;
        const bool i4 = W0.kind == IQ_INT4;
        const int maxw = i4 ? kMaxWaves : kMaxWaves / 2;
        // (3..4 rows of a very wide stage, the lm_head: the B-row route; 7B
        // chain at 3 / 4 sequences 1904 / 1985 -> 1885 / 1965 us; a SwiGLU
        // pair stays fused, 26.7 us against 29.2 for gemvr and its range
        // sums on 7B gate|up at 4 rows)
        const bool wide4 = rows >= 3 && rows <= 4 && !pair && tiles >= 4096;
        if (rows > 1 && rows <= 4 && !wide4 && G <= int64_t(4) * maxw &&
            size_t(rows <= 2 ? 2 : 4) * size_t(G) * (kLimbRec + 16) <= 160 * 1024) {
            // 2..4 rows on short rows: one fused launch (the R-row
            // stage_kernel: 4-group slices, the limbs of every row in LDS)
            hs.fused_r = rows <= 2 ? 2 : 4;
            hs.rows = rows;
            c.rows = rows;
            c.gs = 4;
            c.ks = int((G + 3) / 4);
            hs.ng = 4;
            hs.lds = size_t(hs.fused_r) * size_t(G) * (kLimbRec + 16);
            hs.in.x = a.x;
            hs.in.xstride = xlen;
            hs.W[0] = QView{W0.kind, W0.rows, W0.cols, W0.groups, W0.q, W0.scales, nullptr};
            continue;
        }
        if (rows > 1) {
            // B rows: the rows GEMV (gemvr / gemvq with the input transform)
            // and epi_kernel
            for (int i = 0; i < a.n; i++) {
                const iq_view& Wi = a.W[i];
                hs.W[i] = QView{Wi.kind, Wi.rows, Wi.cols, Wi.groups, Wi.q, Wi.scales,
                                Wi.kind == IQ_INT4 ? Wi.zeros : nullptr};
            }
            if (chain_rows_partials(hs.W, a.n, rows, kStreamPartialFloats) < 0) return IQ_ETOOLARGE;
            hs.in.x = a.x;
            hs.in.xstride = xlen;
            hs.in.gqa_hd = a.in_op == IQ_IN_GQA ? a.gqa_head_dim : 0;
            hs.in.gqa_span = a.in_op == IQ_IN_GQA ? a.gqa_head_dim * a.gqa_group : 0;
            hs.in.norm = a.in_op == IQ_IN_RMSNORM ? a.norm : nullptr;
            hs.in.eps = a.eps;
            CEpi& ep = hs.epi;
            for (int i = 0; i < a.n; i++) {
                ep.y[i] = a.y[i];
                ep.bias[i] = a.bias[i];
                ep.N[i] = int32_t(a.W[i].rows);
                ep.tile0[i] = c.mat[i].tile0;
            }
            ep.nmat = a.n;
            ep.M = rows;
            ep.ld = int64_t(tiles) * 16;
            ep.swiglu = pair ? 1 : 0;
            ep.res = a.out_op == IQ_OUT_RESIDUAL ? a.residual : nullptr;
            ep.ncols = pair ? int32_t(W0.rows) : int32_t(ep.ld);
            // narrow stages (q|k|v, o at 9..32 rows): the input transform
            // into prepared f16 operands, then gemvh with bias, residual and
            // per-tile sums of squares in its own epilogue
            hs.hroute = !pair && (a.out_op != IQ_OUT_RESIDUAL || a.n == 1) && chain_h_applies(hs.W, a.n, rows);
            continue;
        }
        // slices of whole 4-group blocks (measured: fewer, fatter waves beat
        // more waves with 2 groups each), at most 16 waves of <= 12 groups
        // (int4) or 8 waves of <= 20 groups (int8: twice the weight
        // registers per group); a SwiGLU pair holds two tiles per wave
        int gs = int((G + maxw - 1) / maxw);
        gs = (gs + 3) & ~3;
        if (gs > (pair ? 8 : (i4 ? 12 : 20))) return IQ_ETOOLARGE;
        c.gs = gs;
        c.ks = int((G + gs - 1) / gs);
        hs.ng = gs;
        // RMSNorm from the whole input: at most four 16-byte chunks per thread
        if (a.in_op == IQ_IN_RMSNORM && K > 16 * 64 * int64_t(c.ks)) return IQ_ETOOLARGE;
        hs.lds = size_t(G) * (kLimbRec + 16) + (a.in_op == IQ_IN_RMSNORM ? size_t(K) * 4 : 0);
        if (hs.lds > 160 * 1024) return IQ_ETOOLARGE;
    }
    // (a consumer takes the producer's partial sums only when they fit one
    // 16-byte load per lane: <= 256 tiles, K <= 4096)
    // RMSNorm inputs produced by an earlier stage of the chain: that stage
    // also writes per-tile sums of squares, so the consumer's workgroups
    // need not read the whole vector (unless a stage in between rewrites it)
    std::vector<std::pair<int, int>> links;  // (producer, consumer)
    auto rows_of = [&](int i) { return stages[i].rows == 0 ? 1 : stages[i].rows; };
    for (int s = 0; s < n; s++) {
        if (stages[s].in_op != IQ_IN_RMSNORM) continue;
        const float* x = stages[s].x;
        const int64_t K = stages[s].W[0].cols;
        const int B = rows_of(s);
        for (int e = s - 1; e >= 0; e--) {
            const iq_stage& a = stages[e];
            const int nout = a.out_op == IQ_OUT_SWIGLU ? 1 : a.n;
            const int Be = rows_of(e);
            bool hit = false, clash = false;
            for (int i = 0; i < nout; i++) {
                const Range w{reinterpret_cast<uintptr_t>(a.y[i]),
                              reinterpret_cast<uintptr_t>(a.y[i] + int64_t(Be) * a.W[i].rows)};
                if (a.y[i] == x && a.W[i].rows == K && nout == 1 && Be == B && (B > 1 || K <= 4096)) hit = true;
                else if (overlaps(w, Range{reinterpret_cast<uintptr_t>(x), reinterpret_cast<uintptr_t>(x + int64_t(B) * K)}))
                    clash = true;
            }
            if (hit) links.emplace_back(e, s);
            if (hit || clash) break;
        }
    }
    Chain* ch = new Chain();
    if (hipGetDevice(&ch->device) != hipSuccess) {
        delete ch;
        return IQ_EDEVICE;
    }
    auto fail = [&](hipError_t e) {
        chain_destroy(ch);
        return e == hipErrorOutOfMemory ? IQ_ENOMEM : int(e);
    };
    // 1 row: one per-tile partial-sum array per producer
    {
        std::vector<size_t> off(static_cast<size_t>(n), size_t(-1));
        size_t total = 0;
        for (const auto& l : links)
            if (rows_of(l.first) == 1 && off[size_t(l.first)] == size_t(-1)) {
                off[size_t(l.first)] = total;
                total += size_t((prog[size_t(l.first)].st.mat[0].N + 15) / 16 + 63) / 64 * 64;
            }
        if (total) {
            const hipError_t e = hipMalloc(reinterpret_cast<void**>(&ch->partials), total * sizeof(float));
            if (e != hipSuccess) return fail(e);
            for (const auto& l : links) {
                if (rows_of(l.first) != 1) continue;
                float* p = ch->partials + off[size_t(l.first)];
                prog[size_t(l.first)].st.ssq_out = p;
                prog[size_t(l.second)].st.ssq_in = p;
                prog[size_t(l.second)].st.ssq_n = (prog[size_t(l.first)].st.mat[0].N + 15) / 16;
            }
        }
    }
    // B rows: per-row sums of squares of an RMSNorm input, written by the
    // stage that produced it (a B-row epi_kernel: one per 256-column block;
    // an R-row stage_kernel: one per 16-row output tile) or by ssq_kernel
    // (inputs no stage of the chain produces: one per 256-column block), at
    // most 256 per row; one K-range partial-sum buffer for all B-row GEMVs
    {
        std::vector<size_t> off(static_cast<size_t>(n), size_t(-1));  // by producer / own consumer
        std::vector<int> producer(static_cast<size_t>(n), -1);
        auto ssq_count = [&](int e) {
            const HostStage& hp = prog[size_t(e)];
            return (hp.fused_r > 1 || hp.hroute) ? int((hp.st.mat[0].N + 15) / 16) : int((hp.epi.ncols + 255) / 256);
        };
        for (const auto& l : links)
            if (rows_of(l.second) > 1 && ssq_count(l.first) <= 256) producer[size_t(l.second)] = l.first;
        size_t total = 0;
        int64_t part = 0;
        for (int s = 0; s < n; s++) {
            HostStage& h = prog[size_t(s)];
            if (h.rows == 1) continue;
            if (h.fused_r == 1)
                part = std::max<int64_t>(part, chain_rows_partials(h.W, h.st.nmat, h.rows, kStreamPartialFloats));
            if (stages[s].in_op != IQ_IN_RMSNORM) continue;
            const int pe = producer[size_t(s)];
            const int key = pe >= 0 ? pe : s;
            const int64_t K = h.W[0].cols;
            const int ssq_n = pe >= 0 ? ssq_count(pe) : int((K + 255) / 256);
            if (off[size_t(key)] == size_t(-1)) {
                off[size_t(key)] = total;
                total += size_t(h.rows) * size_t(ssq_n);
            }
            h.in.ssq_n = ssq_n;
            h.own_ssq = pe < 0;
        }
        if (total) {
            const hipError_t e = hipMalloc(reinterpret_cast<void**>(&ch->rssq), total * sizeof(float));
            if (e != hipSuccess) return fail(e);
            for (int s = 0; s < n; s++) {
                HostStage& h = prog[size_t(s)];
                if (h.rows == 1 || stages[s].in_op != IQ_IN_RMSNORM) continue;
                const int pe = producer[size_t(s)];
                float* p = ch->rssq + off[size_t(pe >= 0 ? pe : s)];
                h.ssq = p;
                h.in.ssq = p;
                if (h.fused_r > 1) {
                    h.st.ssq_in = p;
                    h.st.ssq_n = h.in.ssq_n;
                }
                if (pe >= 0) {
                    HostStage& hp = prog[size_t(pe)];
                    if (hp.fused_r > 1) {
                        hp.st.ssq_out = p;
                    } else {
                        hp.epi.ssq_out = p;
                        hp.epi.ssq_n = h.in.ssq_n;
                    }
                }
            }
        }
        if (part > 0) {
            const hipError_t e = hipMalloc(reinterpret_cast<void**>(&ch->rpart), size_t(part) * sizeof(float));
            if (e != hipSuccess) return fail(e);
            ch->rpart_floats = part;
        }
        size_t hxq = 0, hmeta = 0;
        for (const HostStage& h : prog) {
            if (!h.hroute) continue;
            size_t xb = 0, mf = 0;
            chain_h_bytes(h.W[0].groups, h.rows, &xb, &mf);
            hxq = std::max(hxq, xb);
            hmeta = std::max(hmeta, mf);
        }
        if (hxq) {
            hipError_t e = hipMalloc(reinterpret_cast<void**>(&ch->hxq), hxq);
            if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&ch->hxmeta), hmeta * sizeof(float));
            if (e != hipSuccess) return fail(e);
        }
    }
    ch->stages = std::move(prog);
    *out = ch;
    return IQ_OK;
}

hipError_t chain_run(const Chain* ch, hipStream_t stream) {
    for (const HostStage& h : ch->stages) {
        hipError_t e;
        if (h.rows > 1 && h.fused_r == 1 && h.hroute) {
            if (h.own_ssq) {
                const int K = int(h.W[0].cols);
                ssq_kernel<<<dim3(unsigned(h.in.ssq_n), unsigned(h.rows)), 256, 0, stream>>>(h.in.x, K, h.in.ssq_n, h.ssq);
            }
            e = launch_chain_h(h.W, h.st.nmat, h.rows, h.in, h.epi.bias, h.epi.y, h.epi.res, h.epi.ssq_out, ch->hxq,
                               ch->hxmeta, stream);
        } else if (h.rows > 1 && h.fused_r == 1) {
            e = run_rows_stage(h, ch->rpart, ch->rpart_floats, stream);
        } else {
            if (h.own_ssq) {
                // (an R-row stage whose RMSNorm input no stage produced)
                ssq_kernel<<<dim3(unsigned(h.in.ssq_n), unsigned(h.rows)), 256, 0, stream>>>(
                    h.in.x, int(h.W[0].cols), h.in.ssq_n, h.ssq);
            }
            e = h.kind == IQ_INT4 ? launch_stage_k<1>(h, stream) : launch_stage_k<0>(h, stream);
        }
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

void chain_destroy(Chain* ch) {
    if (!ch) return;
    if (ch->partials) (void)hipFree(ch->partials);
    if (ch->rpart) (void)hipFree(ch->rpart);
    if (ch->rssq) (void)hipFree(ch->rssq);
    if (ch->hxq) (void)hipFree(ch->hxq);
    if (ch->hxmeta) (void)hipFree(ch->hxmeta);
    delete ch;
}

}  // namespace iq

// The opaque handle of include/iq.h is the library's Chain.
struct iq_chain : iq::Chain {};

extern "C" {

int iq_chain_create(const iq_stage* stages, int n, iq_chain** out) {
    iq::Chain* ch = nullptr;
    const int rc = iq::chain_create(stages, n, &ch);
    if (out) *out = static_cast<iq_chain*>(ch);
    return rc;
}

int iq_chain_run(const iq_chain* chain, void* stream) {
    if (!chain) return IQ_ENULL;
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return int(e);
    if (dev != chain->device) return IQ_EDEVICE;
    const hipError_t r = iq::chain_run(chain, static_cast<hipStream_t>(stream));
    return r == hipSuccess ? IQ_OK : int(r);
}

void iq_chain_destroy(iq_chain* chain) { iq::chain_destroy(chain); }

}  // extern "C"

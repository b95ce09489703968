// iq_gemv.hip -- dequant GEMV for 1..32 activation rows on gfx950 MFMA.
//
// Replaces the reference's gemv_q_direct_kernel / gemv_batched_q_kernel
// (kernels/ops/quant.cu:71-252) and their dispatch (quant.cu:312-345).
// Semantics: y[m,n] = sum_k dequant(W,n,k) * x[m,k] (+ bias[n]).
//
// Two launches:
//  1. xprep: the fp32 activations are cut into 128-column groups (the weight
//     group size).  Each (row, group) is scaled by a power of two 2^e chosen
//     from its absmax so that it fits fp16's range, then split exactly-ish
//     into fp16 hi + lo (x*2^e = hi + lo + O(2^-22)).  hi/lo are written in
//     the column order the weight dequantisation produces (see iq_device.h),
//     2^-e is kept per (group, row).  Scaling by a power of two is exact.
//  2. gemv: MFMA f32_16x16x32_f16 with the activations as the A operand
//     (16 rows, zero beyond M) and the weights as B (16 output rows per
//     tile).  Weight codes stream from HBM as 16-byte loads per lane (a wave
//     reads 16 rows x 64 contiguous bytes per instruction) and are turned
//     into exact fp16 integers in registers (q or q - z).  Per 128-column
//     group the MFMA partial D_g = sum (q-z)*(hi+lo) is formed from zero and
//     folded into the fp32 accumulator as acc += (s * 2^-e) * D_g, so the
//     bf16 scale and the activation prescale are applied in fp32.  A wave
//     owns R tiles of 16 rows (register tiling: the activation fragments
//     are loaded once per group and reused by all R tiles) and one slice of
//     the groups.  When the groups are split across waves (split-K, to put
//     enough waves on the 256 CUs for short-and-wide matrices), every wave
//     writes its partial sums, and the last wave to finish a row block
//     (counted with a device-scope atomic) adds the S partials in slice order
//     - deterministic - adds the bias and writes y.  The counter is reset by
//     that wave, so the kernel needs no clearing between launches and can be
//     captured in a graph.
//
// Accuracy: weight and activation fragments are exact up to the 2^-22
// relative hi/lo residual; products are exact in the MFMA and accumulate in
// fp32.  The result is within a few fp32 ulps of the conditioning
// sum |w*x|, inside the reference test's 5e-6 (tests/test_ops_gpu.cu:199-206).
#include "iq_internal.h"

namespace iq {

namespace {

constexpr int kWaves = 4;  // waves per workgroup
constexpr int kXinvStride = kMaxRowsGemv;

// ------------------------------------------------------------------ xprep
template <bool PERM, bool VECX>
__global__ __launch_bounds__(256) void xprep_kernel(const float* __restrict__ x, int M, int64_t K,
                                                    int64_t G, int64_t Kp, int64_t quads,
                                                    _Float16* __restrict__ xh,
                                                    _Float16* __restrict__ xl,
                                                    float* __restrict__ xinv) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (wave >= int64_t(M) * quads) return;
    const int m = int(wave / quads);
    const int64_t g = (wave % quads) * 4 + (lane >> 4);
    const bool gvalid = g < G;
    const int64_t c0 = g * kGroup + (lane & 15) * 8;
    const float* xr = x + int64_t(m) * K;
    float v[8];
    if (VECX && gvalid && c0 + 8 <= K) {
        const float4 a = *reinterpret_cast<const float4*>(xr + c0);
        const float4 b = *reinterpret_cast<const float4*>(xr + c0 + 4);
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (gvalid && c0 + i < K) ? xr[c0 + i] : 0.0f;
    }
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) amax = fmaxf(amax, __builtin_fabsf(v[i]));
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 16));
    // 2^k with amax * 2^k in [2^14, 2^15): |hi| stays below fp16's 65504.
    int k = 0;
    if (amax > 0.0f && amax <= 3.0e38f) {
        int E;
        (void)frexpf(amax, &E);  // amax = f * 2^E, f in [0.5, 1)
        k = 15 - E;
        k = k < -126 ? -126 : (k > 127 ? 127 : k);
    }
    const float sc = ldexpf(1.0f, k);
    if (!gvalid) return;
    uint32_t hb[4], lb[4];
#pragma unroll
    for (int o = 0; o < 8; o += 2) {
        const int i0 = PERM ? perm8(o) : o, i1 = PERM ? perm8(o + 1) : o + 1;
        const float a0 = v[i0] * sc, a1 = v[i1] * sc;
        const _Float16 h0 = _Float16(a0), h1 = _Float16(a1);
        const _Float16 l0 = _Float16(a0 - float(h0)), l1 = _Float16(a1 - float(h1));
        hb[o / 2] = uint32_t(__builtin_bit_cast(uint16_t, h0)) | (uint32_t(__builtin_bit_cast(uint16_t, h1)) << 16);
        lb[o / 2] = uint32_t(__builtin_bit_cast(uint16_t, l0)) | (uint32_t(__builtin_bit_cast(uint16_t, l1)) << 16);
    }
    *reinterpret_cast<uint4*>(xh + int64_t(m) * Kp + c0) = make_uint4(hb[0], hb[1], hb[2], hb[3]);
    *reinterpret_cast<uint4*>(xl + int64_t(m) * Kp + c0) = make_uint4(lb[0], lb[1], lb[2], lb[3]);
    if ((lane & 15) == 0) xinv[g * kXinvStride + m] = ldexpf(1.0f, -k);
}

// ------------------------------------------------------------------ gemv
struct GemvParams {
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
    int64_t N, K, G, Kp;
    const _Float16* xh;
    const _Float16* xl;
    const float* xinv;
    const uint16_t* bias;
    float* y;
    float* part;
    int* cnt;
    int M, S, gs, nrb, nrb_pad;
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

template <int KIND, int MT, int R, bool FAST>
__global__ __launch_bounds__(256) void gemv_kernel(const GemvParams p) {
    const int lane = threadIdx.x & 63, ln = lane & 15, kg = lane >> 4;
    const int wid = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const int ks = wid / p.nrb_pad, rb = wid % p.nrb_pad;
    if (rb >= p.nrb) return;
    const int64_t row0 = int64_t(rb) * 16 * R;
    const int64_t row_bytes = KIND == 1 ? p.K / 2 : p.K;

    const uint8_t* qrow[R];
    const uint16_t* srow[R];
    const uint8_t* zrow[R];
    bool rv[R];
#pragma unroll
    for (int t = 0; t < R; t++) {
        const int64_t r = row0 + 16 * t + ln;
        rv[t] = r < p.N;
        const int64_t rc = rv[t] ? r : p.N - 1;
        qrow[t] = p.q + rc * row_bytes;
        srow[t] = p.scales + rc * p.G;
        zrow[t] = KIND == 1 ? p.zeros + rc * p.G : nullptr;
    }
    bool mv[MT];
    const _Float16* xhr[MT];
    const _Float16* xlr[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int m = mt * 16 + ln;
        mv[mt] = m < p.M;
        xhr[mt] = p.xh + int64_t(mv[mt] ? m : 0) * p.Kp;
        xlr[mt] = p.xl + int64_t(mv[mt] ? m : 0) * p.Kp;
    }

    float4_t acc[R][MT];
#pragma unroll
    for (int t = 0; t < R; t++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++) acc[t][mt] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int64_t g0 = int64_t(ks) * p.gs;
    const int64_t g1 = g0 + p.gs < p.G ? g0 + p.gs : p.G;
    for (int64_t g = g0; g < g1; g++) {
        // Activation fragments: 4 chunks of 8 columns per lane for this group.
        half8_t xa[MT][4], xb[MT][4];
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int64_t off = g * kGroup + (KIND == 1 ? kg * 32 + 8 * c : (c >> 1) * 64 + kg * 16 + 8 * (c & 1));
                if (mv[mt]) {
                    xa[mt][c] = *reinterpret_cast<const half8_t*>(xhr[mt] + off);
                    xb[mt][c] = *reinterpret_cast<const half8_t*>(xlr[mt] + off);
                } else {
                    xa[mt][c] = half8_t{0, 0, 0, 0, 0, 0, 0, 0};
                    xb[mt][c] = xa[mt][c];
                }
            }
        }
        float4_t inv[MT];
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
            inv[mt] = *reinterpret_cast<const float4_t*>(p.xinv + g * kXinvStride + mt * 16 + 4 * kg);

#pragma unroll
        for (int t = 0; t < R; t++) {
            const float s = bf16_to_f32(srow[t][g]);
            half8_t wf[4];
            if (KIND == 1) {
                const uint4 wv = FAST ? *reinterpret_cast<const uint4*>(qrow[t] + g * 64 + kg * 16)
                                      : load16_slow(qrow[t], g * 64 + kg * 16, row_bytes);
                const uint32_t z = zrow[t][g];
                const uint32_t zb = zpair_1024(z), zc = zpair_64(z);
                const uint32_t d[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    uint32_t o0, o1, o2, o3;
                    dq_int4_x8(d[c], zb, zc, o0, o1, o2, o3);
                    wf[c] = pack_h8(o0, o1, o2, o3);
                }
            } else {
                const uint4 wa = FAST ? *reinterpret_cast<const uint4*>(qrow[t] + g * 128 + kg * 16)
                                      : load16_slow(qrow[t], g * 128 + kg * 16, row_bytes);
                const uint4 wb = FAST ? *reinterpret_cast<const uint4*>(qrow[t] + g * 128 + 64 + kg * 16)
                                      : load16_slow(qrow[t], g * 128 + 64 + kg * 16, row_bytes);
                const uint32_t d[8] = {wa.x, wa.y, wa.z, wa.w, wb.x, wb.y, wb.z, wb.w};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    uint32_t o0, o1, o2, o3;
                    dq_int8_x4(d[2 * c], o0, o1);
                    dq_int8_x4(d[2 * c + 1], o2, o3);
                    wf[c] = pack_h8(o0, o1, o2, o3);
                }
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++) {
                float4_t D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    D = mfma16(xa[mt][c], wf[c], D);
                    D = mfma16(xb[mt][c], wf[c], D);
                }
#pragma unroll
                for (int r = 0; r < 4; r++) acc[t][mt][r] = __builtin_fmaf(s * inv[mt][r], D[r], acc[t][mt][r]);
            }
        }
    }

    // Epilogue.  Lane holds D rows m = mt*16 + 4*kg + r for output n = row0+16t+ln.
    if (p.S == 1) {
#pragma unroll
        for (int t = 0; t < R; t++) {
            if (!rv[t]) continue;
            const int64_t n = row0 + 16 * t + ln;
            const float b = p.bias ? bf16_to_f32(p.bias[n]) : 0.0f;
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = mt * 16 + 4 * kg + r;
                    if (m < p.M) p.y[int64_t(m) * p.N + n] = acc[t][mt][r] + b;
                }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < R; t++) {
        if (!rv[t]) continue;
        const int64_t n = row0 + 16 * t + ln;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = mt * 16 + 4 * kg + r;
                if (m < p.M) p.part[(int64_t(ks) * p.M + m) * p.N + n] = acc[t][mt][r];
            }
    }
    __threadfence();
    int prev = 0;
    if (lane == 0) prev = atomicAdd(p.cnt + rb, 1);
    prev = __shfl(prev, 0);
    if (prev != p.S - 1) return;
    __threadfence();
#pragma unroll
    for (int t = 0; t < R; t++) {
        if (!rv[t]) continue;
        const int64_t n = row0 + 16 * t + ln;
        const float b = p.bias ? bf16_to_f32(p.bias[n]) : 0.0f;
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = mt * 16 + 4 * kg + r;
                if (m >= p.M) continue;
                float sum = 0.0f;
                for (int s = 0; s < p.S; s++) sum += __builtin_nontemporal_load(p.part + (int64_t(s) * p.M + m) * p.N + n);
                p.y[int64_t(m) * p.N + n] = sum + b;
            }
    }
    if (lane == 0) p.cnt[rb] = 0;
}

template <int KIND, int MT, int R>
void launch_gemv_t(const GemvParams& p, bool fast, unsigned grid, hipStream_t stream) {
    if (fast) gemv_kernel<KIND, MT, R, true><<<grid, 256, 0, stream>>>(p);
    else gemv_kernel<KIND, MT, R, false><<<grid, 256, 0, stream>>>(p);
}

}  // namespace

hipError_t launch_xprep(const float* x, int M, int64_t K, int kind, Workspace* ws, hipStream_t stream) {
    const int64_t G = (K + kGroup - 1) / kGroup, Kp = G * kGroup;
    const int64_t quads = (G + 3) / 4;
    const int64_t waves = int64_t(M) * quads;
    const unsigned grid = unsigned((waves + 3) / 4);
    const bool vecx = (K % 4 == 0) && (reinterpret_cast<uintptr_t>(x) % 16 == 0);
    if (kind == 1) {
        if (vecx) xprep_kernel<true, true><<<grid, 256, 0, stream>>>(x, M, K, G, Kp, quads, ws->xh, ws->xl, ws->xinv);
        else xprep_kernel<true, false><<<grid, 256, 0, stream>>>(x, M, K, G, Kp, quads, ws->xh, ws->xl, ws->xinv);
    } else {
        if (vecx) xprep_kernel<false, true><<<grid, 256, 0, stream>>>(x, M, K, G, Kp, quads, ws->xh, ws->xl, ws->xinv);
        else xprep_kernel<false, false><<<grid, 256, 0, stream>>>(x, M, K, G, Kp, quads, ws->xh, ws->xl, ws->xinv);
    }
    ws->prep_M = M;
    ws->prep_K = K;
    ws->prep_kind = kind;
    return hipGetLastError();
}

hipError_t launch_gemv_prepped(const QView& W, const uint16_t* bias, int M, float* y, Workspace* ws,
                               hipStream_t stream) {
    const int64_t N = W.rows, K = W.cols, G = W.groups, Kp = G * kGroup;
    constexpr int R = 2;
    GemvParams p;
    p.q = W.q; p.scales = W.scales; p.zeros = W.zeros;
    p.N = N; p.K = K; p.G = G; p.Kp = Kp;
    p.xh = ws->xh; p.xl = ws->xl; p.xinv = ws->xinv;
    p.bias = bias; p.y = y; p.part = ws->partials; p.cnt = ws->counters;
    p.M = M;
    p.nrb = int((N + 16 * R - 1) / (16 * R));
    p.nrb_pad = (p.nrb + kWaves - 1) / kWaves * kWaves;
    const int target = device_cu_count() * 8;
    int S = (target + p.nrb_pad - 1) / p.nrb_pad;
    if (S > G) S = int(G);
    if (S < 1) S = 1;
    while (S > 1 && (int64_t(S) * M * N > kPartialFloats || p.nrb > kMaxCounters)) S--;
    p.gs = int((G + S - 1) / S);
    p.S = int((G + p.gs - 1) / p.gs);
    const unsigned grid = unsigned(int64_t(p.S) * p.nrb_pad / kWaves);
    const bool fast = (K % kGroup == 0);
    if (W.kind == 1) {
        if (M <= 16) launch_gemv_t<1, 1, R>(p, fast, grid, stream);
        else launch_gemv_t<1, 2, R>(p, fast, grid, stream);
    } else {
        if (M <= 16) launch_gemv_t<0, 1, R>(p, fast, grid, stream);
        else launch_gemv_t<0, 2, R>(p, fast, grid, stream);
    }
    return hipGetLastError();
}

hipError_t launch_gemv(const float* x, const QView& W, const uint16_t* bias, int M, float* y,
                       Workspace* ws, hipStream_t stream) {
    hipError_t e = launch_xprep(x, M, W.cols, W.kind, ws, stream);
    if (e != hipSuccess) return e;
    return launch_gemv_prepped(W, bias, M, y, ws, stream);
}

}  // namespace iq

// iq_gemm.hip -- quantised prefill GEMM on gfx950 MFMA (bf16 in, fp32 out).
//
// Replaces gemm_tiled_q_kernel (kernels/ops/quant.cu:254-302, fp32 SIMT
// 64x64 tiles).  y[t,n] = sum_k x[t,k] * dequant(W,n,k) (+ bias[n]).
//
// Tiling: a 256-thread workgroup (4 waves, 2x2) owns a 128 (activation rows)
// x 128 (output features) tile; each wave a 64x64 block = 2x2 MFMA
// f32_32x32x16_bf16 tiles (64-row and 64-column variants for short T and
// narrow matrices; K split over workgroups when the tiles would leave CUs
// idle, the range sums added by a reduction).  K advances 64 columns per step through
// double-buffered LDS: the next step's activation and weight bytes are
// loaded into registers while the current step's MFMAs run, then written to
// the other buffer -- the weights dequantised on the way in (int8 code, or
// int4 q - z, as an exact bf16 integer).  The bf16 scale of each 128-column
// group multiplies the fp32 MFMA partial of that group (acc += s * P_g), so
// the matrix core only ever sees exact integers on the weight side.
// Activations: bf16 as given (iq_gemm_bf16x).  fp32 activations take the
// fp16 operand path below (gemmh_kernel, after one preparation launch) on
// whole 128-column groups; on ragged shapes they are split on the way into
// LDS into three bf16 terms (x = hi + mid + lo to about 2^-24 |x|), three
// MFMAs per step.
// Block order is XCD-aware: consecutive tiles along the activation rows of
// one weight-column block land on the same XCD, so a weight tile is fetched
// from HBM once per XCD and re-read from that XCD's L2.
#include <algorithm>
#include <type_traits>

#include "iq_internal.h"
#include "iq_limbs.h"

namespace iq {

namespace {

constexpr int BK = 64, LDSW = BK + 8;  // LDS row pitch (bf16)
constexpr int kThreads = 256;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

struct GemmParams {
    const float* xf;      // fp32 activations [T][K] or null
    const uint16_t* xb;   // bf16 activations [T][K] or null
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
    const uint16_t* bias;
    float* y;
    int64_t T, N, K, G;
    int tiles_m, tiles_n;
    int splits;      // K ranges (workgroups per output tile); > 1: range sums go to part
    int64_t kchunk;  // columns per K range (a multiple of 128)
    float* part;     // [splits][T][N] fp32
};

__device__ __forceinline__ uint32_t bf16_pair_from_f32(float a, float b) {
    return __builtin_amdgcn_perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
}

// Exact bf16 of a small integer (|v| < 256).
__device__ __forceinline__ uint32_t bf16_pair_int(int a, int b) {
    return bf16_pair_from_f32(float(a), float(b));
}

// NJ: 32-column MFMA tiles per wave along the output features (tile width
// BN = 64 NJ): 2 for wide matrices, 1 when 128-wide tiles would leave CUs idle.
// BM: activation rows per tile, 128, or 64 for short T (each wave 32 rows).
// BM = 256 (bf16 activations): 8 waves (4 x 2), each dequantised weight
// tile in LDS then feeds twice the MFMAs of a 128-row tile.
template <int KIND, bool XF32, bool FASTW, bool FASTX, int NJ, int BM>
__global__ __launch_bounds__(BM == 256 ? 2 * kThreads : kThreads, BM == 256 ? 1 : 2) void gemm_kernel(const GemmParams p) {
    constexpr int BN = 64 * NJ;
    constexpr int NT = BM == 256 ? 2 * kThreads : kThreads;  // threads
    constexpr int WR = NT / 128;                           // waves along the rows
    constexpr int WROWS = BM / WR;                         // rows per wave
    constexpr int NI = WROWS / 32;  // 32-row MFMA tiles per wave along the rows
    __shared__ __attribute__((aligned(16))) uint16_t As[2][BM][LDSW];
    __shared__ __attribute__((aligned(16))) uint16_t Al[XF32 ? 2 : 1][XF32 ? BM : 1][LDSW];
    __shared__ __attribute__((aligned(16))) uint16_t Am[XF32 ? 2 : 1][XF32 ? BM : 1][LDSW];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[2][BN][LDSW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;

    // XCD-aware tile order: workgroup b runs on XCD b % 8; give each XCD a
    // contiguous run of tiles (a bijection on [0, ntiles)).
    const int ntiles = p.tiles_m * p.tiles_n;
    const int split = int(blockIdx.x) / ntiles;  // K range of this workgroup
    const int b = int(blockIdx.x) - split * ntiles;
    const int xcd = b % 8, base = ntiles / 8, extra = ntiles % 8;
    const int t = xcd * base + (xcd < extra ? xcd : extra) + b / 8;
    const int tm = t % p.tiles_m, tn = t / p.tiles_m;
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;

    const int64_t row_bytes = KIND == 1 ? p.K / 2 : p.K;
    // K range [kbeg, kbeg + klen): the sources below are based at kbeg, so
    // the loop runs over klen columns as over a whole row
    const int64_t kbeg = int64_t(split) * p.kchunk;
    const int64_t klen = p.K - kbeg < p.kchunk ? p.K - kbeg : p.kchunk;
    const int64_t gbeg = kbeg / kGroup, glen = (klen + kGroup - 1) / kGroup;
    const int nk = int((klen + BK - 1) / BK);
    const int64_t range_bytes = KIND == 1 ? (klen + 1) / 2 : klen;

    // ---- register staging of one K step
    constexpr int XCH = BM * (XF32 ? BK / 4 : BK / 8) / NT;  // 16-byte activation chunks per thread
    constexpr int WCH0 = BN * (KIND == 1 ? 2 : 4) / NT;       // 16-byte weight chunks per thread
    constexpr int WCH = WCH0 > 0 ? WCH0 : 1;
    struct Regs {
        uint4 xr[XCH];
        uint4 wr[WCH];
        uint32_t zr[WCH];  // int4: the zero point of each weight chunk's row
    };
    Regs r0, r1;

    // Per-thread source rows, fixed for the whole K loop (a step adds its
    // column offset): the fast paths need no per-step bounds arithmetic.
    const uint8_t* wrow[WCH];
    const uint8_t* zrow[WCH];
    bool wok[WCH];
    int wcol[WCH];
#pragma unroll
    for (int i = 0; i < WCH; i++) {
        const int c = tid + NT * i;
        const int row = KIND == 1 ? c >> 1 : c >> 2;
        const int64_t n = n0 + row;
        wok[i] = row < BN && n < p.N;
        wrow[i] = p.q + (wok[i] ? n : 0) * row_bytes + (KIND == 1 ? kbeg / 2 : kbeg);
        wcol[i] = KIND == 1 ? (c & 1) * 16 : (c & 3) * 16;  // byte offset inside the step
        zrow[i] = KIND == 1 ? p.zeros + (wok[i] ? n : 0) * p.G + gbeg : nullptr;
    }
    const void* xrow[XCH];
    bool xok[XCH];
    int xcol[XCH];
#pragma unroll
    for (int i = 0; i < XCH; i++) {
        const int c = tid + NT * i;
        const int row = XF32 ? c >> 4 : c >> 3;
        const int64_t m = m0 + row;
        xok[i] = m < p.T;
        xrow[i] = XF32 ? static_cast<const void*>(p.xf + (xok[i] ? m : 0) * p.K + kbeg)
                       : static_cast<const void*>(p.xb + (xok[i] ? m : 0) * p.K + kbeg);
        xcol[i] = XF32 ? (c & 15) * 4 : (c & 7) * 8;  // element offset inside the step
    }
    // Fast paths: buffer resources over this tile's rows (wave-uniform), so
    // every global load of the K loop is unconditional (rows past T or N and
    // groups past the range read zero without a memory access).  A load
    // under a branch makes the compiler wait for all outstanding loads
    // before the next use of any of them, which would serialise the
    // two-steps-ahead pipeline.
    constexpr int XE = XF32 ? 4 : 2;
    const int64_t xrows = p.T - m0 < BM ? p.T - m0 : BM;
    const int64_t nrows = p.N - n0 < BN ? p.N - n0 : BN;
    const rsrc_t rx = make_rsrc(XF32 ? static_cast<const void*>(p.xf + m0 * p.K)
                                     : static_cast<const void*>(p.xb + m0 * p.K), xrows * p.K * XE);
    const rsrc_t rw = make_rsrc(p.q + n0 * row_bytes, nrows * row_bytes);
    const rsrc_t rsc = make_rsrc(p.scales + n0 * p.G, nrows * p.G * 2);
    const rsrc_t rzp = make_rsrc(KIND == 1 ? p.zeros + n0 * p.G : nullptr, KIND == 1 ? nrows * p.G : 0);
    uint32_t xoff[XCH], woff[WCH], zoff[WCH];
#pragma unroll
    for (int i = 0; i < XCH; i++) {
        const int c = tid + NT * i;
        const int row = XF32 ? c >> 4 : c >> 3;
        xoff[i] = uint32_t((int64_t(row) * p.K + kbeg + xcol[i]) * XE);
    }
#pragma unroll
    for (int i = 0; i < WCH; i++) {
        const int c = tid + NT * i;
        const int row = KIND == 1 ? c >> 1 : c >> 2;
        woff[i] = wok[i] ? uint32_t(row * row_bytes + (KIND == 1 ? kbeg / 2 : kbeg) + wcol[i]) : kOob;
        zoff[i] = (KIND == 1 && wok[i]) ? uint32_t(row * p.G + gbeg) : kOob;
    }

    auto load_step = [&](Regs& rg, int kt) {
        uint4* xr = rg.xr;
        uint4* wr = rg.wr;
        uint32_t* zr = rg.zr;
        const int64_t k0 = int64_t(kt) * BK;
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int64_t k = k0 + xcol[i];
            if (FASTX) {
                xr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, xoff[i] + uint32_t(k0 * XE), 0, 0));
            } else if (XF32) {
                const float* xp = static_cast<const float*>(xrow[i]);
                float f[4];
#pragma unroll
                for (int e = 0; e < 4; e++) f[e] = (xok[i] && k + e < klen) ? xp[k + e] : 0.0f;
                xr[i] = make_uint4(__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3]));
            } else {
                const uint16_t* xp = static_cast<const uint16_t*>(xrow[i]);
                uint32_t h[4] = {0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 8; e++)
                    if (xok[i] && k + e < klen) h[e / 2] |= uint32_t(xp[k + e]) << (16 * (e & 1));
                xr[i] = make_uint4(h[0], h[1], h[2], h[3]);
            }
        }
#pragma unroll
        for (int i = 0; i < WCH; i++) {
            const int64_t off = (KIND == 1 ? k0 / 2 : k0) + wcol[i];
            if (FASTW) {
                wr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      rw, woff[i] + uint32_t(KIND == 1 ? k0 / 2 : k0), 0, 0));
            } else if (!wok[i]) {
                wr[i] = make_uint4(0, 0, 0, 0);
            } else {
                uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
                for (int e = 0; e < 16; e++)
                    if (off + e < range_bytes) w[e / 4] |= uint32_t(wrow[i][off + e]) << (8 * (e % 4));
                wr[i] = make_uint4(w[0], w[1], w[2], w[3]);
            }
        }
#pragma unroll
        for (int i = 0; i < WCH; i++) {
            if (KIND == 1 && FASTW) zr[i] = __builtin_amdgcn_raw_buffer_load_b8(rzp, zoff[i] + uint32_t(k0 / kGroup), 0, 0);
            else zr[i] = (KIND == 1 && wok[i]) ? zrow[i][k0 / kGroup] : 0u;
        }
    };

    auto store_step = [&](const Regs& rg, int buf) {
        const uint4* xr = rg.xr;
        const uint4* wr = rg.wr;
        const uint32_t* zr = rg.zr;
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + NT * i;
            if (XF32) {
                const int row = c >> 4, kc = c & 15;
                const float f[4] = {__uint_as_float(xr[i].x), __uint_as_float(xr[i].y),
                                    __uint_as_float(xr[i].z), __uint_as_float(xr[i].w)};
                // hi = bf16(x), mid = bf16(x - hi), lo = bf16(x - hi - mid),
                // each rounded to nearest even by the hardware conversion
                // (both differences are exact in fp32): x = hi + mid + lo
                // to about 2^-24 |x|
                uint32_t hi[2], mi[2], lo[2];
#pragma unroll
                for (int e = 0; e < 2; e++) {
                    const bf16x2_t h = {__bf16(f[2 * e]), __bf16(f[2 * e + 1])};
                    const float r0 = f[2 * e] - float(h[0]), r1 = f[2 * e + 1] - float(h[1]);
                    const bf16x2_t md = {__bf16(r0), __bf16(r1)};
                    const bf16x2_t l = {__bf16(r0 - float(md[0])), __bf16(r1 - float(md[1]))};
                    hi[e] = __builtin_bit_cast(uint32_t, h);
                    mi[e] = __builtin_bit_cast(uint32_t, md);
                    lo[e] = __builtin_bit_cast(uint32_t, l);
                }
                *reinterpret_cast<uint2*>(&As[buf][row][kc * 4]) = make_uint2(hi[0], hi[1]);
                *reinterpret_cast<uint2*>(&Am[XF32 ? buf : 0][XF32 ? row : 0][kc * 4]) = make_uint2(mi[0], mi[1]);
                *reinterpret_cast<uint2*>(&Al[XF32 ? buf : 0][XF32 ? row : 0][kc * 4]) = make_uint2(lo[0], lo[1]);
            } else {
                const int row = c >> 3, kc = c & 7;
                *reinterpret_cast<uint4*>(&As[buf][row][kc * 8]) = xr[i];
            }
        }
#pragma unroll
        for (int i = 0; i < WCH; i++) {
            const int c = tid + NT * i;
            const uint32_t d[4] = {wr[i].x, wr[i].y, wr[i].z, wr[i].w};
            // (int4 at BN = 64 or 512 threads: half the threads have no chunk;
            // the test is compiled only there, a divergent branch around the
            // conversion would make every step wait for all its loads)
            if constexpr (WCH0 * NT < BN * (KIND == 1 ? 2 : 4) || WCH0 == 0)
                if ((KIND == 1 ? c >> 1 : c >> 2) >= BN) continue;
            if (KIND == 1) {
                const int row = c >> 1, kc = c & 1;
                const int z = int(zr[i]);
                uint32_t o[16];
#pragma unroll
                for (int j = 0; j < 4; j++) {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const uint32_t byte = (d[j] >> (8 * e)) & 0xFF;
                        o[j * 4 + e] = bf16_pair_int(int(byte & 0xF) - z, int(byte >> 4) - z);
                    }
                }
                uint4* dst = reinterpret_cast<uint4*>(&Bs[buf][row][kc * 32]);
                dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
                dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
                dst[2] = make_uint4(o[8], o[9], o[10], o[11]);
                dst[3] = make_uint4(o[12], o[13], o[14], o[15]);
            } else {
                const int row = c >> 2, kc = c & 3;
                uint32_t o[8];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int8_t b0 = int8_t(d[j] & 0xFF), b1 = int8_t((d[j] >> 8) & 0xFF);
                    const int8_t b2 = int8_t((d[j] >> 16) & 0xFF), b3 = int8_t(d[j] >> 24);
                    o[2 * j] = bf16_pair_int(b0, b1);
                    o[2 * j + 1] = bf16_pair_int(b2, b3);
                }
                uint4* dst = reinterpret_cast<uint4*>(&Bs[buf][row][kc * 16]);
                dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
                dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
            }
        }
    };

    float16_t acc[NI][NJ], P[NI][NJ];
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) { acc[i][j][r] = 0.0f; P[i][j][r] = 0.0f; }

    // Scale row pointers of this lane's two output columns.
    int64_t ncol[NJ];
    bool nval[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        ncol[j] = n0 + wn * (32 * NJ) + j * 32 + (lane & 31);
        nval[j] = ncol[j] < p.N;
    }

    // Scales of this lane's two output columns: group g's are requested a
    // group ahead (a load waited on at the group's close would stall every
    // second step).
    // (buffer loads: no branch around them, see above)
    uint32_t soff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) soff[j] = uint32_t(((ncol[j] - n0) * p.G + gbeg) * 2);
    // (the raw bf16 bits are kept until the group closes: converting right
    // after the request would wait for it there)
    auto load_scales = [&](int64_t g, uint16_t (&s)[NJ]) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t off = (nval[j] && g < glen) ? soff[j] + uint32_t(g * 2) : kOob;
            s[j] = __builtin_amdgcn_raw_buffer_load_b16(rsc, off, 0, 0);
        }
    };
    uint16_t s_cur[NJ], s_nxt[NJ];  // raw bf16 bits (no ALU op on a load until it is used)
    load_scales(0, s_cur);
    load_scales(1, s_nxt);

    // Pipeline: while step kt is multiplied from LDS buffer kt & 1, the
    // registers of one set hold step kt + 1 (stored into the other buffer
    // after the MFMAs) and those of the other set step kt + 2 (requested one
    // step earlier), so global loads have two steps to arrive.
    load_step(r0, 0);
    store_step(r0, 0);
    if (nk > 1) load_step(r1, 1);
    if (nk > 2) load_step(r0, 2);
    __syncthreads();
    // PAR = kt & 1, fixed at compile time (the loop below alternates).
    auto step = [&](auto par, int kt, Regs& rnext, Regs& rlater) {
        constexpr int PAR = decltype(par)::value;
        const int buf = PAR;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            const int kof = ks * 16 + 8 * (lane >> 5);
            bf16x8_t a[NI], am[NI], al[NI], bw[NJ];
#pragma unroll
            for (int i = 0; i < NI; i++) {
                a[i] = *reinterpret_cast<const bf16x8_t*>(&As[buf][wm * WROWS + i * 32 + (lane & 31)][kof]);
                if (XF32) {
                    am[i] = *reinterpret_cast<const bf16x8_t*>(&Am[XF32 ? buf : 0][XF32 ? wm * WROWS + i * 32 + (lane & 31) : 0][kof]);
                    al[i] = *reinterpret_cast<const bf16x8_t*>(&Al[XF32 ? buf : 0][XF32 ? wm * WROWS + i * 32 + (lane & 31) : 0][kof]);
                }
            }
#pragma unroll
            for (int j = 0; j < NJ; j++)
                bw[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[buf][wn * (32 * NJ) + j * 32 + (lane & 31)][kof]);
            // the group's first k slice starts its partial sums from zero
            const bool first = PAR == 0 && ks == 0;
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    P[i][j] = mfma32_bf16(a[i], bw[j], first ? float16_t{} : P[i][j]);
                    if (XF32) {
                        P[i][j] = mfma32_bf16(am[i], bw[j], P[i][j]);
                        P[i][j] = mfma32_bf16(al[i], bw[j], P[i][j]);
                    }
                }
        }
        // Close the 128-column group after its second 64-column step (or at the end).
        if (PAR == 1 || kt + 1 == nk) {
#pragma unroll
            for (int j = 0; j < NJ; j++) {
#pragma unroll
                for (int i = 0; i < NI; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        acc[i][j][r] = __builtin_fmaf(__uint_as_float(uint32_t(s_cur[j]) << 16), P[i][j][r], acc[i][j][r]);
                s_cur[j] = s_nxt[j];
            }
            load_scales(kt / 2 + 2, s_nxt);
        }
        if (kt + 1 < nk) store_step(rnext, buf ^ 1);
        if (kt + 3 < nk) load_step(rnext, kt + 3);
        __syncthreads();
        (void)rlater;
    };
    for (int kt = 0; kt < nk; kt += 2) {
        step(std::integral_constant<int, 0>{}, kt, r1, r0);
        if (kt + 1 < nk) step(std::integral_constant<int, 1>{}, kt + 1, r0, r1);
    }

    // Epilogue: lane holds rows m = 8*(r/4) + 4*(lane/32) + r%4 of each 32x32 tile.
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        if (!nval[j]) continue;
        const float bv = p.bias && p.splits == 1 ? bf16_to_f32(p.bias[ncol[j]]) : 0.0f;
        float* dst = p.splits == 1 ? p.y : p.part + int64_t(split) * p.T * p.N;
#pragma unroll
        for (int i = 0; i < NI; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + wm * WROWS + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                if (m < p.T) dst[m * p.N + ncol[j]] = acc[i][j][r] + bv;
            }
    }
}

// ------------------------------------------------------------------ fp16 operand path
// The activations are prepared once per call into fp16 MFMA operands:
// per activation row m, 2^e_m with max_k |x[m,k]| 2^e_m in [2^14, 2^15),
// hi = f16(x 2^e_m) (round to nearest even) and, for fp32 activations,
// lo = f16(x 2^e_m - hi) (the difference is exact in fp32), so x 2^e_m =
// hi + lo to about 2^-22 of |x| (values below 2^-28 of the row's largest
// fall into fp16's subnormal range, which keeps them to 2^-39 of it).  The
// preparation kernel also takes bf16 rows (XF32 = false: hi alone is then
// exact down to the same range); the library uses it for fp32 activations,
// bf16 ones go to gemm_kernel as they are.  The weights enter as
// the exact integers q or q - z through the fp16 exponent-bias constants
// (dq_int8_x4 / dq_int4_x8: about one VALU op per code, against four for a
// bf16 conversion), and each output is scaled back by 2^-e_m at the end
// (exact).  For int4 weights the prepared columns of every octet are stored
// in the order dq_int4_x8 leaves the nibbles (slot i = column perm8(i)), so
// both operands agree on the column order of every MFMA k slot.
// Non-finite activations make their row's outputs NaN.
struct GemmhParams {
    const _Float16* ah;  // [T][K] prepared hi
    const _Float16* al;  // [T][K] prepared lo (fp32 activations) or null
    const float* rs;     // [T] 2^-e_m (NaN: the row holds a non-finite value)
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
    const uint16_t* bias;
    float* y;
    int64_t T, N, K, G;
    int tiles_m, tiles_n;
    int splits;
    int64_t kchunk;
    float* part;
};

// The fp16 hi + lo operands of fp32 activations, 2^e per row: one row
// over `seg` workgroups (grid T x seg).  Each workgroup takes the row's
// largest |x| (and whether anything is non-finite) over the whole row, then
// converts its segment of the row's 8-value chunks.  Both passes request
// four 32-byte chunks per thread at a time through a buffer resource over
// the row (chunks past the end read zero), so a long row costs a few
// memory latencies, not one per chunk.  RES (rows of at most 8 chunks per
// thread, seg = 1): every chunk is requested once, kept in registers
// through the reduction and converted from there (one memory latency).
template <bool PERM, bool LO, bool RES>
__global__ __launch_bounds__(512) void gemm_xprep_kernel(const float* __restrict__ xf, int64_t K, int seg,
                                                         _Float16* __restrict__ ah, _Float16* __restrict__ al,
                                                         float* __restrict__ rs) {
    constexpr int NT = 512, U = 4;
    const int64_t m = blockIdx.x / seg;
    const int s = int(blockIdx.x % seg);
    const int tid = threadIdx.x;
    __shared__ uint32_t red[2][NT / 64];
    const rsrc_t rx = make_rsrc(xf + m * K, K * 4);
    const int64_t nch = K / 8;
    auto load8 = [&](int64_t ch, float (&v)[8]) {
        const uint32_t off = ch < nch ? uint32_t(ch * 32) : kOob;
        const float4_t a = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0));
        const float4_t b = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rx, off, 16, 0));
#pragma unroll
        for (int e = 0; e < 4; e++) {
            v[e] = a[e];
            v[4 + e] = b[e];
        }
    };
    // 1. largest |x| (as bits: order-preserving for non-negative floats) and
    //    whether anything is non-finite
    uint32_t am = 0, nf = 0;
    constexpr int NR = RES ? 8 : 1;
    float vr[NR][8];
    if constexpr (RES) {
#pragma unroll
        for (int j = 0; j < NR; j++) load8(tid + j * NT, vr[j]);
#pragma unroll
        for (int j = 0; j < NR; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t a = __float_as_uint(vr[j][e]) & 0x7FFFFFFFu;
                nf |= a >= 0x7F800000u ? 1u : 0u;
                am = a > am ? a : am;
            }
    }
    for (int64_t c0 = tid; !RES && c0 < nch; c0 += U * NT) {
        float v[U][8];
#pragma unroll
        for (int j = 0; j < U; j++) load8(c0 + j * NT, v[j]);
#pragma unroll
        for (int j = 0; j < U; j++)
#pragma unroll
            for (int e = 0; e < 8; e++) {
                const uint32_t a = __float_as_uint(v[j][e]) & 0x7FFFFFFFu;
                nf |= a >= 0x7F800000u ? 1u : 0u;
                am = a > am ? a : am;
            }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint32_t o = __shfl_xor(am, off), f = __shfl_xor(nf, off);
        am = o > am ? o : am;
        nf |= f;
    }
    if ((tid & 63) == 0) {
        red[0][tid >> 6] = am;
        red[1][tid >> 6] = nf;
    }
    __syncthreads();
    am = red[0][0];
    nf = red[1][0];
#pragma unroll
    for (int w = 1; w < NT / 64; w++) {
        am = red[0][w] > am ? red[0][w] : am;
        nf |= red[1][w];
    }
    // amax = f 2^E, f in [0.5, 1): e = 15 - E; kept within [-126, 126] so
    // that 2^-e is a normal float
    int e = (am > 0 && !nf) ? 15 - __builtin_amdgcn_frexp_expf(__uint_as_float(am)) : 0;
    e = e > 126 ? 126 : (e < -126 ? -126 : e);
    if (s == 0 && tid == 0) rs[m] = nf ? __builtin_nanf("") : __builtin_amdgcn_ldexpf(1.0f, -e);
    auto store8 = [&](int64_t ch, const float (&v)[8]) {
        half8_t h, l;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = PERM ? perm8(i) : i;
            const float sv = __builtin_amdgcn_ldexpf(v[c], e);
            h[i] = _Float16(sv);
            l[i] = _Float16(sv - float(h[i]));
        }
        *reinterpret_cast<half8_t*>(ah + m * K + ch * 8) = h;
        if (LO) *reinterpret_cast<half8_t*>(al + m * K + ch * 8) = l;
    };
    if constexpr (RES) {
#pragma unroll
        for (int j = 0; j < NR; j++)
            if (tid + j * NT < nch) store8(tid + j * NT, vr[j]);
        return;
    }
    // 2. this workgroup's chunks [cb, ce) of the row
    const int64_t cps = (nch + seg - 1) / seg, cb = s * cps, ce = cb + cps < nch ? cb + cps : nch;
    for (int64_t c0 = cb + tid; c0 < ce; c0 += U * NT) {
        float v[U][8];
#pragma unroll
        for (int j = 0; j < U; j++) load8(c0 + j * NT < ce ? c0 + j * NT : nch, v[j]);
#pragma unroll
        for (int j = 0; j < U; j++) {
            const int64_t ch = c0 + j * NT;
            if (ch >= ce) break;
            store8(ch, v[j]);
        }
    }
}

// Same tiling as gemm_kernel (waves 2 along the columns, BM / (NT / 128)
// rows each; 32x32 MFMA tiles; 64-column K steps double-buffered in LDS with
// the step after next in registers), on the prepared fp16 operands (LO: hi
// and lo, two MFMAs per weight operand).  K % 128 == 0.
// NR: K steps whose loads are in flight in registers (2, or 4 for short
// T, where each workgroup's steps wait on memory rather than on the MFMAs,
// and for int8 on 128-row tiles)
template <int KIND, bool LO, int NJ, int BM, int NR = 2>
__global__ __launch_bounds__(BM >= 128 ? 2 * kThreads : kThreads, (BM == 256 || LO) ? 1 : 2) void gemmh_kernel(
    const GemmhParams p) {
    constexpr int BN = 64 * NJ;
    constexpr int NT = BM >= 128 ? 2 * kThreads : kThreads;
    constexpr int WR = NT / 128;
    constexpr int WROWS = BM / WR;
    constexpr int NI = WROWS / 32;
    __shared__ __attribute__((aligned(16))) _Float16 As[2][BM][LDSW];
    __shared__ __attribute__((aligned(16))) _Float16 Al[LO ? 2 : 1][LO ? BM : 1][LDSW];
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN][LDSW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int ntiles = p.tiles_m * p.tiles_n;
    const int split = int(blockIdx.x) / ntiles;
    const int b = int(blockIdx.x) - split * ntiles;
    const int xcd = b % 8, base = ntiles / 8, extra = ntiles % 8;
    const int t = xcd * base + (xcd < extra ? xcd : extra) + b / 8;
    const int tm = t % p.tiles_m, tn = t / p.tiles_m;
    const int64_t m0 = int64_t(tm) * BM, n0 = int64_t(tn) * BN;

    const int64_t row_bytes = KIND == 1 ? p.K / 2 : p.K;
    const int64_t kbeg = int64_t(split) * p.kchunk;
    const int64_t klen = p.K - kbeg < p.kchunk ? p.K - kbeg : p.kchunk;
    const int64_t gbeg = kbeg / kGroup, glen = klen / kGroup;
    const int nk = int(klen / BK);

    constexpr int XCH = BM * (BK / 8) / NT;              // 16-byte activation chunks per thread
    constexpr int WCH0 = BN * (KIND == 1 ? 2 : 4) / NT;  // 16-byte weight chunks per thread
    constexpr int WCH = WCH0 > 0 ? WCH0 : 1;
    struct Regs {
        uint4 xr[XCH];
        uint4 xl[LO ? XCH : 1];
        uint4 wr[WCH];
        uint32_t zr;
    };
    Regs rr[NR];

    bool wok[WCH];
    int wcol[WCH];
#pragma unroll
    for (int i = 0; i < WCH; i++) {
        const int c = tid + NT * i;
        const int row = KIND == 1 ? c >> 1 : c >> 2;
        wok[i] = row < BN && n0 + row < p.N;
        wcol[i] = KIND == 1 ? (c & 1) * 16 : (c & 3) * 16;
    }
    // buffer resources over this tile's rows: every load of the K loop is
    // unconditional (out-of-range rows read zero), so the waits before a
    // step's use cover only that step's requests
    const int64_t xrows = p.T - m0 < BM ? p.T - m0 : BM;
    const int64_t nrows = p.N - n0 < BN ? p.N - n0 : BN;
    const rsrc_t rah = make_rsrc(p.ah + m0 * p.K, xrows * p.K * 2);
    const rsrc_t ral = make_rsrc(LO ? p.al + m0 * p.K : nullptr, LO ? xrows * p.K * 2 : 0);
    const rsrc_t rw = make_rsrc(p.q + n0 * row_bytes, nrows * row_bytes);
    const rsrc_t rsc = make_rsrc(p.scales + n0 * p.G, nrows * p.G * 2);
    const rsrc_t rzp = make_rsrc(KIND == 1 ? p.zeros + n0 * p.G : nullptr, KIND == 1 ? nrows * p.G : 0);
    uint32_t xoff[XCH], woff[WCH], zoff = kOob;
#pragma unroll
    for (int i = 0; i < XCH; i++) {
        const int c = tid + NT * i;
        xoff[i] = uint32_t((int64_t(c >> 3) * p.K + kbeg + (c & 7) * 8) * 2);
    }
#pragma unroll
    for (int i = 0; i < WCH; i++) {
        const int c = tid + NT * i;
        const int row = KIND == 1 ? c >> 1 : c >> 2;
        woff[i] = wok[i] ? uint32_t(row * row_bytes + (KIND == 1 ? kbeg / 2 : kbeg) + wcol[i]) : kOob;
        if (KIND == 1 && i == 0) zoff = wok[0] ? uint32_t(row * p.G + gbeg) : kOob;
    }
    auto load_step = [&](Regs& rg, int kt) {
        const uint32_t k0 = uint32_t(kt) * BK;
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            rg.xr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rah, xoff[i] + k0 * 2, 0, 0));
            if (LO) rg.xl[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(ral, xoff[i] + k0 * 2, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < WCH; i++)
            rg.wr[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     rw, woff[i] + (KIND == 1 ? k0 / 2 : k0), 0, 0));
        rg.zr = KIND == 1 ? __builtin_amdgcn_raw_buffer_load_b8(rzp, zoff + k0 / kGroup, 0, 0) : 0u;
    };

    auto store_step = [&](const Regs& rg, int buf) {
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + NT * i;
            *reinterpret_cast<uint4*>(&As[buf][c >> 3][(c & 7) * 8]) = rg.xr[i];
            if (LO) *reinterpret_cast<uint4*>(&Al[LO ? buf : 0][LO ? c >> 3 : 0][(c & 7) * 8]) = rg.xl[i];
        }
#pragma unroll
        for (int i = 0; i < WCH; i++) {
            const int c = tid + NT * i;
            if constexpr (WCH0 == 0)  // int4 with fewer chunks than threads
                if ((KIND == 1 ? c >> 1 : c >> 2) >= BN) continue;
            const uint32_t d[4] = {rg.wr[i].x, rg.wr[i].y, rg.wr[i].z, rg.wr[i].w};
            if (KIND == 1) {
                const int row = c >> 1, kc = c & 1;
                const uint32_t zb = zpair_1024(rg.zr), zc = zpair_64(rg.zr);
                uint4* dst = reinterpret_cast<uint4*>(&Bs[buf][row][kc * 32]);
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    uint32_t o0, o1, o2, o3;
                    dq_int4_x8(d[j], zb, zc, o0, o1, o2, o3);
                    dst[j] = make_uint4(o0, o1, o2, o3);
                }
            } else {
                const int row = c >> 2, kc = c & 3;
                uint32_t o[8];
#pragma unroll
                for (int j = 0; j < 4; j++) dq_int8_x4(d[j], o[2 * j], o[2 * j + 1]);
                uint4* dst = reinterpret_cast<uint4*>(&Bs[buf][row][kc * 16]);
                dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
                dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
            }
        }
    };

    float16_t acc[NI][NJ], P[NI][NJ];
#pragma unroll
    for (int i = 0; i < NI; i++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) { acc[i][j][r] = 0.0f; P[i][j][r] = 0.0f; }

    int64_t ncol[NJ];
    bool nval[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        ncol[j] = n0 + wn * (32 * NJ) + j * 32 + (lane & 31);
        nval[j] = ncol[j] < p.N;
    }
    uint32_t soff[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) soff[j] = uint32_t(((ncol[j] - n0) * p.G + gbeg) * 2);
    auto load_scales = [&](int64_t g, uint16_t (&sc)[NJ]) {
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const uint32_t off = (nval[j] && g < glen) ? soff[j] + uint32_t(g * 2) : kOob;
            sc[j] = __builtin_amdgcn_raw_buffer_load_b16(rsc, off, 0, 0);
        }
    };
    uint16_t s_cur[NJ], s_nxt[NJ];  // raw bf16 bits (no ALU op on a load until it is used)
    load_scales(0, s_cur);
    load_scales(1, s_nxt);

    load_step(rr[0], 0);
    store_step(rr[0], 0);
#pragma unroll
    for (int j = 1; j <= NR; j++)
        if (nk > j) load_step(rr[j % NR], j);
    __syncthreads();
    auto step = [&](auto par, int kt, Regs& rnext) {
        constexpr int PAR = decltype(par)::value;
        const int buf = PAR;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ks++) {
            const int kof = ks * 16 + 8 * (lane >> 5);
            half8_t a[NI], al[NI], bw[NJ];
#pragma unroll
            for (int i = 0; i < NI; i++) {
                a[i] = *reinterpret_cast<const half8_t*>(&As[buf][wm * WROWS + i * 32 + (lane & 31)][kof]);
                if (LO)
                    al[i] = *reinterpret_cast<const half8_t*>(
                        &Al[LO ? buf : 0][LO ? wm * WROWS + i * 32 + (lane & 31) : 0][kof]);
            }
#pragma unroll
            for (int j = 0; j < NJ; j++)
                bw[j] = *reinterpret_cast<const half8_t*>(&Bs[buf][wn * (32 * NJ) + j * 32 + (lane & 31)][kof]);
            const bool first = PAR == 0 && ks == 0;
#pragma unroll
            for (int i = 0; i < NI; i++)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
                    P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[i], bw[j], first ? float16_t{} : P[i][j], 0, 0, 0);
                    if (LO) P[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i], bw[j], P[i][j], 0, 0, 0);
                }
        }
        if (PAR == 1) {
#pragma unroll
            for (int j = 0; j < NJ; j++) {
#pragma unroll
                for (int i = 0; i < NI; i++)
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        acc[i][j][r] = __builtin_fmaf(__uint_as_float(uint32_t(s_cur[j]) << 16), P[i][j][r], acc[i][j][r]);
                s_cur[j] = s_nxt[j];
            }
            load_scales(kt / 2 + 2, s_nxt);
        }
        if (kt + 1 < nk) store_step(rnext, buf ^ 1);
        if (kt + 1 + NR < nk) load_step(rnext, kt + 1 + NR);
        __syncthreads();
    };
    // nk is even (K ranges are whole 128-column groups); register set
    // (kt + 1) % NR holds step kt + 1 while step kt runs
    for (int kt = 0; kt < nk; kt += NR) {
        step(std::integral_constant<int, 0>{}, kt, rr[1 % NR]);
        step(std::integral_constant<int, 1>{}, kt + 1, rr[2 % NR]);
        if constexpr (NR == 4) {
            if (kt + 2 < nk) {
                step(std::integral_constant<int, 0>{}, kt + 2, rr[3]);
                step(std::integral_constant<int, 1>{}, kt + 3, rr[0]);
            }
        }
    }

    // Epilogue: lane holds rows m = 8*(r/4) + 4*(lane/32) + r%4 of each 32x32 tile.
#pragma unroll
    for (int i = 0; i < NI; i++) {
        float rsc[16];
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int64_t m = m0 + wm * WROWS + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
            rsc[r] = m < p.T ? p.rs[m] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (!nval[j]) continue;
            const float bv = p.bias && p.splits == 1 ? bf16_to_f32(p.bias[ncol[j]]) : 0.0f;
            float* dst = p.splits == 1 ? p.y : p.part + int64_t(split) * p.T * p.N;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int64_t m = m0 + wm * WROWS + i * 32 + 8 * (r / 4) + 4 * (lane >> 5) + (r % 4);
                if (m < p.T) dst[m * p.N + ncol[j]] = acc[i][j][r] * rsc[r] + bv;
            }
        }
    }
}

// y[t, n] = sum over K ranges s of part[s][t][n] (in range order) + bias[n].
__global__ __launch_bounds__(256) void gemm_reduce_kernel(const float* __restrict__ part, int S, int64_t T,
                                                          int64_t N, const uint16_t* __restrict__ bias,
                                                          float* __restrict__ y) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= T * N) return;
    const float sum = sum_slices(part, S, T * N, i);
    y[i] = sum + (bias ? bf16_to_f32(bias[i % N]) : 0.0f);
}

// The same, four consecutive outputs per thread (N % 4 == 0: they share a
// row; y 16-byte aligned): one 16-byte load per range, the ranges added in
// the same order, so the sums are gemm_reduce_kernel's bit for bit (7B gate
// at T = 256: 117.6 -> 113.9 us with fp32, 83.9 -> 80.6 with bf16
// activations; where the partial sums are small, no change).
__global__ __launch_bounds__(256) void gemm_reduce4_kernel(const float* __restrict__ part, int S, int64_t T,
                                                           int64_t N, const uint16_t* __restrict__ bias,
                                                           float* __restrict__ y) {
    const int64_t i = (int64_t(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i >= T * N) return;
    const int64_t stride = T * N;
    const rsrc_t r = make_rsrc(part, int64_t(S) * stride * 4);
    float4_t sum = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < S; s0 += 8) {
        float4_t v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const uint32_t off = s0 + j < S ? uint32_t((int64_t(s0 + j) * stride + i) * 4) : kOob;
            v[j] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
            if (s0 + j < S) sum += v[j];
    }
    const int64_t n = i % N;
    float4_t o;
#pragma unroll
    for (int e = 0; e < 4; e++) o[e] = sum[e] + (bias ? bf16_to_f32(bias[n + e]) : 0.0f);
    *reinterpret_cast<float4_t*>(y + i) = o;
}

template <int KIND, bool XF32, int NJ>
void launch_gemm_t(const GemmParams& p, bool fastw, bool fastx, int bm, hipStream_t stream) {
    const unsigned grid = unsigned(p.tiles_m * p.tiles_n * p.splits);
    if constexpr (!XF32) {
        if (bm == 256) {  // (fast paths only)
            gemm_kernel<KIND, XF32, true, true, NJ, 256><<<grid, 2 * kThreads, 0, stream>>>(p);
            return;
        }
    }
    if (bm == 64) gemm_kernel<KIND, XF32, true, true, NJ, 64><<<grid, kThreads, 0, stream>>>(p);  // (fast paths only)
    else if (fastw && fastx) gemm_kernel<KIND, XF32, true, true, NJ, 128><<<grid, kThreads, 0, stream>>>(p);
    else if (fastw) gemm_kernel<KIND, XF32, true, false, NJ, 128><<<grid, kThreads, 0, stream>>>(p);
    else if (fastx) gemm_kernel<KIND, XF32, false, true, NJ, 128><<<grid, kThreads, 0, stream>>>(p);
    else gemm_kernel<KIND, XF32, false, false, NJ, 128><<<grid, kThreads, 0, stream>>>(p);
}

// Few output tiles (short T): split K into ranges of whole 128-column groups
// so that the tiles x ranges fill the workgroup slots of the CUs (per_cu
// resident workgroups of the instance per CU) in one round, the range sums
// added by gemm_reduce_kernel; needs the fast (aligned) paths and room for
// the sums.  Rounding the range count down rather than up keeps a second,
// mostly idle round of workgroups off the critical path (7B down 3584 x
// 18944 at T = 80 / 200, fp32 activations: 76.8 / 140.6 -> 60.7 / 111.0
// us; bf16 activations 50.1 / 94.9 -> 36.6 / 69.4 us; 7B gate 18944 x 3584
// with bf16 activations at T = 17..48, on the three-term kernel's one
// workgroup per CU: 29.5..32.6 -> 24.1..27.0 us).  The exception: tiles
// that fill only half to two thirds of one round, on rows of at least 24
// groups, take 3 ranges (two full rounds of shorter workgroups; 7B gate at
// T = 65 / 96 / 128, int8, fp32 activations 78.0 / 72.9 / 73.3 -> 66.4 /
// 64.9 / 68.7 us, bf16 activations 49.6 / 49.7 / 50.2 -> 41.8 / 43.8 /
// 46.5 us, int4 8-16 % faster; 1.5B gate 8960 x 1536, 12 groups, at T =
// 256 lost 38.2 -> 44.5 us), and so do tiles that fill one round up to 2.5
// rounds (7B gate at T = 256, int8 / int4: fp32 activations 125.9 / 119.8
// -> 116.3 / 107.5 us, bf16 84.9 / 95.9 -> 81.8 / 88.9 us; wider ones
// overrun the partial sums).  part_floats: the workspace's partial-sum
// capacity.
int pick_splits(int tiles, int slots, int64_t G, int64_t T, int64_t N, int64_t part_floats) {
    if (G < 2) return 1;
    if (tiles >= slots) {
        if (2 * tiles < 5 * slots && G >= 24 && 3 * T * N <= part_floats) return 3;
        return 1;
    }
    int S = slots / tiles;
    S = S > 16 ? 16 : S;
    while (S > 1 && int64_t(S) * T * N > part_floats) S--;
    if (S == 1 && 3 * tiles <= 2 * slots && G >= 24 && 3 * T * N <= part_floats) S = 3;
    return S;
}

void plan_splits(GemmParams& p, bool fast, int64_t part_floats, int per_cu) {
    p.splits = 1;
    p.kchunk = p.K;
    const int tiles = p.tiles_m * p.tiles_n, want = per_cu * device_cu_count();
    if (!fast || !p.part) return;
    const int64_t G = p.K / kGroup;
    const int S = pick_splits(tiles, want, G, p.T, p.N, part_floats);
    if (S < 2 || G < 2) return;
    const int64_t gch = (G + S - 1) / S;
    p.kchunk = gch * kGroup;
    p.splits = int((G + gch - 1) / gch);
}

template <int KIND, bool XF32>
void launch_gemm_nj(GemmParams& p, bool fastw, bool fastx, int bm, int64_t part_floats, hipStream_t stream) {
    // 128-wide tiles unless they leave CUs without two workgroups to run;
    // with 64-row tiles (short T) always, the K split filling the CUs: each
    // workgroup then re-reads the activations for twice the columns (7B int8
    // at T = 64, fp32 activations: gate 58.5 -> 44.8, down 58.0 -> 43.7 us;
    // down at T = 256: 168 -> 119 us)
    // ... and when 128-wide tiles take at most half as many rounds of the
    // instance's workgroup slots as 64-wide ones (bf16 activations: 7B down
    // 3584 x 18944 at T = 1536 / 2048 int8 481 / 534 -> 397 / 419 us, int4
    // 533 / 536 -> 412 / 422 us, at 4096 int4 1166 -> 867 us; 7B o 3584 x
    // 3584 int8 at 2048 99 -> 78 us; 1.5B down 1536 x 8960 at 3072 / 4096
    // 212 / 240 -> 170 / 183 us)
    const int per_cu = XF32 || bm == 256 ? 1 : 2, slots = per_cu * device_cu_count();
    const int t128 = p.tiles_m * int((p.N + 127) / 128), t64 = p.tiles_m * int((p.N + 63) / 64);
    const bool nj2_rounds = 2 * ((t128 + slots - 1) / slots) <= (t64 + slots - 1) / slots;
    if (t128 >= 2 * device_cu_count() || bm == 64 || nj2_rounds) {
        p.tiles_n = int((p.N + 127) / 128);
        plan_splits(p, fastw && fastx, part_floats, per_cu);
        launch_gemm_t<KIND, XF32, 2>(p, fastw, fastx, bm, stream);
    } else {
        p.tiles_n = int((p.N + 63) / 64);
        plan_splits(p, fastw && fastx, part_floats, per_cu);
        launch_gemm_t<KIND, XF32, 1>(p, fastw, fastx, bm, stream);
    }
    if (p.splits > 1) {
        const int64_t n = p.T * p.N;
        if (p.N % 4 == 0 && reinterpret_cast<uintptr_t>(p.y) % 16 == 0)
            gemm_reduce4_kernel<<<unsigned((n / 4 + 255) / 256), 256, 0, stream>>>(p.part, p.splits, p.T, p.N, p.bias, p.y);
        else
            gemm_reduce_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(p.part, p.splits, p.T, p.N, p.bias, p.y);
    }
}

// The fp16 operand path (K % 128 == 0, 16-byte aligned activations): one
// preparation launch, the GEMM, and the range sums when K is split, for T
// rows whose operands fit the workspace's operand area.
hipError_t launch_gemmh_chunk(const float* x_f32, const QView& W, const uint16_t* bias, int64_t T, float* y,
                              Workspace* ws, hipStream_t stream) {
    constexpr bool lo = true;
    const int64_t K = W.cols;
    _Float16* ah = nullptr;
    float* rs = nullptr;
    hipError_t e = gemm_operands(ws, T, K, lo, &ah, &rs);
    if (e != hipSuccess) return e;
    _Float16* al = lo ? ah + T * K : nullptr;
    const bool perm = W.kind == 1;
    // rows of up to 8 chunks per thread in registers, one workgroup each;
    // longer rows over enough workgroups for two per CU (at most 8)
    const bool res = K <= 8 * 512 * 8;
    const int seg = res ? 1 : int(std::min<int64_t>(8, std::max<int64_t>(1, (2 * device_cu_count() + T - 1) / T)));
    const unsigned grid = unsigned(T * seg);
    if (res) {
        if (perm) gemm_xprep_kernel<true, true, true><<<grid, 512, 0, stream>>>(x_f32, K, seg, ah, al, rs);
        else gemm_xprep_kernel<false, true, true><<<grid, 512, 0, stream>>>(x_f32, K, seg, ah, al, rs);
    } else {
        if (perm) gemm_xprep_kernel<true, true, false><<<grid, 512, 0, stream>>>(x_f32, K, seg, ah, al, rs);
        else gemm_xprep_kernel<false, true, false><<<grid, 512, 0, stream>>>(x_f32, K, seg, ah, al, rs);
    }
    GemmhParams p;
    p.ah = ah; p.al = al; p.rs = rs;
    p.q = W.q; p.scales = W.scales; p.zeros = W.zeros; p.bias = bias; p.y = y;
    p.T = T; p.N = W.rows; p.K = K; p.G = W.groups;
    p.part = ws->partials;
    // 64 x 128 tiles on 4 waves, two workgroups per CU (a 4-wave workgroup
    // of 128 rows, whose hi + lo operand buffers fill the LDS, runs alone
    // on its CU: 7B int8 at T = 128 / 512 / 1024, down 3584 x 18944 99 /
    // 334 / 684 -> 66 / 212 / 433 us, gate 18944 x 3584 266 / 440 -> 201 /
    // 393 us at 512 / 1024, o 3584 x 3584 at 1024 142 -> 93 us).  From T =
    // 512, int4 and rows of K >= 2048 take 128 x 128 tiles on 8 waves, each
    // converted weight tile feeding twice the rows: 7B int4 at T = 1024 /
    // 2048 down 426 / 936 -> 378 / 782 us, gate 389 / 801 -> 354 / 721 us,
    // int8 gate 402 -> 381 us at 1024 (1.5B int8 gate 8960 x 1536: 110 ->
    // 116 us, kept at 64 rows).
    const bool wide_t = T >= 512 && (W.kind == 1 || K >= 2048);
    const int bm = wide_t ? 128 : 64;
    p.tiles_m = int((T + bm - 1) / bm);
    p.tiles_n = int((p.N + 127) / 128);
    // K ranges (pick_splits)
    p.splits = 1;
    p.kchunk = K;
    {
        // (as plan_splits: 1.5B o 1536 x 1536 at T = 80 / 256 18.5 / 23.0
        // -> 13.6 / 16.5 us)
        const int tiles = p.tiles_m * p.tiles_n, want = (bm == 128 ? 1 : 2) * device_cu_count();
        const int64_t G = K / kGroup;
        if (G >= 2) {
            const int S = pick_splits(tiles, want, G, T, p.N, ws->part_floats);
            if (S >= 2) {
                const int64_t gch = (G + S - 1) / S;
                p.kchunk = gch * kGroup;
                p.splits = int((G + gch - 1) / gch);
            }
        }
    }
    const unsigned ggrid = unsigned(p.tiles_m * p.tiles_n * p.splits);
    if (bm == 128) {
        // (int8 with four K steps in flight, int4 with two: 7B at T = 512 /
        // 1024 / 2048, int8 gate|up 392 / 789 / 1526 -> 374 / 748 / 1446 us,
        // down 212 / 374 / 756 -> 199 / 352 / 714 us; int4 3-5 % slower so)
        if (W.kind == 1) gemmh_kernel<1, true, 2, 128><<<ggrid, 2 * kThreads, 0, stream>>>(p);
        else gemmh_kernel<0, true, 2, 128, 4><<<ggrid, 2 * kThreads, 0, stream>>>(p);
    } else {
        if (W.kind == 1) gemmh_kernel<1, true, 2, 64, 4><<<ggrid, kThreads, 0, stream>>>(p);
        else gemmh_kernel<0, true, 2, 64, 4><<<ggrid, kThreads, 0, stream>>>(p);
    }
    if (p.splits > 1) {
        const int64_t n = p.T * p.N;
        if (p.N % 4 == 0 && reinterpret_cast<uintptr_t>(p.y) % 16 == 0)
            gemm_reduce4_kernel<<<unsigned((n / 4 + 255) / 256), 256, 0, stream>>>(p.part, p.splits, p.T, p.N, p.bias, p.y);
        else
            gemm_reduce_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(p.part, p.splits, p.T, p.N, p.bias, p.y);
    }
    return hipGetLastError();
}

// launch_gemmh_chunk over row chunks whose operands fit the workspace
// (one chunk up to 1024 rows at K = 18944): the operand area is reserved
// with the workspace, so no call allocates.  Chunks are stream-ordered, so
// each reuses the area after the previous chunk's GEMM has read it.
hipError_t launch_gemmh(const float* x_f32, const QView& W, const uint16_t* bias, int64_t T, float* y,
                        Workspace* ws, hipStream_t stream) {
    const int64_t cap = gemm_operand_rows(ws, W.cols);
    if (cap < 128) return hipErrorInvalidValue;
    for (int64_t t0 = 0; t0 < T; t0 += cap) {
        const int64_t tc = T - t0 < cap ? T - t0 : cap;
        const hipError_t e = launch_gemmh_chunk(x_f32 + t0 * W.cols, W, bias, tc, y + t0 * W.rows, ws, stream);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

}  // namespace

hipError_t launch_gemm(const float* x_f32, const uint16_t* x_bf16, const QView& W,
                       const uint16_t* bias, int64_t T, float* y, Workspace* ws, hipStream_t stream) {
    {
        const uintptr_t xa = x_f32 ? reinterpret_cast<uintptr_t>(x_f32) : reinterpret_cast<uintptr_t>(x_bf16);
        // fp32 activations: 17..32 rows of wide or long-K matrices on
        // gemvq's row blocks; past 32 rows on whole 128-column groups the
        // fp16 operand path (22 significant bits against the 24 of three
        // bf16 terms at 1.5x the MFMAs, and faster: 7B at T = 1024, gate
        // 18944 x 3584 int4 648 -> 440 us, down 1053 -> 681 us); up to 32
        // rows the three-term split inside gemm_kernel, whose single launch
        // beats the preparation launch on the narrower matrices left here
        // (1.5B at 32 rows: o 1536 x 1536 16.9 -> 11.6 us, down 1536 x 8960
        // 25.4 -> 21.8; 7B o 22.9 either way), and so up to 64 rows on
        // matrices of at most 2^24 weights (T = 64: 1.5B o 15.6 -> 10.2, down
        // 24.1 -> 19.7, 7B o 23.7 -> 21.4 us; 7B gate 44.8 against 64.7) and
        // up to 256 rows on matrices of at most 2^22 (T = 96..256: 7B k 512
        // x 3584 18.0..22.4 -> 13.3..14.6 us, 1.5B o 23.2..25.1 ->
        // 17.7..22.4), at any T on matrices of at most 2^19 (1.5B k 256 x
        // 1536 at T = 257 / 512 / 2048: 17.3 / 20.7 / 34.0 -> 12.7 / 12.4 /
        // 25.9 us)
        if (x_f32) {
            hipError_t e = hipSuccess;
            if (launch_gemm_rows(x_f32, W, bias, T, y, ws, stream, &e)) return e;
        }
        const int64_t nk = W.rows * W.cols;
        const bool split_in_kernel = T <= 32 || (T <= 64 && nk <= (int64_t(1) << 24)) ||
                                     (T <= 256 && nk <= (int64_t(1) << 22)) || nk <= (int64_t(1) << 19);
        if (x_f32 && !split_in_kernel && W.cols % kGroup == 0 && xa % 16 == 0)
            return launch_gemmh(x_f32, W, bias, T, y, ws, stream);
    }
    GemmParams p;
    p.part = ws->partials;
    p.xf = x_f32; p.xb = x_bf16;
    p.q = W.q; p.scales = W.scales; p.zeros = W.zeros; p.bias = bias; p.y = y;
    p.T = T; p.N = W.rows; p.K = W.cols; p.G = W.groups;
    const bool fastw = (p.K % kGroup == 0);
    const uintptr_t xa = x_f32 ? reinterpret_cast<uintptr_t>(x_f32) : reinterpret_cast<uintptr_t>(x_bf16);
    const bool fastx = (p.K % BK == 0) && (xa % 16 == 0);
    // 64-row tiles for short T (less MFMA work on padding rows, more tiles):
    // 7B int8, fp32 activations, gate 18944 x 3584 at T = 33 / 64 / 128 /
    // 256: 115 / 113 / 137 / 202 -> 55 / 58 / 97 / 139 us; down 3584 x
    // 18944 at T = 64 / 256: 115 / 186 -> 58 / 170 us, but at T = 128 (a
    // narrow matrix, already split over K) 93 -> 103: kept at 128 rows there
    const bool short_t = T <= 64 || (T > 128 && T <= 256) || (T <= 128 && W.rows >= 8192);
    // 256-row tiles (8 waves) for long bf16 prefills of narrow int4
    // matrices: each dequantised weight tile (nibble unpack + zero point,
    // the costlier conversion) feeds twice the MFMAs.  7B at T = 1024 with
    // 256 / 128 rows: int4 down 259 / 275 us, int4 gate|up 235 / 208 us,
    // int8 down 269 / 249 us (one 8-wave workgroup per CU leaves the step
    // barriers uncovered, which costs more than the conversion saves on a
    // wide matrix or with int8's cheaper conversion).
    const bool big = !x_f32 && fastw && fastx && T >= 512 && W.kind == 1 && W.rows < 8192;
    const int bm = (short_t && fastw && fastx) ? 64 : (big ? 256 : 128);
    p.tiles_m = int((T + bm - 1) / bm);
    if (x_f32) {
        if (W.kind == 1) launch_gemm_nj<1, true>(p, fastw, fastx, bm, ws->part_floats, stream);
        else launch_gemm_nj<0, true>(p, fastw, fastx, bm, ws->part_floats, stream);
    } else {
        if (W.kind == 1) launch_gemm_nj<1, false>(p, fastw, fastx, bm, ws->part_floats, stream);
        else launch_gemm_nj<0, false>(p, fastw, fastx, bm, ws->part_floats, stream);
    }
    return hipGetLastError();
}

}  // namespace iq

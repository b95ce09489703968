// iq_quant.hip -- on-device quantize + pack and the quantised embedding
// gather for gfx950.
//
// quantize: bit-exact to llm::quantize (src/quant.cpp:34-84).  One wave64
// covers four 128-column groups of one row: each 16-lane DPP row of the wave
// owns one group, each lane 8 consecutive columns (one 16-byte load of bf16).
// The group's absmax (int8) or [min,max] widened to 0 (int4) is reduced
// inside the 16 lanes; every lane then derives the same bf16 scale and writes
// its 8 codes (8 bytes int8, 4 bytes int4), so stores stay coalesced.
// Arithmetic follows the reference operation by operation: fp32 correctly
// rounded division, round-half-even (std::lrint under the default mode),
// the reference's clamps, and its comparison forms for max/min so that NaN
// inputs are skipped the same way (the file is built without fast-math and
// with -ffp-contract=off).
//
// embedding: out[t,i] = s * float(q - z) exactly as dequant()
// (src/quant.cpp:86-93; kernels/ops/quant.cu:304-309).
#include <algorithm>

#include "iq_internal.h"

namespace iq {

namespace {

constexpr int kQThreads = 256;

// Max / min over the 16 lanes of a DPP row (one quantisation group), by
// row rotations: exact in any order.  v_max_f32 / v_min_f32 return the other
// operand for a NaN (IEEE maxNum), which is what the reference's `a < b`
// updates do; the running values start at 0 and never become NaN.
template <int N>
__device__ __forceinline__ float row_ror_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + N, 0xF, 0xF, true));
}
__device__ __forceinline__ float row16_maxf(float v) {
    v = __builtin_fmaxf(v, row_ror_f<8>(v));
    v = __builtin_fmaxf(v, row_ror_f<4>(v));
    v = __builtin_fmaxf(v, row_ror_f<2>(v));
    return __builtin_fmaxf(v, row_ror_f<1>(v));
}
__device__ __forceinline__ float row16_minf(float v) {
    v = __builtin_fminf(v, row_ror_f<8>(v));
    v = __builtin_fminf(v, row_ror_f<4>(v));
    v = __builtin_fminf(v, row_ror_f<2>(v));
    return __builtin_fminf(v, row_ror_f<1>(v));
}

// Reference clamp (std::max(lo, std::min(hi, v))).
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// lrint(w / s) of the reference (fp32 division rounded to nearest, then
// round-half-even to an integer), for bf16 w and a bf16 scale s > 0 given
// with r = 1 / s (correctly rounded).  Both w and s carry 8-bit
// significands, W 2^a and S 2^b, so the exact quotient q* = (W / S) 2^(a-b)
// is either a half-integer or at least 2^(a-b) / (2 S) away from every
// half-integer, while both fl(q*) (what the reference rounds) and t = w * r
// are within 2^-22 |q*| <= 2^-22 (255 / S) 2^(a-b) of q*: far inside that
// gap.  So rint(t) equals lrint(fl(q*)) except at exact ties q* = h, which
// fma(h, s, -w) == 0 detects exactly (h has 9 and s 8 significant bits, so
// h * s is exact), and there rint(h) rounds half to even as lrint does.
// Non-finite t (s = 0 or infinite, or a NaN input) gives 0, as int(lrint)
// does on x86-64 for such quotients (lrint yields LONG_MIN, int(long) keeps
// its low 32 bits); |q*| < 2^31 otherwise, since s is w's group maximum / 127
// (or the range / 15) rounded to bf16.
__device__ __forceinline__ int qdiv(float w, float s, float r) {
    const float t = w * r;
    if (!(__builtin_fabsf(t) < 9.2233720368547758e18f)) return 0;
    const float h = __builtin_floorf(t) + 0.5f;
    const bool tie = __builtin_fmaf(h, s, -w) == 0.0f;
    return int(__builtin_rintf(tie ? h : t));
}

// Scale and reciprocal used by qdiv: very small scales (bf16 subnormals
// included) are moved up by 2^64 together with the values (exact powers of
// two), so that 1 / s stays finite.
struct QScale {
    float s, r, up;  // scale (moved), its reciprocal, factor applied to w
};
__device__ __forceinline__ QScale qscale(float s) {
    QScale q;
    q.up = s < 5.421010862427522e-20f ? 1.8446744073709552e19f : 1.0f;  // 2^-64, 2^64
    q.s = s * q.up;
    q.r = 1.0f / q.s;
    return q;
}

template <int KIND, bool FAST>
__global__ __launch_bounds__(kQThreads) void quantize_kernel(const uint16_t* __restrict__ w,
                                                             int64_t rows, int64_t cols, int64_t G,
                                                             int64_t quads, uint8_t* __restrict__ q,
                                                             uint16_t* __restrict__ scales,
                                                             uint8_t* __restrict__ zeros) {
    const int lane = threadIdx.x & 63;
    // Grid-stride over (row, 4-group quad) items; the bf16 values of the
    // next QD items are requested before the current one is converted.
    // (row, quad) cursors advance without division (a 64-bit division is a
    // long instruction sequence on the GPU).
    const int64_t items = rows * quads;
    const int64_t stride = int64_t(gridDim.x) * (kQThreads / 64);
    const int64_t first = int64_t(blockIdx.x) * (kQThreads / 64) + (threadIdx.x >> 6);
    if (first >= items) return;
    const int64_t sr = stride / quads, sq = stride % quads;
    struct Cursor {
        int64_t r, qd;
    };
    auto advance = [&](Cursor& c) {
        c.r += sr;
        c.qd += sq;
        if (c.qd >= quads) {
            c.qd -= quads;
            c.r += 1;
        }
    };
    auto fetch = [&](const Cursor& c) {
        uint4 raw = make_uint4(0, 0, 0, 0);
        const int64_t gg = c.qd * 4 + (lane >> 4);
        if (FAST && c.r < rows && gg < G) raw = *reinterpret_cast<const uint4*>(w + c.r * cols + gg * kGroup + (lane & 15) * 8);
        return raw;
    };
    constexpr int QD = 2;
    Cursor cc{first / quads, first % quads}, fc = cc;
    uint4 ring[QD];
#pragma unroll
    for (int d = 0; d < QD; d++) {
        ring[d] = fetch(fc);
        advance(fc);
    }
    for (; cc.r < rows; advance(cc)) {
    const uint4 cur = ring[0];
#pragma unroll
    for (int d = 0; d < QD - 1; d++) ring[d] = ring[d + 1];
    ring[QD - 1] = fetch(fc);
    advance(fc);
    const int64_t r = cc.r;
    const int64_t g = cc.qd * 4 + (lane >> 4);  // this 16-lane row's group
    const bool gvalid = g < G;
    const int64_t c0 = g * kGroup + (lane & 15) * 8;    // first of my 8 columns
    const uint16_t* wr = w + r * cols;

    float v[8];
    if (FAST) {  // cols % 128 == 0: whole groups, 16-byte aligned rows
        const uint4 raw = cur;
        const uint32_t wd[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
            v[2 * i] = __uint_as_float(wd[i] << 16);
            v[2 * i + 1] = __uint_as_float(wd[i] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (gvalid && c0 + i < cols) ? bf16_to_f32(wr[c0 + i]) : 0.0f;
    }
    const int nvalid = FAST ? 8 : (gvalid ? int(cols - c0 < 0 ? 0 : (cols - c0 < 8 ? cols - c0 : 8)) : 0);

    if (KIND == 0) {
        // amax = std::max(amax, fabs(v)) in column order; comparisons skip NaN.
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float a = __builtin_fabsf(v[i]);
            if (i < nvalid && amax < a) amax = a;
        }
        amax = row16_maxf(amax);
        const uint16_t sb = f32_to_bf16(amax > 0.0f ? amax / 127.0f : 1.0f);
        const QScale qs = qscale(bf16_to_f32(sb));
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = clampi(qdiv(v[i] * qs.up, qs.s, qs.r), -127, 127);
            const uint32_t b = uint32_t(uint8_t(int8_t(c)));
            if (i < 4) lo |= b << (8 * i);
            else hi |= b << (8 * (i - 4));
        }
        if (!gvalid) continue;
        if ((lane & 15) == 0) scales[r * G + g] = sb;
        uint8_t* qr = q + r * cols + c0;
        if (FAST) {
            *reinterpret_cast<uint2*>(qr) = make_uint2(lo, hi);
        } else {
            for (int i = 0; i < nvalid; i++) qr[i] = uint8_t((i < 4 ? lo >> (8 * i) : hi >> (8 * (i - 4))) & 0xFF);
        }
    } else {
        // lo = std::min(lo, v), hi = std::max(hi, v), both starting at 0.
        float mn = 0.0f, mx = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (i < nvalid) {
                if (v[i] < mn) mn = v[i];
                if (mx < v[i]) mx = v[i];
            }
        }
        mn = row16_minf(mn);
        mx = row16_maxf(mx);
        const uint16_t sb = f32_to_bf16(mx > mn ? (mx - mn) / 15.0f : 1.0f);
        const QScale qs = qscale(bf16_to_f32(sb));
        const int z = clampi(qdiv(-mn * qs.up, qs.s, qs.r), 0, 15);
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = clampi(qdiv(v[i] * qs.up, qs.s, qs.r) + z, 0, 15);
            packed |= uint32_t(c) << (4 * i);
        }
        if (!gvalid) continue;
        if ((lane & 15) == 0) {
            scales[r * G + g] = sb;
            zeros[r * G + g] = uint8_t(z);
        }
        // (r*cols + c0) is even: the lane owns whole bytes.
        uint8_t* qb = q + (r * cols + c0) / 2;
        if (FAST) {
            *reinterpret_cast<uint32_t*>(qb) = packed;
        } else {
            for (int i = 0; i < nvalid; i += 2) qb[i / 2] = uint8_t((packed >> (4 * i)) & 0xFF);
        }
    }
    }
}

template <bool FAST>
__global__ __launch_bounds__(256) void embedding_kernel(QView t, const int64_t* __restrict__ ids,
                                                        int64_t T, int64_t H, float* __restrict__ out) {
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;  // one thread per 4 outputs
    const int64_t per_row = (H + 3) / 4;
    if (idx >= T * per_row) return;
    const int64_t tk = idx / per_row, c0 = (idx % per_row) * 4;
    const int64_t id = ids[tk];
    float* o = out + tk * H + c0;
    const int n = int(H - c0 < 4 ? H - c0 : 4);
    if (id < 0 || id >= t.rows) {
        for (int i = 0; i < n; i++) o[i] = __builtin_nanf("");
        return;
    }
    for (int i = 0; i < n; i++) {
        const int64_t c = c0 + i, g = c / kGroup;
        const float s = bf16_to_f32(t.scales[id * t.groups + g]);
        float val;
        if (t.kind == 0) {
            val = s * float(int8_t(t.q[id * t.cols + c]));
        } else {
            const uint8_t byte = t.q[(id * t.cols + c) / 2];
            const int nib = (c & 1) ? (byte >> 4) : (byte & 0xF);
            val = s * float(nib - int(t.zeros[id * t.groups + g]));
        }
        o[i] = val;
    }
}

}  // namespace

hipError_t launch_quantize(const uint16_t* w, int64_t rows, int64_t cols, int kind, uint8_t* q,
                           uint16_t* scales, uint8_t* zeros, hipStream_t stream) {
    const int64_t G = (cols + kGroup - 1) / kGroup;
    const int64_t quads = (G + 3) / 4;
    const int64_t waves = rows * quads;
    // enough resident waves to stream; each walks items in strides of the grid
    const int64_t cap = int64_t(device_cu_count()) * 8;
    const unsigned grid = unsigned(std::min<int64_t>((waves + 3) / 4, cap));
    const bool fast = cols % kGroup == 0;
    if (kind == 0) {
        if (fast) quantize_kernel<0, true><<<grid, kQThreads, 0, stream>>>(w, rows, cols, G, quads, q, scales, zeros);
        else quantize_kernel<0, false><<<grid, kQThreads, 0, stream>>>(w, rows, cols, G, quads, q, scales, zeros);
    } else {
        if (fast) quantize_kernel<1, true><<<grid, kQThreads, 0, stream>>>(w, rows, cols, G, quads, q, scales, zeros);
        else quantize_kernel<1, false><<<grid, kQThreads, 0, stream>>>(w, rows, cols, G, quads, q, scales, zeros);
    }
    return hipGetLastError();
}

hipError_t launch_embedding(const QView& t, const int64_t* ids, int64_t T, int64_t H, float* out,
                            hipStream_t stream) {
    const int64_t n = T * ((H + 3) / 4);
    const unsigned grid = unsigned((n + 255) / 256);
    embedding_kernel<true><<<grid, 256, 0, stream>>>(t, ids, T, H, out);
    return hipGetLastError();
}

}  // namespace iq

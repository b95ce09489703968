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
#include "iq_internal.h"

namespace iq {

namespace {

constexpr int kQThreads = 256;

// Reference clamp (std::max(lo, std::min(hi, v))).
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// int(std::lrint(f)) as the reference computes it on x86-64: lrint rounds
// half-to-even into a 64-bit long, and yields LONG_MIN ("integer indefinite")
// for NaN, +-inf and |f| >= 2^63; int(long) keeps the low 32 bits.  Finite
// quotients here are small, but a bf16 scale that underflows to 0 makes w/s
// infinite or NaN, and then the code the reference stores is 0 (+ z).
__device__ __forceinline__ int lrint_i(float f) {
    if (!(__builtin_fabsf(f) < 9.2233720368547758e18f)) return 0;
    const long long v = (long long)__builtin_rintf(f);
    return int(uint32_t(uint64_t(v)));
}

template <int KIND, bool FAST>
__global__ __launch_bounds__(kQThreads) void quantize_kernel(const uint16_t* __restrict__ w,
                                                             int64_t rows, int64_t cols, int64_t G,
                                                             int64_t quads, uint8_t* __restrict__ q,
                                                             uint16_t* __restrict__ scales,
                                                             uint8_t* __restrict__ zeros) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = int64_t(blockIdx.x) * (kQThreads / 64) + (threadIdx.x >> 6);
    if (wave >= rows * quads) return;
    const int64_t r = wave / quads;
    const int64_t g = (wave % quads) * 4 + (lane >> 4);  // this 16-lane row's group
    const bool gvalid = g < G;
    const int64_t c0 = g * kGroup + (lane & 15) * 8;    // first of my 8 columns
    const uint16_t* wr = w + r * cols;

    float v[8];
    if (FAST) {  // cols % 128 == 0: whole groups, 16-byte aligned rows
        uint4 raw = make_uint4(0, 0, 0, 0);
        if (gvalid) raw = *reinterpret_cast<const uint4*>(wr + c0);
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
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            const float o = __shfl_xor(amax, off, 16);
            if (amax < o) amax = o;
        }
        const uint16_t sb = f32_to_bf16(amax > 0.0f ? amax / 127.0f : 1.0f);
        const float s = bf16_to_f32(sb);
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = clampi(lrint_i(v[i] / s), -127, 127);
            const uint32_t b = uint32_t(uint8_t(int8_t(c)));
            if (i < 4) lo |= b << (8 * i);
            else hi |= b << (8 * (i - 4));
        }
        if (!gvalid) return;
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
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) {
            const float a = __shfl_xor(mn, off, 16);
            const float b = __shfl_xor(mx, off, 16);
            if (a < mn) mn = a;
            if (mx < b) mx = b;
        }
        const uint16_t sb = f32_to_bf16(mx > mn ? (mx - mn) / 15.0f : 1.0f);
        const float s = bf16_to_f32(sb);
        const int z = clampi(lrint_i(-mn / s), 0, 15);
        uint32_t packed = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const int c = clampi(lrint_i(v[i] / s) + z, 0, 15);
            packed |= uint32_t(c) << (4 * i);
        }
        if (!gvalid) return;
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
    const unsigned grid = unsigned((waves + 3) / 4);
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

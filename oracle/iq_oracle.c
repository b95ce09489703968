/*
 * iq_oracle.c -- CPU restatement of the reference's quantized-weight path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker: tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it; the
 * product (infer_amd/, libiq.so) never links, loads or calls it.
 *
 * Every function restates one piece of the reference (RyanXiaoo/infer),
 * written here in plain C from the reference's behaviour:
 *   iqo_f32_to_bf16 / iqo_bf16_to_f32   src/f16.h:37-51
 *   iqo_quantize                         src/quant.cpp:34-84
 *   iqo_dequant / iqo_dequant_matrix     src/quant.cpp:86-93
 *   iqo_linear_q_f32                     src/forward.cpp:35-47 with dequant()
 *                                        in place of bf16_to_f32 (the CPU
 *                                        matvec "on dequantized weights")
 *   iqo_linear_q_f64                     tests/test_ops_gpu.cu:676-687 (double
 *                                        reference + conditioning sum |w*x|)
 *   iqo_embedding                        kernels/ops/quant.cu:304-309 semantics
 *                                        (= dequant() of the gathered row)
 *
 * Kind codes follow the device ABI enum gpu::QuantKind (kernels/ops/ops.cuh:165):
 * 0 = int8, 1 = int4.  Layout (src/quant.h:34-58): group 128 along a row;
 * int8 codes rows*cols bytes; int4 codes rows*cols/2 bytes, element (r,c) at
 * byte (r*cols+c)/2, low nibble when c is even; scales bf16 bits [rows][G];
 * zeros u8 [rows][G] (int4 only).
 *
 * How each function is pinned (tests/test_oracle.py): quantize against the
 * fixtures written by the reference's own compiled quant.cpp
 * (tests/golden/gen_golden.py), bf16 against the exhaustive round-trip and
 * spot values of tests/test_f16.cpp, dequant against closed forms, linear
 * against an independent numpy float64 matmul.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define IQO_GROUP 128

static inline float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* src/f16.h:37-39: widening is a 16-bit left shift. */
float iqo_bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

/* src/f16.h:41-51: NaN stays NaN (quiet bit forced), otherwise round to
 * nearest even by adding 0x7fff plus the lowest surviving bit. */
uint16_t iqo_f32_to_bf16(float f) {
    uint32_t u = f32_bits(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
    return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* int(std::lrint(f)) as the reference evaluates it on x86-64 (the platform
 * the fixtures come from): round half to even into a 64-bit long, LONG_MIN
 * ("integer indefinite") for NaN, +-inf and |f| >= 2^63, then int(long) keeps
 * the low 32 bits.  Spelled out so the oracle does not depend on the host
 * libm for non-finite quotients (a bf16 scale that underflows to 0). */
static inline int lrint_ref(float f) {
    if (!(fabsf(f) < 9.2233720368547758e18f)) return 0;
    return (int)(uint32_t)(uint64_t)(long long)rintf(f);
}

/* src/quant.cpp:34-84.  Returns 0 on success, -1 on a bad kind, -2 when int4
 * is asked for with odd cols (the reference throws std::runtime_error). */
int iqo_quantize(const uint16_t* w, int64_t rows, int64_t cols, int kind,
                 uint8_t* q, uint16_t* scales, uint8_t* zeros, float* rowbuf) {
    if (kind != 0 && kind != 1) return -1;
    if (kind == 1 && (cols % 2)) return -2;
    const int64_t G = (cols + IQO_GROUP - 1) / IQO_GROUP;
    memset(q, 0, (size_t)(kind == 1 ? rows * cols / 2 : rows * cols));
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t c = 0; c < cols; c++) rowbuf[c] = iqo_bf16_to_f32(w[r * cols + c]);
        for (int64_t g = 0; g < G; g++) {
            const int64_t c0 = g * IQO_GROUP;
            const int64_t c1 = cols < c0 + IQO_GROUP ? cols : c0 + IQO_GROUP;
            if (kind == 0) {
                float amax = 0.0f;
                /* std::max(amax, fabs(v)) == (amax < |v|) ? |v| : amax */
                for (int64_t c = c0; c < c1; c++) { float a = fabsf(rowbuf[c]); if (amax < a) amax = a; }
                const uint16_t sb = iqo_f32_to_bf16(amax > 0 ? amax / 127.0f : 1.0f);
                const float s = iqo_bf16_to_f32(sb);
                scales[r * G + g] = sb;
                for (int64_t c = c0; c < c1; c++) {
                    int v = lrint_ref(rowbuf[c] / s);
                    v = clampi(v, -127, 127);
                    q[r * cols + c] = (uint8_t)(int8_t)v;
                }
            } else {
                float lo = 0.0f, hi = 0.0f;
                /* std::min(lo, v) == (v < lo) ? v : lo ; std::max(hi, v) == (hi < v) ? v : hi */
                for (int64_t c = c0; c < c1; c++) {
                    const float v = rowbuf[c];
                    if (v < lo) lo = v;
                    if (hi < v) hi = v;
                }
                const uint16_t sb = iqo_f32_to_bf16(hi > lo ? (hi - lo) / 15.0f : 1.0f);
                const float s = iqo_bf16_to_f32(sb);
                int z = lrint_ref(-lo / s);
                z = clampi(z, 0, 15);
                scales[r * G + g] = sb;
                zeros[r * G + g] = (uint8_t)z;
                for (int64_t c = c0; c < c1; c++) {
                    int v = lrint_ref(rowbuf[c] / s) + z;
                    v = clampi(v, 0, 15);
                    uint8_t* byte = &q[(r * cols + c) / 2];
                    if (c % 2 == 0) *byte = (uint8_t)((*byte & 0xF0) | v);
                    else *byte = (uint8_t)((*byte & 0x0F) | (v << 4));
                }
            }
        }
    }
    return 0;
}

/* src/quant.cpp:86-93 */
float iqo_dequant(const uint8_t* q, const uint16_t* scales, const uint8_t* zeros, int kind,
                  int64_t cols, int64_t r, int64_t c) {
    const int64_t G = (cols + IQO_GROUP - 1) / IQO_GROUP, g = c / IQO_GROUP;
    const float s = iqo_bf16_to_f32(scales[r * G + g]);
    if (kind == 0) return s * (float)(int8_t)q[r * cols + c];
    const uint8_t byte = q[(r * cols + c) / 2];
    const int v = (c % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
    return s * (float)(v - (int)zeros[r * G + g]);
}

void iqo_dequant_matrix(const uint8_t* q, const uint16_t* scales, const uint8_t* zeros, int kind,
                        int64_t rows, int64_t cols, float* out) {
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < cols; c++)
            out[r * cols + c] = iqo_dequant(q, scales, zeros, kind, cols, r, c);
}

/* src/forward.cpp:35-47 with dequant() in place of bf16_to_f32: for each
 * activation row t and output o, acc starts at the bf16 bias (or 0) and adds
 * w(o,i)*x[t,i] in order i = 0..in-1 in fp32.  The dequantised value is
 * formed per element exactly as dequant() does (s * float(q - z)), so this is
 * the reference CPU path's arithmetic, one multiply-add per weight.
 * The product and the add are separate fp32 roundings (no contraction;
 * the file is compiled with -ffp-contract=off). */
void iqo_linear_q_f32(const float* x, const uint8_t* q, const uint16_t* scales, const uint8_t* zeros,
                      int kind, const uint16_t* bias, int64_t T, int64_t in, int64_t out, float* y) {
    const int64_t G = (in + IQO_GROUP - 1) / IQO_GROUP;
    for (int64_t t = 0; t < T; t++) {
        const float* xr = x + t * in;
        for (int64_t o = 0; o < out; o++) {
            float acc = bias ? iqo_bf16_to_f32(bias[o]) : 0.0f;
            const uint16_t* sr = scales + o * G;
            if (kind == 0) {
                const int8_t* qr = (const int8_t*)(q + o * in);
                for (int64_t i = 0; i < in; i++) {
                    const float w = iqo_bf16_to_f32(sr[i / IQO_GROUP]) * (float)qr[i];
                    acc += w * xr[i];
                }
            } else {
                const uint8_t* zr = zeros + o * G;
                for (int64_t i = 0; i < in; i++) {
                    const uint8_t byte = q[(o * in + i) / 2];
                    const int v = ((o * in + i) % 2 == 0) ? (byte & 0x0F) : (byte >> 4);
                    const float w = iqo_bf16_to_f32(sr[i / IQO_GROUP]) * (float)(v - (int)zr[i / IQO_GROUP]);
                    acc += w * xr[i];
                }
            }
            y[t * out + o] = acc;
        }
    }
}

/* tests/test_ops_gpu.cu:676-687: double-precision dot product over the
 * dequantised weights, plus the conditioning sum |b| + sum_i |w*x| that the
 * reference normalises errors by (kGemvTol = 5e-6, test_ops_gpu.cu:199-206). */
void iqo_linear_q_f64(const float* x, const uint8_t* q, const uint16_t* scales, const uint8_t* zeros,
                      int kind, const uint16_t* bias, int64_t T, int64_t in, int64_t out,
                      double* y, double* cond) {
    for (int64_t t = 0; t < T; t++)
        for (int64_t o = 0; o < out; o++) {
            double acc = bias ? (double)iqo_bf16_to_f32(bias[o]) : 0.0, mag = fabs(acc);
            for (int64_t i = 0; i < in; i++) {
                const double p = (double)iqo_dequant(q, scales, zeros, kind, in, o, i) * (double)x[t * in + i];
                acc += p;
                mag += fabs(p);
            }
            y[t * out + o] = acc;
            cond[t * out + o] = mag;
        }
}

/* kernels/ops/quant.cu:304-309: out[t,i] = dequant(table, ids[t], i). */
void iqo_embedding(const uint8_t* q, const uint16_t* scales, const uint8_t* zeros, int kind,
                   int64_t H, const int64_t* ids, int64_t T, float* out) {
    for (int64_t t = 0; t < T; t++)
        for (int64_t i = 0; i < H; i++) out[t * H + i] = iqo_dequant(q, scales, zeros, kind, H, ids[t], i);
}

/*
 * iq.h -- C ABI of the MI355X (gfx950) quantized-weight matrix path.
 *
 * Drop-in boundary for the quantised part of the reference's device ABI
 * (RyanXiaoo/infer kernels/ops/ops.cuh:165-178).  Plain C: no HIP, CUDA or
 * torch types; device memory is passed as plain pointers owned by the caller,
 * the stream as an opaque pointer (a hipStream_t; NULL = the null stream).
 *
 * Layout (the reference's src/quant.h:34-58, produced by src/quant.cpp and
 * tools/quantize.cpp), one [rows x cols] matrix, row-major, groups of
 * IQ_GROUP consecutive columns along a row:
 *   q       int8: rows*cols bytes (two's complement codes -127..127)
 *           int4: rows*cols/2 bytes, element (r,c) in byte (r*cols+c)/2,
 *                 low nibble when c is even (codes 0..15)
 *   scales  bf16 bits, rows x ceil(cols/128)
 *   zeros   int4 only: u8 zero points, rows x ceil(cols/128); NULL for int8
 *   dequant: int8 w = s*q ; int4 w = s*(q - z)          (src/quant.cpp:86-93)
 *
 * Every entry point enqueues work on `stream` and returns without
 * synchronising.  Return value: 0 on success, a negative IQ_E* code when the
 * arguments are rejected on the host (nothing was enqueued), or a positive
 * hipError_t when the HIP runtime reported an error.  No exception crosses
 * this boundary.  The library keeps one workspace (activation operands,
 * split-K partial sums, the prefill GEMM's prepared operands; about 167 MB)
 * per (device, stream) pair, allocated by iq_init / iq_init_stream or on the
 * first call on that stream: calls on different streams may overlap, and
 * calls on one stream are ordered by the stream.  After that no call
 * allocates, frees or synchronises, so any call can be graph-captured the
 * first time it is made.  A stream under graph capture cannot allocate: a
 * call on a capturing stream that has no workspace yet (no iq_init_stream
 * before the capture) returns an error and enqueues nothing.
 */
#ifndef IQ_H
#define IQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IQ_GROUP 128

/* gpu::QuantKind (kernels/ops/ops.cuh:165): kInt8 = 0, kInt4 = 1. */
enum { IQ_INT8 = 0, IQ_INT4 = 1 };

/* Error codes (negative). */
enum {
    IQ_OK = 0,
    IQ_EKIND = -1,      /* kind is neither IQ_INT8 nor IQ_INT4 */
    IQ_ESHAPE = -2,     /* inconsistent or unsupported sizes */
    IQ_ENULL = -3,      /* a required pointer is NULL */
    IQ_ETOOLARGE = -4,  /* problem exceeds the workspace limits */
    IQ_ENOMEM = -5,     /* workspace allocation failed */
    IQ_EDEVICE = -6,    /* no usable gfx950 device, or not the chain's device */
    IQ_EALIAS = -7      /* a chain stage's output overlaps its input */
};

/* gpu::QuantView (kernels/ops/ops.cuh:166-172), byte-compatible on LP64:
 * a 4-byte kind, 4 bytes padding, then rows/cols/groups and three pointers. */
typedef struct iq_view {
    int32_t kind;
    int64_t rows, cols, groups;  /* groups = ceil(cols / 128) */
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;        /* int4: rows*groups bytes; int8: NULL */
} iq_view;

/* y[b, o] = sum_c dequant(W, o, c) * x[b, c] (+ bf16 bias[o]), b < B, o < out.
 * Replaces launch_gemv_batched_q (kernels/ops/ops.cuh:173-174,
 * kernels/ops/quant.cu:312-345).  1 <= B <= 32.  x is fp32 [B][in]
 * (only B rows are read; the reference reads up to 32), y fp32 [B][out]
 * (only B rows are written).  in == W->cols, out == W->rows.  bias may be NULL. */
int iq_gemv(const float* x, const iq_view* W, const uint16_t* bias, int B, int64_t in,
            int64_t out, float* y, void* stream);

/* iq_gemv without any allocation, for callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops and harnesses that
 * forbid hipMalloc).  No counterpart in the reference.  Same contract and
 * kernels as iq_gemv, limited to in <= 32768 (IQ_ETOOLARGE beyond), with
 * its scratch (activation operands and split-K partial sums, ~20.1 MiB) in
 * a static device array of the library that each device holds until the
 * process ends.  Every call on a device shares that array, whatever the
 * stream: calls that overlap in time on one device race, so order them
 * (e.g. one stream).  No state carries from one call to the next. */
int iq_gemv_noalloc(const float* x, const iq_view* W, const uint16_t* bias, int B, int64_t in,
                    int64_t out, float* y, void* stream);

/* The two halves of iq_gemv, for callers that multiply one activation
 * block by several matrices (q/k/v, gate/up share their input):
 * iq_gemv_prep takes x [B][in] (fp32) once into the device workspace: a
 * copy for B <= 4 (the GEMV kernel converts it itself), otherwise per row
 * and 128-column group a power-of-two scale 2^-k and x * 2^k as two fp16
 * terms (or as four signed byte limbs of rint(x * 2^k)), in the column
 * order that `kind`'s weight unpacking produces;
 * iq_gemv_prepped then runs the GEMV of any matrix of that kind and width on
 * the prepared block.  A prepared block belongs to the stream it was made
 * on and stays valid until the next iq_gemv_prep on that stream, or until
 * an iq_gemv / iq_gemv_multi / iq_linear on that stream reuses its buffers.
 * iq_gemv_prepped returns IQ_ESHAPE when there is no valid preparation or
 * (B, in, kind) differ from it.
 * No reference counterpart: the reference's launcher re-reads x per matrix. */
int iq_gemv_prep(const float* x, int B, int64_t in, int kind, void* stream);
int iq_gemv_prepped(const iq_view* W, const uint16_t* bias, int B, int64_t in, int64_t out,
                    float* y, void* stream);

/* iq_gemv_prepped for n <= 4 matrices of one kind and width at once
 * (y_i = x * W_i^T + bias_i, out_i = Ws[i]->rows): q|k|v or gate|up of a
 * layer in one launch.  The reference runs them as separate launches
 * (kernels/batch_gpu.cu:192-194,210-211) and fuses only bf16 weights
 * (kernels/model_gpu.cu:31-38).  biases may be NULL (no bias anywhere) or
 * hold NULL entries. */
int iq_gemv_prepped_multi(const iq_view* const* Ws, int n, const uint16_t* const* biases, int B,
                          int64_t in, float* const* ys, void* stream);

/* iq_gemv for n <= 4 matrices of one kind and width sharing the activations
 * x [B][in]: one GEMV launch reads x and all n matrices (at B <= 4 the
 * activation conversion happens inside it; at larger B a conversion launch
 * precedes it, and split-K shapes add a reduction launch).  Same matrix/bias
 * conventions as iq_gemv_prepped_multi; the prepared block of the workspace
 * may be overwritten.  No reference counterpart (see iq_gemv_prepped_multi). */
int iq_gemv_multi(const float* x, const iq_view* const* Ws, int n, const uint16_t* const* biases, int B,
                  int64_t in, float* const* ys, void* stream);

/* Same contract for any T >= 1 (fp32 activations).  Replaces
 * launch_gemm_tiled_q (kernels/ops/ops.cuh:175-176, kernels/ops/quant.cu:347-351).
 * Runs the MFMA prefill GEMM with the activations split into bf16 hi + lo. */
int iq_gemm(const float* x, const iq_view* W, const uint16_t* bias, int64_t T, int64_t in,
            int64_t out, float* y, void* stream);

/* Prefill GEMM with bf16 activations x [T][in] (bf16 bits), fp32 output.
 * No reference counterpart (the reference's activations are fp32); it is the
 * bf16-activation form of iq_gemm used for the Qwen2.5-7B prefill shapes. */
int iq_gemm_bf16x(const uint16_t* x, const iq_view* W, const uint16_t* bias, int64_t T,
                  int64_t in, int64_t out, float* y, void* stream);

/* The quantised linear call site, GpuBatch::Impl::linear_b
 * (kernels/batch_gpu.cu:137-147): T <= 32 -> iq_gemv, T > 32 -> iq_gemm. */
int iq_linear(const float* x, const iq_view* W, const uint16_t* bias, int64_t T, int64_t in,
              int64_t out, float* y, void* stream);

/* out[t, i] = dequant(table, ids[t], i), exactly.  Replaces launch_embedding_q
 * (kernels/ops/ops.cuh:177-178, kernels/ops/quant.cu:304-309,353-357).
 * H == table->cols.  An id outside [0, rows) yields a row of NaN (the
 * reference reads out of bounds). */
int iq_embedding(const iq_view* table, const int64_t* ids, int64_t T, int64_t H, float* out,
                 void* stream);

/* On-device quantize + pack of a bf16 [rows x cols] matrix, bit-exact to
 * llm::quantize (src/quant.cpp:34-84, src/quant.h:61), which the reference
 * runs on the CPU only (tools/quantize.cpp:30-49).  Writes q, scales and (int4)
 * zeros in the layout above.  int4 needs even cols (as the reference). */
int iq_quantize(const uint16_t* w_bf16, int64_t rows, int64_t cols, int kind, uint8_t* q,
                uint16_t* scales, uint8_t* zeros, void* stream);

/* ---------------------------------------------------------------- chains
 * A chain is a program of dependent GEMV stages of 1..32 activation rows:
 * the quantised linears of a (batched) decode step in the order of
 * GpuBatch::Impl::launch_sequence (kernels/batch_gpu.cu:186-215), each
 * stage reading what earlier stages wrote, with the elementwise work
 * between them fused into the stages.  A run is one launch per 1-row stage
 * and two per B-row stage (the GEMV with the input transform, then the
 * K-range sums with the output transform), on one stream, capturable into
 * a HIP graph.  No reference counterpart as an entry point: the reference
 * issues launch_gemv_batched_q, launch_rmsnorm, launch_swiglu and
 * launch_residual_add separately.
 *
 * Stage = y_i = f_out( dequant(W_i) . f_in(x) + bias_i ), i < n <= 3, all W_i
 * of one kind and width K (K % 256 == 0; 1 row: int4 K <= 24576, int8
 * K <= 20480, halved for IQ_OUT_SWIGLU), x 16-byte aligned, for each of
 * the stage's `rows` activation rows B (1..32; 0 means 1): x is [B][K]
 * ([B][K / group] for IQ_IN_GQA), residual and every y_i [B][W_i->rows],
 * row-major, each row transformed on its own (RMSNorm per row):
 *   f_in   IQ_IN_PLAIN    x[k]
 *          IQ_IN_RMSNORM  x[k] / sqrt(mean(x^2) + eps) * norm[k], norm bf16
 *                         (src/forward.cpp:21-31); K <= 16384
 *          IQ_IN_GQA      x[(k / (head_dim * group)) * head_dim + k % head_dim]:
 *                         the attention output of a sequence of one token,
 *                         whose softmax over its single key is 1, so every
 *                         query head receives the value row of its key/value
 *                         head (x = v, K / group values)
 *   f_out  IQ_OUT_STORE     y_i[o] = acc + bias_i[o]
 *          IQ_OUT_RESIDUAL  y_0[o] = residual[o] + (acc + bias_0[o])  (n == 1)
 *          IQ_OUT_SWIGLU    y_0[o] = silu(acc_0 + b_0) * (acc_1 + b_1), n == 2
 *                           (gate, up; kernels/ops/elementwise.cu:6-11)
 * A stage's outputs may not overlap its own inputs (IQ_EALIAS).  Outputs
 * are fp32 vectors of W_i->rows. */
enum { IQ_IN_PLAIN = 0, IQ_IN_RMSNORM = 1, IQ_IN_GQA = 2 };
enum { IQ_OUT_STORE = 0, IQ_OUT_RESIDUAL = 1, IQ_OUT_SWIGLU = 2 };

typedef struct iq_stage {
    int32_t in_op, out_op, n;
    int32_t gqa_head_dim, gqa_group;  /* IQ_IN_GQA */
    float eps;                        /* IQ_IN_RMSNORM */
    const float* x;
    const uint16_t* norm;             /* IQ_IN_RMSNORM: bf16 [K], 16-byte aligned */
    const float* residual;            /* IQ_OUT_RESIDUAL: [rows] */
    iq_view W[3];
    const uint16_t* bias[3];          /* bf16 or NULL */
    float* y[3];                      /* IQ_OUT_SWIGLU: y[0] only */
    int32_t rows;                     /* activation rows B, 1..32 (0: 1) */
} iq_stage;

typedef struct iq_chain iq_chain;

/* Validates the n stages and records their launch shapes for the current
 * device.  The chain allocates its own device buffers here: the sums of
 * squares passed from a stage to a later RMSNorm stage (a float per 16-row
 * tile, or per row and tile / 256-column block with rows > 1), and for
 * stages with rows > 1 the K-range partial sums of the rows GEMV and the
 * prepared f16 operands of narrow stages (5..16 rows: G * 8 KiB).  So
 * create a chain outside graph capture, in code that may allocate;
 * iq_chain_destroy frees them.  iq_chain_run allocates nothing. */
int iq_chain_create(const iq_stage* stages, int n, iq_chain** out);
/* Enqueues one run of the whole program on `stream`. */
int iq_chain_run(const iq_chain* chain, void* stream);
void iq_chain_destroy(iq_chain* chain);

/* Reserve the workspace of (device, null stream) (done lazily by the first
 * call that needs it).  Call before capturing a graph.  Returns 0 or an
 * error code. */
int iq_init(int device);

/* Reserve the workspace of (device, stream): call before capturing a graph
 * on a stream other than the null stream, since capture forbids the
 * allocation.  Library set-up, no reference counterpart (the reference's
 * launchers keep no workspace). */
int iq_init_stream(int device, void* stream);

/* Static description of an error code (never NULL). */
const char* iq_error_string(int code);

/* Library version string. */
const char* iq_version(void);

#ifdef __cplusplus
}
#endif

#endif /* IQ_H */

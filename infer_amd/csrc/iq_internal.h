// iq_internal.h -- declarations shared by the HIP translation units of
// libiq.so (kernel launchers and the per-device workspace).  Not installed;
// the public boundary is include/iq.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "iq_device.h"

namespace iq {

// Kernel-argument copy of iq_view / gpu::QuantView (kernels/ops/ops.cuh:166-172).
struct QView {
    int32_t kind;  // 0 int8, 1 int4
    int64_t rows, cols, groups;
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
};

// Per-device scratch used by the GEMV: a copy of a prepared 1-row
// activation, the activations as byte limbs with their per-(group, row)
// exponent and limb sums, and split-K partial sums.
struct Workspace {
    void* base = nullptr;
    size_t bytes = 0;
    float* xf = nullptr;       // [4][kMaxKp] fp32: 1..4 activation rows copied by a prep
    int8_t* xq = nullptr;      // [kMaxRowsGemv][kMaxKp/128][4*128] limbs, or the f16 hi/lo
                               // A operands [kMaxRowsGemv/16][kMaxKp/128][8 KiB] (gemvh)
    int4* xmeta = nullptr;     // [kMaxKp/128][kMaxRowsGemv] {2^-k, 256 sum X0 + sum X1, 256 sum X2 + sum X3, 0}
    float* partials = nullptr; // part_floats (>= kPartialFloats)
    int64_t part_floats = 0;   // capacity of partials
    size_t xq_bytes = 0, xmeta_bytes = 0;
    // the prefill GEMM's prepared activations (kGemmOperandBytes, reserved
    // with the workspace; null in the static workspace)
    void* gx = nullptr;
    size_t gx_bytes = 0;
    // Shape of the activations last prepared into xq/xmeta (host-side record).
    int prep_M = 0;
    int64_t prep_K = 0;
    int prep_kind = -1;
    bool prep_copy = false;   // the preparation is a copy of x in xf (1..4 rows)
    bool prep_h = false;      // the preparation is the f16 hi/lo split for gemvh (xq, xmeta)
    // Forget the preparation (its buffers were reused by a direct call).
    void invalidate_prep() {
        prep_M = 0;
        prep_K = 0;
        prep_kind = -1;
        prep_copy = false;
        prep_h = false;
    }
};

constexpr int kMaxRowsGemv = 32;            // GpuBatch::kMaxRows (kernels/batch_gpu.h:80)
constexpr int64_t kMaxKp = 131072;          // padded K limit of the GEMV
constexpr int64_t kPartialFloats = int64_t(4) << 20;  // 16 MiB of split-K partials (every workspace)
constexpr int64_t kStreamPartialFloats = int64_t(16) << 20;  // 64 MiB in a per-stream workspace
// The fp32-activation prefill GEMM's prepared operands (fp16 hi + lo, 4 B
// per value): 1024 rows of 7B down's 18944 columns in one pass, longer
// prefills in row chunks (at the 131072-column limit, 128 rows a chunk).
constexpr size_t kGemmOperandBytes = size_t(80) << 20;

// Returns the workspace of (current device, stream), allocating it on first
// use.  Every stream has its own, so calls on different streams never share
// activation or partial-sum buffers; calls on one stream are ordered by it.
hipError_t get_workspace(hipStream_t stream, Workspace** ws);
// The workspace of iq_gemv_noalloc on the current device: views into the
// library's static device array (no allocation; shared by every call on
// the device).
hipError_t static_workspace(Workspace** ws);

hipError_t launch_quantize(const uint16_t* w, int64_t rows, int64_t cols, int kind, uint8_t* q,
                           uint16_t* scales, uint8_t* zeros, hipStream_t stream);
hipError_t launch_embedding(const QView& t, const int64_t* ids, int64_t T, int64_t H, float* out,
                            hipStream_t stream);
hipError_t launch_gemv(const float* x, const QView& W, const uint16_t* bias, int M, float* y,
                       Workspace* ws, hipStream_t stream);
hipError_t launch_xprep(const float* x, int M, int64_t K, int kind, Workspace* ws, hipStream_t stream);
hipError_t launch_gemv_prepped(const QView& W, const uint16_t* bias, int M, float* y, Workspace* ws,
                               hipStream_t stream);
// Several matrices of one kind and width on the same prepared activations
// (n <= 4): one launch for 1 row, one launch per matrix otherwise.
hipError_t launch_gemv_prepped_multi(const QView* W, const uint16_t* const* bias, float* const* y, int n,
                                     int M, Workspace* ws, hipStream_t stream);
// Several matrices of one kind and width on the activations x [M][K]
// (n <= 4): the 1-row kernel reads x itself (one launch for all n); other
// shapes prepare x once into the workspace, then one launch per matrix.
hipError_t launch_gemv_multi(const float* x, const QView* W, const uint16_t* const* bias, float* const* y,
                             int n, int M, Workspace* ws, hipStream_t stream);
// Uses the workspace for the prepared fp16 activations and the split-K
// partials (short T splits K over workgroups).
// 17..32 activation rows (fp32) on gemvq's two 16-row blocks, the f16
// split made in the kernel, where that beats the GEMM's tiles (wide or
// long-K matrices); false: not applicable, nothing launched.
bool launch_gemm_rows(const float* x, const QView& W, const uint16_t* bias, int64_t T, float* y, Workspace* ws,
                      hipStream_t stream, hipError_t* err);
hipError_t launch_gemm(const float* x_f32, const uint16_t* x_bf16, const QView& W,
                       const uint16_t* bias, int64_t T, float* y, Workspace* ws, hipStream_t stream);
// The prefill GEMM's prepared activations for T rows of K columns: fp16
// hi (and lo) [T][K] and T row factors, in the workspace's operand area
// (hipErrorInvalidValue when they do not fit: callers split T into chunks
// of at most gemm_operand_rows(ws, K) rows, a multiple of 128).
hipError_t gemm_operands(Workspace* ws, int64_t T, int64_t K, bool lo, _Float16** ah, float** rs);
int64_t gemm_operand_rows(const Workspace* ws, int64_t K);

// Activations of a B-row chain stage: row m, column c is x[m xstride + c]
// (gqa_span > 0: the value row of c's key/value head, x[m xstride +
// (c / gqa_span) gqa_hd + c % gqa_hd]), RMSNorm'd when norm is set, with
// row m's factor from the ssq_n partial sums of squares ssq[m][0 .. ssq_n).
struct RowsIn {
    const float* x;
    int64_t xstride;
    int gqa_hd, gqa_span;
    const uint16_t* norm;
    const float* ssq;
    int ssq_n;
    float eps;
};
// The rows GEMV of a chain stage on n <= 4 matrices sharing K and kind
// (M in 1..32): every K range's sums into part [S][M][tiles * 16] (16-row
// tiles of the matrices in order), S returned.  chain_rows_partials gives
// the floats that needs for a capacity `cap` (-1: shape not covered).
int64_t chain_rows_partials(const QView* W, int n, int M, int64_t cap);
hipError_t launch_chain_rows(const QView* W, int n, int M, const RowsIn& in, float* part, int64_t part_floats,
                             int* S, hipStream_t stream);
// A narrow chain stage at 5..16 rows (under 1024 tiles, G < 128): the
// input transform into f16 hi / lo operands at xq / xmeta (one 16-row
// block: G * 8 KiB and G * 64 bytes), then gemvh storing y = (res +) sum +
// bias and, when ssq_out, the sum of squares of each 16-column tile of each
// row (ssq_out[m * tiles + tile]).
bool chain_h_applies(const QView* W, int n, int M);
void chain_h_bytes(int64_t G, int M, size_t* xq_bytes, size_t* meta_floats);
hipError_t launch_chain_h(const QView* W, int n, int M, const RowsIn& in, const uint16_t* const* bias,
                          float* const* y, const float* res, float* ssq_out, int8_t* xq, float* xmeta,
                          hipStream_t stream);

// A validated stage program on the device (iq_chain.hip).
struct Chain;
void chain_destroy(Chain* ch);

// Lets kernel F take up to 160 KiB of LDS (gfx950's LDS per CU) in static
// plus dynamic allocations; once per kernel instance and process.  A failed
// attribute call is cleared from the runtime's last-error slot (a launch
// past the default limit then reports its own error).
template <auto F>
inline void allow_big_lds() {
    static const bool once = [] {
        const void* f = reinterpret_cast<const void*>(F);
        hipFuncAttributes a{};
        size_t stat = 0;
        if (hipFuncGetAttributes(&a, f) == hipSuccess) stat = a.sharedSizeBytes;
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, int(160 * 1024 - stat)) != hipSuccess)
            (void)hipGetLastError();
        return true;
    }();
    (void)once;
}

// Device properties used by the dispatch heuristics.
int device_cu_count();

}  // namespace iq

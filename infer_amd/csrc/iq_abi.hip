// iq_abi.hip -- the extern "C" boundary (include/iq.h): argument validation,
// the per-device workspace, and dispatch to the gfx950 kernels.
//
// Validation mirrors what the reference rejects on the host
// (src/quant.cpp:35-36 kind / odd int4 cols; src/quant.cpp:204-205 shape
// mismatch) and adds the checks a C boundary needs (null pointers, sizes the
// kernels assume).  Nothing is enqueued when a check fails.
#include <map>
#include <mutex>
#include <utility>

#include "../../include/iq.h"
#include "iq_internal.h"

namespace iq {

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
// One workspace per (device, stream); entries live until the process ends
// (a stream handle that is destroyed and reused maps to the same buffers,
// which is safe because work on a destroyed stream has completed).
std::map<std::pair<int, hipStream_t>, Workspace*> g_ws;
int g_cus[kMaxDevices];

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

hipError_t create_workspace(Workspace* ws) {
    const int64_t gmax = kMaxKp / kGroup;
    const size_t xf = align256(sizeof(float) * 4 * kMaxKp);  // up to 4 rows copied by a prep
    // limbs or f16 hi + lo (4 B per value)
    const size_t xq = align256(size_t(kMaxRowsGemv) * gmax * 4 * kGroup);
    const size_t meta = align256(sizeof(int4) * gmax * kMaxRowsGemv);
    const size_t part = align256(sizeof(float) * kStreamPartialFloats);
    const size_t gx = align256(kGemmOperandBytes);
    const size_t total = xf + xq + meta + part + gx;
    void* base = nullptr;
    hipError_t e = hipMalloc(&base, total);
    if (e != hipSuccess) return e;
    char* p = static_cast<char*>(base);
    ws->base = base;
    ws->bytes = total;
    ws->xf = reinterpret_cast<float*>(p);
    ws->xq = reinterpret_cast<int8_t*>(p + xf);
    ws->xmeta = reinterpret_cast<int4*>(p + xf + xq);
    ws->partials = reinterpret_cast<float*>(p + xf + xq + meta);
    ws->part_floats = kStreamPartialFloats;
    ws->xq_bytes = xq;
    ws->xmeta_bytes = meta;
    ws->gx = p + xf + xq + meta + part;
    ws->gx_bytes = gx;
    return hipSuccess;
}

// Workspace sizes of iq_gemv_noalloc: activations of up to kStaticMaxK
// columns x 32 rows, and the same split-K partial-sum capacity as a
// workspace of get_workspace().
constexpr int64_t kStaticMaxK = 32768;
constexpr size_t kStaticXq = size_t(kMaxRowsGemv) * (kStaticMaxK / kGroup) * 4 * kGroup;  // 4 MiB
constexpr size_t kStaticMeta = sizeof(int4) * (kStaticMaxK / kGroup) * kMaxRowsGemv;       // 128 KiB
constexpr size_t kStaticPart = sizeof(float) * kPartialFloats;                              // 16 MiB
constexpr size_t kStaticBytes = kStaticXq + kStaticMeta + kStaticPart;

}  // namespace
}  // namespace iq

// The scratch of iq_gemv_noalloc: part of the code object, so every device
// the library runs on holds its own copy until the process ends.  Host code
// never passes `scratch` itself to a kernel (on the host it is only a
// stand-in symbol): it uses the device address that hipGetSymbolAddress
// returns for the current device (static_workspace below).
static __device__ __align__(256) unsigned char scratch[iq::kStaticBytes];

namespace iq {
namespace {

Workspace g_static_ws[kMaxDevices];
bool g_static_ready[kMaxDevices];

}  // namespace

hipError_t static_workspace(Workspace** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_static_ready[dev]) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!ptr) return hipErrorInvalidSymbol;
        char* p = static_cast<char*>(ptr);
        Workspace& w = g_static_ws[dev];
        w.base = ptr;
        w.bytes = kStaticBytes;
        w.xf = nullptr;  // no preparation API on this workspace
        w.xq = reinterpret_cast<int8_t*>(p);
        w.xmeta = reinterpret_cast<int4*>(p + kStaticXq);
        w.partials = reinterpret_cast<float*>(p + kStaticXq + kStaticMeta);
        w.part_floats = kPartialFloats;
        w.xq_bytes = kStaticXq;
        w.xmeta_bytes = kStaticMeta;
        g_static_ready[dev] = true;
    }
    *out = &g_static_ws[dev];
    return hipSuccess;
}

hipError_t get_workspace(hipStream_t stream, Workspace** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lk(g_mu);
    const auto key = std::make_pair(dev, stream);
    if (!g_ws.count(key) && stream) {
        // A stream under graph capture cannot allocate, and sharing another
        // stream's workspace would race with that stream's calls: it needs
        // its own, made by iq_init_stream before the capture.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
            return hipErrorStreamCaptureUnsupported;
    }
    Workspace*& ws = g_ws[key];
    if (!ws) {
        Workspace* w = new Workspace();
        e = create_workspace(w);
        if (e != hipSuccess) {
            delete w;
            g_ws.erase(std::make_pair(dev, stream));
            return e;
        }
        ws = w;
    }
    *out = ws;
    return hipSuccess;
}

int64_t gemm_operand_rows(const Workspace* ws, int64_t K) {
    // hi + lo fp16 (4 B per value) and one fp32 row factor per row
    const int64_t rows = int64_t(ws->gx_bytes) / (4 * K + 4 + 256);
    return rows / 128 * 128;
}

hipError_t gemm_operands(Workspace* ws, int64_t T, int64_t K, bool lo, _Float16** ah, float** rs) {
    const size_t op = size_t(T) * size_t(K) * 2 * (lo ? 2 : 1);
    const size_t need = align256(op) + align256(sizeof(float) * size_t(T));
    if (!ws->gx || need > ws->gx_bytes) return hipErrorInvalidValue;
    *ah = static_cast<_Float16*>(ws->gx);
    *rs = reinterpret_cast<float*>(static_cast<char*>(ws->gx) + align256(op));
    return hipSuccess;
}

int device_cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
    int v = __atomic_load_n(&g_cus[dev], __ATOMIC_RELAXED);
    if (v > 0) return v;
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    __atomic_store_n(&g_cus[dev], cus, __ATOMIC_RELAXED);
    return cus;
}

}  // namespace iq

namespace {

int from_hip(hipError_t e) { return e == hipSuccess ? IQ_OK : int(e); }

// Status of a workspace request: allocation failure is IQ_ENOMEM.
int ws_status(hipError_t e) { return e == hipErrorOutOfMemory ? IQ_ENOMEM : from_hip(e); }

// Shared view checks; `in`/`out` must match the matrix (quant.cpp:204-205).
int check_view(const iq_view* W, int64_t in, int64_t out) {
    if (!W) return IQ_ENULL;
    if (W->kind != IQ_INT8 && W->kind != IQ_INT4) return IQ_EKIND;
    if (W->rows <= 0 || W->cols <= 0) return IQ_ESHAPE;
    if (W->groups != (W->cols + IQ_GROUP - 1) / IQ_GROUP) return IQ_ESHAPE;
    if (in != W->cols || out != W->rows) return IQ_ESHAPE;
    if (W->kind == IQ_INT4 && (W->cols % 2)) return IQ_ESHAPE;
    if (!W->q || !W->scales) return IQ_ENULL;
    if (W->kind == IQ_INT4 && !W->zeros) return IQ_ENULL;
    return IQ_OK;
}

iq::QView to_qview(const iq_view* W) {
    iq::QView v;
    v.kind = W->kind;
    v.rows = W->rows;
    v.cols = W->cols;
    v.groups = W->groups;
    v.q = W->q;
    v.scales = W->scales;
    v.zeros = W->kind == IQ_INT4 ? W->zeros : nullptr;
    return v;
}

}  // namespace

extern "C" {

int iq_init_stream(int device, void* stream) {
    int cur = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return from_hip(e);
    if (device != cur) {
        e = hipSetDevice(device);
        if (e != hipSuccess) return from_hip(e);
    }
    iq::Workspace* ws = nullptr;
    e = iq::get_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e == hipSuccess) e = iq::static_workspace(&ws);  // iq_gemv_noalloc's scratch address
    (void)iq::device_cu_count();
    if (device != cur) (void)hipSetDevice(cur);
    return ws_status(e);
}

int iq_init(int device) { return iq_init_stream(device, nullptr); }

int iq_gemv(const float* x, const iq_view* W, const uint16_t* bias, int B, int64_t in, int64_t out,
            float* y, void* stream) {
    int rc = check_view(W, in, out);
    if (rc) return rc;
    if (!x || !y) return IQ_ENULL;
    if (B < 1 || B > iq::kMaxRowsGemv) return IQ_ESHAPE;
    if (W->groups * IQ_GROUP > iq::kMaxKp) return IQ_ETOOLARGE;
    iq::Workspace* ws = nullptr;
    hipError_t e = iq::get_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return ws_status(e);
    return from_hip(iq::launch_gemv(x, to_qview(W), bias, B, y, ws, static_cast<hipStream_t>(stream)));
}

int iq_gemv_noalloc(const float* x, const iq_view* W, const uint16_t* bias, int B, int64_t in, int64_t out,
                    float* y, void* stream) {
    int rc = check_view(W, in, out);
    if (rc) return rc;
    if (!x || !y) return IQ_ENULL;
    if (B < 1 || B > iq::kMaxRowsGemv) return IQ_ESHAPE;
    if (W->groups * IQ_GROUP > iq::kStaticMaxK) return IQ_ETOOLARGE;
    iq::Workspace* ws = nullptr;
    const hipError_t e = iq::static_workspace(&ws);
    if (e != hipSuccess) return from_hip(e);
    return from_hip(iq::launch_gemv(x, to_qview(W), bias, B, y, ws, static_cast<hipStream_t>(stream)));
}

int iq_gemv_prep(const float* x, int B, int64_t in, int kind, void* stream) {
    if (kind != IQ_INT8 && kind != IQ_INT4) return IQ_EKIND;
    if (!x) return IQ_ENULL;
    if (B < 1 || B > iq::kMaxRowsGemv || in < 1) return IQ_ESHAPE;
    if (kind == IQ_INT4 && (in % 2)) return IQ_ESHAPE;
    if ((in + IQ_GROUP - 1) / IQ_GROUP * IQ_GROUP > iq::kMaxKp) return IQ_ETOOLARGE;
    iq::Workspace* ws = nullptr;
    hipError_t e = iq::get_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return ws_status(e);
    return from_hip(iq::launch_xprep(x, B, in, kind, ws, static_cast<hipStream_t>(stream)));
}

int iq_gemv_prepped(const iq_view* W, const uint16_t* bias, int B, int64_t in, int64_t out,
                    float* y, void* stream) {
    int rc = check_view(W, in, out);
    if (rc) return rc;
    if (!y) return IQ_ENULL;
    iq::Workspace* ws = nullptr;
    hipError_t e = iq::get_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return ws_status(e);
    if (B != ws->prep_M || in != ws->prep_K || W->kind != ws->prep_kind) return IQ_ESHAPE;
    return from_hip(iq::launch_gemv_prepped(to_qview(W), bias, B, y, ws, static_cast<hipStream_t>(stream)));
}

namespace {

// Validates n <= 4 matrices of one kind and width `in` and unpacks them.
int gather_views(const iq_view* const* Ws, int n, const uint16_t* const* biases, int64_t in,
                 float* const* ys, iq::QView* v, const uint16_t** b, float** y) {
    if (n < 1 || n > 4) return IQ_ESHAPE;
    if (!Ws || !ys) return IQ_ENULL;
    for (int i = 0; i < n; i++) {
        if (!Ws[i]) return IQ_ENULL;
        const int rc = check_view(Ws[i], in, Ws[i]->rows);
        if (rc) return rc;
        if (Ws[i]->kind != Ws[0]->kind) return IQ_EKIND;
        if (!ys[i]) return IQ_ENULL;
        v[i] = to_qview(Ws[i]);
        b[i] = biases ? biases[i] : nullptr;
        y[i] = ys[i];
    }
    return IQ_OK;
}

}  // namespace

int iq_gemv_prepped_multi(const iq_view* const* Ws, int n, const uint16_t* const* biases, int B,
                          int64_t in, float* const* ys, void* stream) {
    iq::QView v[4];
    const uint16_t* b[4];
    float* y[4];
    const int rc = gather_views(Ws, n, biases, in, ys, v, b, y);
    if (rc) return rc;
    iq::Workspace* ws = nullptr;
    hipError_t e = iq::get_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return ws_status(e);
    if (B != ws->prep_M || in != ws->prep_K || Ws[0]->kind != ws->prep_kind) return IQ_ESHAPE;
    return from_hip(iq::launch_gemv_prepped_multi(v, b, y, n, B, ws, static_cast<hipStream_t>(stream)));
}

int iq_gemv_multi(const float* x, const iq_view* const* Ws, int n, const uint16_t* const* biases, int B,
                  int64_t in, float* const* ys, void* stream) {
    iq::QView v[4];
    const uint16_t* b[4];
    float* y[4];
    const int rc = gather_views(Ws, n, biases, in, ys, v, b, y);
    if (rc) return rc;
    if (!x) return IQ_ENULL;
    if (B < 1 || B > iq::kMaxRowsGemv) return IQ_ESHAPE;
    if (Ws[0]->groups * IQ_GROUP > iq::kMaxKp) return IQ_ETOOLARGE;
    iq::Workspace* ws = nullptr;
    hipError_t e = iq::get_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return ws_status(e);
    return from_hip(iq::launch_gemv_multi(x, v, b, y, n, B, ws, static_cast<hipStream_t>(stream)));
}

int iq_gemm(const float* x, const iq_view* W, const uint16_t* bias, int64_t T, int64_t in,
            int64_t out, float* y, void* stream) {
    int rc = check_view(W, in, out);
    if (rc) return rc;
    if (!x || !y) return IQ_ENULL;
    if (T < 1) return IQ_ESHAPE;
    if ((T + 127) / 128 * ((out + 127) / 128) > 0x7fffffff) return IQ_ETOOLARGE;
    iq::Workspace* ws = nullptr;
    const hipError_t e = iq::get_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return ws_status(e);
    return from_hip(iq::launch_gemm(x, nullptr, to_qview(W), bias, T, y, ws, static_cast<hipStream_t>(stream)));
}

int iq_gemm_bf16x(const uint16_t* x, const iq_view* W, const uint16_t* bias, int64_t T,
                  int64_t in, int64_t out, float* y, void* stream) {
    int rc = check_view(W, in, out);
    if (rc) return rc;
    if (!x || !y) return IQ_ENULL;
    if (T < 1) return IQ_ESHAPE;
    if ((T + 127) / 128 * ((out + 127) / 128) > 0x7fffffff) return IQ_ETOOLARGE;
    iq::Workspace* ws = nullptr;
    const hipError_t e = iq::get_workspace(static_cast<hipStream_t>(stream), &ws);
    if (e != hipSuccess) return ws_status(e);
    return from_hip(iq::launch_gemm(nullptr, x, to_qview(W), bias, T, y, ws, static_cast<hipStream_t>(stream)));
}

int iq_linear(const float* x, const iq_view* W, const uint16_t* bias, int64_t T, int64_t in,
              int64_t out, float* y, void* stream) {
    if (T >= 1 && T <= iq::kMaxRowsGemv) return iq_gemv(x, W, bias, int(T), in, out, y, stream);
    return iq_gemm(x, W, bias, T, in, out, y, stream);
}

int iq_embedding(const iq_view* table, const int64_t* ids, int64_t T, int64_t H, float* out,
                 void* stream) {
    if (!table) return IQ_ENULL;
    int rc = check_view(table, H, table->rows);
    if (rc) return rc;
    if (!ids || !out) return IQ_ENULL;
    if (T < 1) return IQ_ESHAPE;
    return from_hip(iq::launch_embedding(to_qview(table), ids, T, H, out, static_cast<hipStream_t>(stream)));
}

int iq_quantize(const uint16_t* w_bf16, int64_t rows, int64_t cols, int kind, uint8_t* q,
                uint16_t* scales, uint8_t* zeros, void* stream) {
    if (kind != IQ_INT8 && kind != IQ_INT4) return IQ_EKIND;
    if (rows <= 0 || cols <= 0) return IQ_ESHAPE;
    if (kind == IQ_INT4 && (cols % 2)) return IQ_ESHAPE;
    if (!w_bf16 || !q || !scales || (kind == IQ_INT4 && !zeros)) return IQ_ENULL;
    const int64_t waves = rows * (((cols + IQ_GROUP - 1) / IQ_GROUP + 3) / 4);
    if ((waves + 3) / 4 > 0x7fffffff) return IQ_ETOOLARGE;
    return from_hip(iq::launch_quantize(w_bf16, rows, cols, kind, q, scales, zeros, static_cast<hipStream_t>(stream)));
}

const char* iq_error_string(int code) {
    switch (code) {
        case IQ_OK: return "ok";
        case IQ_EKIND: return "iq: quant kind must be IQ_INT8 (0) or IQ_INT4 (1)";
        case IQ_ESHAPE: return "iq: inconsistent or unsupported shape";
        case IQ_ENULL: return "iq: required pointer is NULL";
        case IQ_ETOOLARGE: return "iq: problem exceeds workspace limits";
        case IQ_ENOMEM: return "iq: workspace allocation failed";
        case IQ_EDEVICE: return "iq: no usable device (or not the device the chain was made on)";
        case IQ_EALIAS: return "iq: a chain stage's output overlaps its input";
        default: break;
    }
    if (code > 0) return hipGetErrorString(static_cast<hipError_t>(code));
    return "iq: unknown error";
}

const char* iq_version(void) { return "iq 0.1 gfx950"; }

}  // extern "C"

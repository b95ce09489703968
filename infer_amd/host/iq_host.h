// iq_host.h -- C++ host side of the MI355X quantised-weight matrix path.
//
// The reference's own C++ surface for this path, kept so that its callers
// drop in: the packed layout and container (src/quant.h:34-115: QKind,
// QTensor, QMatrix, QuantWriter, QuantFile, QuantModel), the model config
// it needs (src/model_config.h), and the device launchers with their
// QuantView (kernels/ops/ops.cuh:165-178).  Everything on the device goes
// through the C ABI of include/iq.h; this layer adds ownership, the .llmq
// file format and C++ error handling (std::runtime_error where the reference
// throws at load time or exits at the next CUDA_CHECK).
//
// Differences from the reference, each deliberate:
//   * quantize() runs on the GPU (iq_quantize), bit-exact to the reference's
//     CPU quantiser; it throws when no gfx950 device is usable.
//   * bias pointers are bf16 bits (const uint16_t*), not __nv_bfloat16.
//   * launchers take an optional stream (default: the null stream).
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "iq.h"

namespace llm {

constexpr int kGroup = IQ_GROUP;  // src/quant.h:34

enum class QKind { kBf16, kInt8, kInt4 };  // src/quant.h:36
const char* qkind_name(QKind k);

// Non-owning view of one packed matrix or bf16 vector (src/quant.h:40-49).
// Pointer sizes: codes q_bytes(); scales and (int4) zero points
// rows x groups() entries each; bf16 holds rows x cols values when kind is
// kBf16 (the layer norms and the attention biases) and is null otherwise.
struct QTensor {
    QKind kind = QKind::kBf16;
    int64_t rows = 0, cols = 0;
    const uint8_t* q = nullptr;
    const uint16_t* scales = nullptr;
    const uint8_t* zeros = nullptr;
    const uint16_t* bf16 = nullptr;
    int64_t groups() const { return (cols + kGroup - 1) / kGroup; }
    size_t q_bytes() const { return kind == QKind::kInt4 ? size_t(rows) * cols / 2 : size_t(rows) * cols; }
};

// A packed matrix that owns its bytes, e.g. what quantize() returns
// (src/quant.h:52-58).
struct QMatrix {
    QKind kind = QKind::kInt8;
    int64_t rows = 0, cols = 0;
    std::vector<uint8_t> q, zeros;
    std::vector<uint16_t> scales;
    QTensor view() const;
};

// Packs a host bf16 matrix [rows x cols] with the GPU quantiser; the bytes
// equal the reference's CPU quantiser's (src/quant.h:61).  int4 requires an
// even column count.
QMatrix quantize(const uint16_t* w_bf16, int64_t rows, int64_t cols, QKind kind);
// s * q (int8) or s * (q - z) (int4) of element (r, c): the value every
// kernel multiplies by (src/quant.h:63, src/quant.cpp:86-93).
float dequant(const QTensor& t, int64_t r, int64_t c);

// .llmq writer (src/quant.h:66-77): 8-byte magic "LLMQ0001", u64 header
// length, a JSON header {name: {dtype, shape, group, data, scales?, zeros?}}
// of [begin, end) byte ranges into the blob that follows, then the blob in
// insertion order (q, scales, zeros per matrix; the data of a bf16 tensor).
class QuantWriter {
public:
    void add(const std::string& name, const QMatrix& m);
    void add_bf16(const std::string& name, const uint16_t* data, std::vector<int64_t> shape);
    void write(const std::string& path) const;
    // The bytes write() would put in the file.
    std::vector<uint8_t> serialize() const;

private:
    struct Entry {
        std::string name;
        QKind kind;
        std::vector<int64_t> shape;
        std::vector<uint8_t> q, zeros;
        std::vector<uint16_t> scales;  // bf16 payload of a kBf16 entry
    };
    std::vector<Entry> entries_;
};

// .llmq reader (src/quant.h:80-96).  open() maps the file read-only and
// indexes its header; the QTensor views point into the mapping, so they are
// valid until the next open() or the destructor.  A file that fails
// validation throws and leaves the previously opened file in place.
class QuantFile {
public:
    QuantFile() = default;
    ~QuantFile();
    QuantFile(const QuantFile&) = delete;
    QuantFile& operator=(const QuantFile&) = delete;
    void open(const std::string& path);
    bool has(const std::string& name) const { return tensors_.count(name) > 0; }
    const QTensor& get(const std::string& name) const;
    std::vector<std::string> names() const;          // sorted
    std::vector<std::string> names_in_file() const;  // in blob (write) order
    QKind kind() const { return kind_; }             // kind of the packed matrices

private:
    void* map_ = nullptr;
    size_t map_size_ = 0;
    std::map<std::string, QTensor> tensors_;
    std::map<std::string, size_t> offset_;  // blob offset of each tensor's first payload
    QKind kind_ = QKind::kBf16;
};

// The config.json fields the quantised path reads (src/model_config.h).
struct ModelConfig {
    std::string architecture;
    int64_t hidden_size = 0, num_hidden_layers = 0, num_attention_heads = 0, num_key_value_heads = 0,
            intermediate_size = 0, vocab_size = 0, head_dim = 0;
    double rope_theta = 0, rms_norm_eps = 0;
    bool tie_word_embeddings = false, attention_bias = false;
    static ModelConfig from_file(const std::string& path);
};

// The views of one decoder layer.  Without attention biases the three bias
// views stay empty (rows == 0).
struct QLayer {
    QTensor q_w, k_w, v_w, o_w, gate_w, up_w, down_w;
    QTensor q_b, k_b, v_b;
    QTensor input_ln, post_attn_ln;
    bool has_bias = false;
};
// Every tensor of a quantised model, as views into its .llmq file, which the
// model keeps open (src/quant.h:99-115).  With tied embeddings lm_head is
// empty and embed_tokens doubles as the output projection.
struct QuantModel {
    ModelConfig cfg;
    QTensor embed_tokens;
    QTensor lm_head;
    QTensor final_norm;
    std::vector<QLayer> layers;
    QKind kind = QKind::kInt8;
    // Reads model_dir/config.json, then the int8 or int4 container that
    // file_for() names, checking every tensor's kind and shape against the
    // config.
    void load(const std::string& model_dir, QKind kind);
    static std::string file_for(const std::string& model_dir, QKind kind);

private:
    QuantFile file_;
};

// A bf16 tensor of a model held in host memory (a source for quantize_model).
struct BF16Tensor {
    const uint16_t* data = nullptr;
    std::vector<int64_t> shape;
};

// What quantize_model reports (tools/quantize.cpp:76-81): bytes before and
// after, the worst per-group error |w - dequant(w)| as a fraction of the
// group's absmax over sampled rows (every rows / 64-th row, every group),
// and the wall time.
struct QuantizeReport {
    size_t bytes_in = 0, bytes_out = 0;
    double worst = 0.0;
    double seconds = 0.0;
    int matrices = 0, vectors = 0;
};

// The offline quantiser's loop (tools/quantize.cpp:30-73) with the packing on
// the GPU: every linear matrix and the embedding table of the model `src`
// holds (names as in the reference's files; `cfg` gives the layer count) is
// quantised to `kind` by iq_quantize, bit-exact to the reference's CPU
// quantiser, and added to `w` with the norms and biases copied as bf16, in
// the reference's order (embedding, lm_head when present, final norm, then
// per layer q, k, v, o, gate, up, down, the two norms, the q/k/v biases when
// present), so w.write() produces the reference's .llmq file byte for byte.
// Missing required tensors throw.  One device staging buffer, reused.
QuantizeReport quantize_model(const std::map<std::string, BF16Tensor>& src, const ModelConfig& cfg, QKind kind,
                              QuantWriter& w);

namespace gpu {

// kernels/ops/ops.cuh:165-172; byte-compatible with iq_view.
enum class QuantKind { kInt8, kInt4 };
struct QuantView {
    QuantKind kind;
    int64_t rows, cols, groups;
    const uint8_t* q;
    const uint16_t* scales;
    const uint8_t* zeros;
};

// kernels/ops/ops.cuh:173-178.  Enqueue on `stream` without synchronising;
// a rejected call or a runtime error throws std::runtime_error.
void launch_gemv_batched_q(const float* x, const QuantView& W, const uint16_t* bias, int B, int64_t in,
                           int64_t out, float* y, hipStream_t stream = nullptr);
void launch_gemm_tiled_q(const float* x, const QuantView& W, const uint16_t* bias, int64_t T, int64_t in,
                         int64_t out, float* y, hipStream_t stream = nullptr);
void launch_embedding_q(const QuantView& table, const int64_t* ids, int64_t T, int64_t H, float* out,
                        hipStream_t stream = nullptr);
// The quantised linear call site, GpuBatch::Impl::linear_b
// (kernels/batch_gpu.cu:137-147): T <= 32 -> GEMV, else GEMM.
void linear_q(const float* x, const QuantView& W, const uint16_t* bias, int64_t T, int64_t in, int64_t out,
              float* y, hipStream_t stream = nullptr);

// Device copy of one quantised matrix or bf16 vector
// (DevTensor::upload_q, kernels/model_gpu_internal.cuh:57-83).
class DevQuant {
public:
    DevQuant() = default;
    explicit DevQuant(const QTensor& t);
    ~DevQuant();
    DevQuant(DevQuant&& o) noexcept;
    DevQuant& operator=(DevQuant&& o) noexcept;
    DevQuant(const DevQuant&) = delete;
    DevQuant& operator=(const DevQuant&) = delete;
    const QuantView& view() const { return view_; }
    const uint16_t* bf16() const { return static_cast<const uint16_t*>(data_); }  // kBf16 tensors
    bool empty() const { return data_ == nullptr; }

private:
    void release();
    void* data_ = nullptr;  // one allocation: q | scales | zeros (or the bf16 data)
    QuantView view_{};
};

// Every matrix and vector of a QuantModel on the device
// (GpuModel(const QuantModel&), kernels/model_gpu.cu:55-80).
struct DevLayer {
    DevQuant q_w, k_w, v_w, o_w, gate_w, up_w, down_w;
    DevQuant q_b, k_b, v_b, input_ln, post_attn_ln;
};
struct DevQuantModel {
    explicit DevQuantModel(const QuantModel& m);
    DevQuant embed_tokens, lm_head, final_norm;
    std::vector<DevLayer> layers;
    const QuantView& head() const { return lm_head.empty() ? embed_tokens.view() : lm_head.view(); }
};

// The quantised part of the reference's decode step
// (GpuBatch::Impl::launch_sequence, kernels/batch_gpu.cu:186-215) for one
// sequence of one token at position 0, as one chain (include/iq.h
// iq_chain_*): the quantised embedding gather, then per layer RMSNorm ->
// q|k|v (+ biases), single-key attention (each query head takes its kv
// head's value row: the softmax over one key is 1) -> o + residual,
// RMSNorm -> gate|up with the SwiGLU epilogue, down + residual, and the
// final RMSNorm -> LM head.  `rows` sequences (1..32, GpuBatch::kMaxRows,
// kernels/batch_gpu.h:80) of one token each run together, as GpuBatch::step
// runs its batch (kernels/batch_gpu.cu:186-215): every vector is [rows][n].
// Every intermediate vector has its own device buffer.  The model's widths
// must be multiples of 256 (the chain's stage rule).  run(stream) issues
// only device work (capturable into a HIP graph) after the token ids are in
// ids().
class DecodeStep {
public:
    DecodeStep(const DevQuantModel& m, const ModelConfig& cfg, int rows = 1);
    ~DecodeStep();
    DecodeStep(const DecodeStep&) = delete;
    DecodeStep& operator=(const DecodeStep&) = delete;
    // copies the token ids to ids() (host to device, on `stream`; `token`
    // for every row), then run()
    void step(int64_t token, hipStream_t stream = nullptr);
    void step(const int64_t* tokens, int n, hipStream_t stream = nullptr);  // n == rows()
    void run(hipStream_t stream = nullptr);
    int rows() const { return B_; }
    int64_t* ids() const { return ids_; }            // device, rows() ids
    const float* logits() const { return logits_; }  // device, [rows()][vocab_size]
    const float* hidden(int layer) const;            // residual stream entering `layer` (layers: the last), [rows()][H]

private:
    const DevQuantModel& m_;
    int64_t H_ = 0, V_ = 0;
    int B_ = 1;
    float* arena_ = nullptr;
    int64_t* ids_ = nullptr;
    float* logits_ = nullptr;
    std::vector<float*> h_;  // h_[l]: hidden state entering layer l; h_[L]: final
    iq_chain* chain_ = nullptr;
};

}  // namespace gpu
}  // namespace llm

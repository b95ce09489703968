// test_host.cpp -- tests of the C++ host layer (infer_amd/host/iq_host.h),
// in the shape of the reference's tests/test_quant.cpp (container round trip)
// and tests/test_ops_gpu.cu:638-708 (quantised launchers against a
// double-precision dot product over dequant(), kGemvTol = 5e-6 of the
// conditioning sum).  The checker is the oracle (oracle/liboracle.so).
//
//   test_host dump <model_dir> int8|int4
//       loads the model with QuantModel::load and prints one line per tensor
//       of the file (write order): name dtype rows cols fnv(q) fnv(scales)
//       fnv(zeros) -- or fnv(data) for bf16 -- for the pytest wrapper to
//       compare with the fixture's manifest
//   test_host roundtrip <in.llmq> <out.llmq>
//       re-writes every tensor of <in> with QuantWriter, in file order
//   test_host errors <dir>
//       malformed containers must throw std::runtime_error
//   test_host qmodel <tensors.bin> <model_dir> int8|int4 <out.llmq>
//       quantize_model (the offline quantiser's loop, packing on the GPU) over
//       the bf16 tensors of <tensors.bin> (u32 count; per tensor u32 name
//       length, name, u32 ndim, i64 dims, bf16 data), config from
//       <model_dir>/config.json; writes <out.llmq> and prints the report
//   test_host chain <tensors.bin> <dir> int8|int4 <token> <out.bin>
//       the whole host path: quantize_model -> <dir>/model.q8|q4.llmq (config
//       from <dir>/config.json) -> QuantModel::load -> DevQuantModel ->
//       gpu::DecodeStep::step(token); writes the logits (fp32) to <out.bin>
//   test_host gpu <model_dir>
//       on-device quantize (bit-exact), linear_q / embedding on every matrix
//       of the tiny model (int8 and int4) against the oracle
#include "iq_host.h"

#include <execinfo.h>
#include <unistd.h>

#include <cmath>
#include <csignal>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <random>
#include <stdexcept>
#include <string>
#include <vector>

extern "C" {
int iqo_quantize(const uint16_t* w, int64_t rows, int64_t cols, int kind, uint8_t* q, uint16_t* scales,
                 uint8_t* zeros, float* rowbuf);
void iqo_linear_q_f64(const float* x, const uint8_t* q, const uint16_t* scales, const uint8_t* zeros, int kind,
                      const uint16_t* bias, int64_t T, int64_t in, int64_t out, double* y, double* cond);
void iqo_embedding(const uint8_t* q, const uint16_t* scales, const uint8_t* zeros, int kind, int64_t H,
                   const int64_t* ids, int64_t T, float* out);
uint16_t iqo_f32_to_bf16(float f);
}

#define STEP(...) std::fprintf(stderr, "test_host: " __VA_ARGS__)

namespace {

int failures = 0;
#define CHECK(cond, ...)                                               \
    do {                                                               \
        if (!(cond)) {                                                 \
            failures++;                                                \
            std::printf("FAIL %s:%d: ", __FILE__, __LINE__);           \
            std::printf(__VA_ARGS__);                                  \
            std::printf("\n");                                         \
        }                                                              \
    } while (0)

uint64_t fnv1a64(const void* p, size_t n) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    uint64_t h = 0xCBF29CE484222325ull;
    for (size_t i = 0; i < n; i++) {
        h ^= b[i];
        h *= 0x100000001B3ull;
    }
    return h;
}

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

llm::QKind kind_of(const std::string& s) { return s == "int4" ? llm::QKind::kInt4 : llm::QKind::kInt8; }

int cmd_dump(const std::string& dir, const std::string& kind) {
    llm::QuantModel m;
    m.load(dir, kind_of(kind));
    llm::QuantFile f;
    f.open(llm::QuantModel::file_for(dir, kind_of(kind)));
    std::printf("layers %zu tied %d bias %d\n", m.layers.size(), int(m.cfg.tie_word_embeddings),
                int(m.cfg.attention_bias));
    for (const std::string& n : f.names_in_file()) {
        const llm::QTensor& t = f.get(n);
        if (t.kind == llm::QKind::kBf16) {
            std::printf("%s bf16 %lld %lld %016llx\n", n.c_str(), (long long)t.rows, (long long)t.cols,
                        (unsigned long long)fnv1a64(t.bf16, size_t(t.rows * t.cols) * 2));
        } else {
            const size_t ns = size_t(t.rows * t.groups());
            std::printf("%s %s %lld %lld %016llx %016llx %016llx\n", n.c_str(), llm::qkind_name(t.kind),
                        (long long)t.rows, (long long)t.cols, (unsigned long long)fnv1a64(t.q, t.q_bytes()),
                        (unsigned long long)fnv1a64(t.scales, ns * 2),
                        (unsigned long long)(t.zeros ? fnv1a64(t.zeros, ns) : 0));
        }
    }
    // the QuantModel views are the file's
    CHECK(m.layers.size() == size_t(m.cfg.num_hidden_layers), "layer count");
    CHECK(m.layers[0].q_w.q == f.get("model.layers.0.self_attn.q_proj.weight").q ||
              fnv1a64(m.layers[0].q_w.q, m.layers[0].q_w.q_bytes()) ==
                  fnv1a64(f.get("model.layers.0.self_attn.q_proj.weight").q, m.layers[0].q_w.q_bytes()),
          "QuantModel view differs from the file");
    return failures ? 1 : 0;
}

int cmd_roundtrip(const std::string& in, const std::string& out) {
    llm::QuantFile f;
    f.open(in);
    llm::QuantWriter w;
    for (const std::string& n : f.names_in_file()) {
        const llm::QTensor& t = f.get(n);
        if (t.kind == llm::QKind::kBf16) {
            w.add_bf16(n, t.bf16, {t.rows});
            continue;
        }
        llm::QMatrix m;
        m.kind = t.kind;
        m.rows = t.rows;
        m.cols = t.cols;
        const size_t ns = size_t(t.rows * t.groups());
        m.q.assign(t.q, t.q + t.q_bytes());
        m.scales.assign(t.scales, t.scales + ns);
        if (t.zeros) m.zeros.assign(t.zeros, t.zeros + ns);
        w.add(n, m);
    }
    w.write(out);
    // read back: identical views (tests/test_quant.cpp:66-84)
    llm::QuantFile g;
    g.open(out);
    for (const std::string& n : f.names()) {
        const llm::QTensor &a = f.get(n), &b = g.get(n);
        bool same = a.kind == b.kind && a.rows == b.rows && a.cols == b.cols;
        if (same && a.kind != llm::QKind::kBf16)
            for (int64_t r = 0; r < a.rows && same; r += 7)
                for (int64_t c = 0; c < a.cols; c++)
                    if (llm::dequant(a, r, c) != llm::dequant(b, r, c)) { same = false; break; }
        CHECK(same, "round trip differs for %s", n.c_str());
    }
    CHECK(g.kind() == f.kind(), "container kind");
    return failures ? 1 : 0;
}

bool throws(const std::string& path) {
    try {
        llm::QuantFile f;
        f.open(path);
    } catch (const std::runtime_error&) {
        return true;
    }
    return false;
}

int cmd_errors(const std::string& dir) {
    const std::string p = dir + "/bad.llmq";
    auto put = [&](const std::string& bytes) {
        std::ofstream f(p, std::ios::binary);
        f.write(bytes.data(), std::streamsize(bytes.size()));
    };
    auto with_header = [](const std::string& h, size_t blob) {
        std::string s = "LLMQ0001";
        const uint64_t n = h.size();
        for (int i = 0; i < 8; i++) s += char((n >> (8 * i)) & 0xFF);
        return s + h + std::string(blob, '\0');
    };
    put("NOTLLMQ0");
    CHECK(throws(p), "bad magic accepted");
    put("LLMQ0001\xff\xff\xff\x00\x00\x00\x00\x00{}");
    CHECK(throws(p), "header length past the end accepted");
    put(with_header("{\"m\":{\"data\":[0,64],\"dtype\":\"int8\",\"group\":128,\"scales\":[64,66],\"shape\":[1,64]}}", 10));
    CHECK(throws(p), "range past the blob accepted");
    put(with_header("{\"m\":{\"data\":[0,64],\"dtype\":\"int8\",\"group\":64,\"scales\":[64,66],\"shape\":[1,64]}}", 66));
    CHECK(throws(p), "group size 64 accepted");
    put(with_header("{\"m\":{\"data\":[0,32],\"dtype\":\"int4\",\"group\":128,\"scales\":[32,34],\"shape\":[1,64]}}", 34));
    CHECK(throws(p), "int4 without zeros accepted");
    put(with_header("{\"m\":{\"data\":[0,64],\"dtype\":\"int8\",\"group\":128,\"scales\":[64,66],\"shape\":[1,64]", 66));
    CHECK(throws(p), "truncated JSON accepted");
    put(with_header("{\"m\":{\"data\":[0,64],\"dtype\":\"int8\",\"group\":128,\"scales\":[64,66],\"shape\":[-1,-64]}}", 66));
    CHECK(throws(p), "negative dimensions accepted");
    put(with_header("{\"m\":{\"data\":[0,0],\"dtype\":\"bf16\",\"shape\":[0]}}", 0));
    CHECK(throws(p), "zero dimension accepted");
    put(with_header("{\"m\":{\"data\":[0,64],\"dtype\":\"int8\",\"group\":128,\"scales\":[64,66],\"shape\":[1,64,1]}}", 66));
    CHECK(throws(p), "three dimensions accepted");
    put(with_header("{\"m\":{\"data\":[0,64],\"dtype\":\"int8\",\"group\":128,\"scales\":[64,66],\"shape\":[64]}}", 66));
    CHECK(throws(p), "one-dimensional quantised tensor accepted");
    // 2^32 x 2^32 elements: the count wraps to 0 in 64-bit arithmetic
    put(with_header("{\"m\":{\"data\":[0,0],\"dtype\":\"bf16\",\"shape\":[4294967296,4294967296]}}", 0));
    CHECK(throws(p), "overflowing shape accepted");
    put(with_header("{\"m\":{\"data\":[0,64],\"dtype\":\"int8\",\"group\":128,\"scales\":[64,66],\"shape\":[1,64]}}", 66));
    CHECK(!throws(p), "valid minimal container rejected");
    llm::QuantModel m;
    bool threw = false;
    try {
        m.load(dir + "/does-not-exist", llm::QKind::kInt8);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK(threw, "missing model directory accepted");
    std::remove(p.c_str());
    return failures ? 1 : 0;
}

// y = x W^T over every matrix of a layer through linear_q, checked like
// tests/test_ops_gpu.cu:676-692 (canaries past y).
void check_linear(const char* what, const llm::QTensor& t, const llm::gpu::DevQuant& d, const uint16_t* bias_host,
                  const uint16_t* bias_dev, int T, std::mt19937& rng) {
    const int64_t in = t.cols, out = t.rows;
    std::vector<float> x(size_t(T) * in);
    std::normal_distribution<float> nd(0.0f, 1.0f);
    for (float& v : x) v = nd(rng);
    float *dx = nullptr, *dy = nullptr;
    const size_t ny = size_t(T) * out + 16;
    hip_ok(hipMalloc(&dx, x.size() * 4), "hipMalloc");
    hip_ok(hipMalloc(&dy, ny * 4), "hipMalloc");
    std::vector<float> y(ny, -12345.5f);
    hip_ok(hipMemcpy(dx, x.data(), x.size() * 4, hipMemcpyHostToDevice), "upload");
    hip_ok(hipMemcpy(dy, y.data(), ny * 4, hipMemcpyHostToDevice), "upload");
    llm::gpu::linear_q(dx, d.view(), bias_dev, T, in, out, dy);
    hip_ok(hipDeviceSynchronize(), "sync");
    hip_ok(hipMemcpy(y.data(), dy, ny * 4, hipMemcpyDeviceToHost), "download");
    std::vector<double> ref(size_t(T) * out), cond(size_t(T) * out);
    iqo_linear_q_f64(x.data(), t.q, t.scales, t.zeros, t.kind == llm::QKind::kInt4 ? 1 : 0, bias_host, T, in, out,
                     ref.data(), cond.data());
    double worst = 0, maxerr = 0, maxref = 0;
    bool finite = true;
    for (size_t i = 0; i < ref.size(); i++) {
        const double e = std::fabs(double(y[i]) - ref[i]);
        finite &= std::isfinite(y[i]);
        worst = std::max(worst, e / std::max(cond[i], 1e-30));
        maxerr = std::max(maxerr, e);
        maxref = std::max(maxref, std::fabs(ref[i]));
    }
    bool canary = true;
    for (size_t i = ref.size(); i < ny; i++) canary &= y[i] == -12345.5f;
    CHECK(finite && worst <= 5e-6 && maxerr <= 1e-3 * maxref && canary,
          "%s T=%d: cond err %.3g, max rel %.3g, canary %d", what, T, worst, maxerr / maxref, int(canary));
    (void)hipFree(dx);
    (void)hipFree(dy);
}

int cmd_gpu(const std::string& dir) {
    std::mt19937 rng(7);
    // on-device quantize vs the oracle (bit-exact), including a partial group
    for (llm::QKind kind : {llm::QKind::kInt8, llm::QKind::kInt4}) {
        for (int64_t cols : {128, 130, 896, 1536}) {
            const int64_t rows = 37;
            std::normal_distribution<float> nd(0.0f, 0.05f);
            std::vector<uint16_t> w(size_t(rows * cols));
            for (auto& v : w) v = iqo_f32_to_bf16(nd(rng));
            STEP("quantize %s cols=%lld\n", llm::qkind_name(kind), (long long)cols);
            const llm::QMatrix m = llm::quantize(w.data(), rows, cols, kind);
            const int64_t G = (cols + 127) / 128;
            std::vector<uint8_t> q(m.q.size()), z(size_t(rows * G));
            std::vector<uint16_t> s(size_t(rows * G));
            std::vector<float> rowbuf(static_cast<size_t>(cols));
            CHECK(iqo_quantize(w.data(), rows, cols, kind == llm::QKind::kInt4 ? 1 : 0, q.data(), s.data(), z.data(),
                               rowbuf.data()) == 0,
                  "oracle quantize");
            CHECK(q == m.q && s == m.scales && (kind == llm::QKind::kInt8 || z == m.zeros), "quantize %s cols=%lld differs",
                  llm::qkind_name(kind), (long long)cols);
        }
    }
    for (llm::QKind kind : {llm::QKind::kInt8, llm::QKind::kInt4}) {
        STEP("load + upload %s\n", llm::qkind_name(kind));
        llm::QuantModel m;
        m.load(dir, kind);
        llm::gpu::DevQuantModel d(m);
        for (size_t li = 0; li < m.layers.size(); li++) {
            const llm::QLayer& L = m.layers[li];
            const llm::gpu::DevLayer& D = d.layers[li];
            for (int T : {1, 3, 40}) {
                STEP("layer %zu T=%d\n", li, T);
                check_linear("q_proj", L.q_w, D.q_w, L.q_b.bf16, D.q_b.bf16(), T, rng);
                check_linear("k_proj", L.k_w, D.k_w, L.k_b.bf16, D.k_b.bf16(), T, rng);
                check_linear("v_proj", L.v_w, D.v_w, L.v_b.bf16, D.v_b.bf16(), T, rng);
                check_linear("o_proj", L.o_w, D.o_w, nullptr, nullptr, T, rng);
                check_linear("gate_proj", L.gate_w, D.gate_w, nullptr, nullptr, T, rng);
                check_linear("up_proj", L.up_w, D.up_w, nullptr, nullptr, T, rng);
                check_linear("down_proj", L.down_w, D.down_w, nullptr, nullptr, T, rng);
            }
        }
        check_linear("lm_head", m.lm_head, d.lm_head, nullptr, nullptr, 2, rng);
        STEP("embedding %s\n", llm::qkind_name(kind));
        // embedding gather: exact (tests/test_ops_gpu.cu:886-893)
        const int64_t H = m.cfg.hidden_size;
        const std::vector<int64_t> ids = {0, m.cfg.vocab_size - 1, 7, 7, 42};
        int64_t* did = nullptr;
        float* dout = nullptr;
        hip_ok(hipMalloc(&did, ids.size() * 8), "hipMalloc");
        hip_ok(hipMalloc(&dout, ids.size() * H * 4), "hipMalloc");
        hip_ok(hipMemcpy(did, ids.data(), ids.size() * 8, hipMemcpyHostToDevice), "upload");
        llm::gpu::launch_embedding_q(d.embed_tokens.view(), did, int64_t(ids.size()), H, dout);
        std::vector<float> got(ids.size() * H), ref(ids.size() * H);
        hip_ok(hipMemcpy(got.data(), dout, got.size() * 4, hipMemcpyDeviceToHost), "download");
        iqo_embedding(m.embed_tokens.q, m.embed_tokens.scales, m.embed_tokens.zeros, kind == llm::QKind::kInt4 ? 1 : 0,
                      H, ids.data(), int64_t(ids.size()), ref.data());
        CHECK(std::memcmp(got.data(), ref.data(), got.size() * 4) == 0, "embedding %s differs", llm::qkind_name(kind));
        (void)hipFree(did);
        (void)hipFree(dout);
    }
    // a rejected call throws (bad shape: in != W.cols)
    llm::QuantModel m;
    m.load(dir, llm::QKind::kInt8);
    llm::gpu::DevQuantModel d(m);
    bool threw = false;
    try {
        llm::gpu::launch_gemv_batched_q(nullptr, d.layers[0].q_w.view(), nullptr, 1, 3, 3, nullptr);
    } catch (const std::runtime_error&) {
        threw = true;
    }
    CHECK(threw, "rejected launch did not throw");
    return failures ? 1 : 0;
}

}  // namespace

// A crash report names the failing step (stdout to a pipe is block-buffered).
void on_fault(int sig) {
    void* fr[32];
    const int n = backtrace(fr, 32);
    std::fprintf(stderr, "test_host: signal %d\n", sig);
    backtrace_symbols_fd(fr, n, 2);
    _exit(128 + sig);
}

int cmd_qmodel(const std::string& bin, const std::string& dir, const std::string& kind, const std::string& out) {
    std::ifstream f(bin, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + bin);
    auto rd = [&](void* p, size_t n) {
        f.read(static_cast<char*>(p), std::streamsize(n));
        if (!f) throw std::runtime_error("truncated " + bin);
    };
    uint32_t count = 0;
    rd(&count, 4);
    std::vector<std::vector<uint16_t>> store(count);
    std::map<std::string, llm::BF16Tensor> src;
    for (uint32_t i = 0; i < count; i++) {
        uint32_t nl = 0, nd = 0;
        rd(&nl, 4);
        std::string name(nl, '\0');
        rd(&name[0], nl);
        rd(&nd, 4);
        std::vector<int64_t> shape(nd);
        rd(shape.data(), 8 * nd);
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        store[i].resize(size_t(n));
        rd(store[i].data(), size_t(n) * 2);
        src[name] = llm::BF16Tensor{store[i].data(), shape};
    }
    const llm::ModelConfig cfg = llm::ModelConfig::from_file(dir + "/config.json");
    llm::QuantWriter w;
    const llm::QuantizeReport r = llm::quantize_model(src, cfg, kind_of(kind), w);
    w.write(out);
    std::printf("quantized %d matrices, %d vectors: %zu -> %zu bytes, worst group error %.6f of absmax\n", r.matrices,
                r.vectors, r.bytes_in, r.bytes_out, r.worst);
    return 0;
}

std::map<std::string, llm::BF16Tensor> read_tensors(const std::string& bin, std::vector<std::vector<uint16_t>>& store) {
    std::ifstream f(bin, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + bin);
    auto rd = [&](void* p, size_t n) {
        f.read(static_cast<char*>(p), std::streamsize(n));
        if (!f) throw std::runtime_error("truncated " + bin);
    };
    uint32_t count = 0;
    rd(&count, 4);
    store.assign(count, {});
    std::map<std::string, llm::BF16Tensor> src;
    for (uint32_t i = 0; i < count; i++) {
        uint32_t nl = 0, nd = 0;
        rd(&nl, 4);
        std::string name(nl, '\0');
        rd(&name[0], nl);
        rd(&nd, 4);
        std::vector<int64_t> shape(nd);
        rd(shape.data(), 8 * nd);
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        store[i].resize(size_t(n));
        rd(store[i].data(), size_t(n) * 2);
        src[name] = llm::BF16Tensor{store[i].data(), shape};
    }
    return src;
}

int cmd_chain(const std::string& bin, const std::string& dir, const std::string& kind, int64_t token,
              const std::string& out) {
    std::vector<std::vector<uint16_t>> store;
    const auto src = read_tensors(bin, store);
    const llm::ModelConfig cfg = llm::ModelConfig::from_file(dir + "/config.json");
    llm::QuantWriter w;
    llm::quantize_model(src, cfg, kind_of(kind), w);
    w.write(llm::QuantModel::file_for(dir, kind_of(kind)));
    llm::QuantModel qm;
    qm.load(dir, kind_of(kind));
    llm::gpu::DevQuantModel dm(qm);
    // rows > 1 (env IQ_TEST_ROWS): row b takes token + 7 b
    const char* re = std::getenv("IQ_TEST_ROWS");
    const int rows = re ? std::atoi(re) : 1;
    llm::gpu::DecodeStep step(dm, qm.cfg, rows);
    std::vector<int64_t> toks(static_cast<size_t>(rows));
    for (int b = 0; b < rows; b++) toks[size_t(b)] = (token + 7 * b) % cfg.vocab_size;
    step.step(toks.data(), rows);
    std::vector<float> logits(size_t(cfg.vocab_size) * size_t(rows));
    hip_ok(hipMemcpy(logits.data(), step.logits(), logits.size() * 4, hipMemcpyDeviceToHost), "logits");
    std::ofstream f(out, std::ios::binary);
    f.write(reinterpret_cast<const char*>(logits.data()), std::streamsize(logits.size() * 4));
    std::printf("chain ok: %zu logits\n", logits.size());
    return 0;
}

int main(int argc, char** argv) {
    std::setvbuf(stdout, nullptr, _IOLBF, 0);
    std::signal(SIGSEGV, on_fault);
    std::signal(SIGBUS, on_fault);
    if (argc < 3) {
        std::fprintf(stderr, "usage: %s dump|roundtrip|errors|gpu ...\n", argv[0]);
        return 2;
    }
    const std::string cmd = argv[1];
    try {
        int rc = 2;
        if (cmd == "dump" && argc == 4) rc = cmd_dump(argv[2], argv[3]);
        else if (cmd == "roundtrip" && argc == 4) rc = cmd_roundtrip(argv[2], argv[3]);
        else if (cmd == "errors") rc = cmd_errors(argv[2]);
        else if (cmd == "gpu") rc = cmd_gpu(argv[2]);
        else if (cmd == "qmodel" && argc == 6) rc = cmd_qmodel(argv[2], argv[3], argv[4], argv[5]);
        else if (cmd == "chain" && argc == 7) rc = cmd_chain(argv[2], argv[3], argv[4], std::atoll(argv[5]), argv[6]);
        if (rc == 0) std::fprintf(stderr, "test_host %s: all checks passed\n", cmd.c_str());
        return rc;
    } catch (const std::exception& e) {
        std::printf("error: %s\n", e.what());
        return 3;
    }
}

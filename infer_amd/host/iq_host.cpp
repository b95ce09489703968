// iq_host.cpp -- the C++ host layer of iq_host.h: .llmq container,
// config.json, model loading and upload, and the QuantView launchers over the
// C ABI of include/iq.h.
#include "iq_host.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <stdexcept>

namespace llm {

namespace {

// ------------------------------------------------------------------ JSON
// The subset .llmq headers and config.json use: objects, arrays, strings,
// numbers, true / false / null.
struct JVal {
    enum Type { kNull, kBool, kNum, kStr, kArr, kObj } type = kNull;
    bool b = false;
    double num = 0;
    bool is_int = false;
    int64_t inum = 0;
    std::string str;
    std::vector<JVal> arr;
    std::vector<std::pair<std::string, JVal>> obj;

    const JVal* find(const std::string& k) const {
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
    const JVal& at(const std::string& k) const {
        const JVal* v = find(k);
        if (!v) throw std::runtime_error("missing key \"" + k + "\"");
        return *v;
    }
    int64_t as_int() const {
        if (type != kNum) throw std::runtime_error("expected a number");
        return is_int ? inum : int64_t(num);
    }
    double as_double() const {
        if (type != kNum) throw std::runtime_error("expected a number");
        return is_int ? double(inum) : num;
    }
    bool as_bool() const {
        if (type != kBool) throw std::runtime_error("expected true or false");
        return b;
    }
    const std::string& as_str() const {
        if (type != kStr) throw std::runtime_error("expected a string");
        return str;
    }
};

class JParser {
public:
    JParser(const char* b, const char* e) : p_(b), e_(e) {}
    JVal parse() {
        JVal v = value();
        ws();
        if (p_ != e_) fail("trailing characters");
        return v;
    }

private:
    const char* p_;
    const char* e_;

    [[noreturn]] void fail(const char* what) { throw std::runtime_error(std::string("JSON: ") + what); }
    void ws() {
        while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
    }
    bool lit(const char* s) {
        const size_t n = std::strlen(s);
        if (size_t(e_ - p_) >= n && std::memcmp(p_, s, n) == 0) {
            p_ += n;
            return true;
        }
        return false;
    }
    JVal value() {
        ws();
        if (p_ >= e_) fail("unexpected end");
        JVal v;
        if (*p_ == '{') {
            v.type = JVal::kObj;
            p_++;
            ws();
            if (p_ < e_ && *p_ == '}') { p_++; return v; }
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p_ >= e_ || *p_ != ':') fail("expected ':'");
                p_++;
                v.obj.emplace_back(std::move(k), value());
                ws();
                if (p_ < e_ && *p_ == ',') { p_++; continue; }
                if (p_ < e_ && *p_ == '}') { p_++; return v; }
                fail("expected ',' or '}'");
            }
        }
        if (*p_ == '[') {
            v.type = JVal::kArr;
            p_++;
            ws();
            if (p_ < e_ && *p_ == ']') { p_++; return v; }
            for (;;) {
                v.arr.push_back(value());
                ws();
                if (p_ < e_ && *p_ == ',') { p_++; continue; }
                if (p_ < e_ && *p_ == ']') { p_++; return v; }
                fail("expected ',' or ']'");
            }
        }
        if (*p_ == '"') {
            v.type = JVal::kStr;
            v.str = string();
            return v;
        }
        if (lit("true")) { v.type = JVal::kBool; v.b = true; return v; }
        if (lit("false")) { v.type = JVal::kBool; v.b = false; return v; }
        if (lit("null")) return v;
        return number();
    }
    std::string string() {
        if (p_ >= e_ || *p_ != '"') fail("expected a string");
        p_++;
        std::string s;
        while (p_ < e_ && *p_ != '"') {
            char c = *p_++;
            if (c != '\\') { s += c; continue; }
            if (p_ >= e_) fail("bad escape");
            c = *p_++;
            switch (c) {
                case '"': s += '"'; break;
                case '\\': s += '\\'; break;
                case '/': s += '/'; break;
                case 'b': s += '\b'; break;
                case 'f': s += '\f'; break;
                case 'n': s += '\n'; break;
                case 'r': s += '\r'; break;
                case 't': s += '\t'; break;
                case 'u': {
                    if (e_ - p_ < 4) fail("bad \\u escape");
                    unsigned cp = 0;
                    for (int i = 0; i < 4; i++) {
                        const char h = *p_++;
                        cp = cp * 16 + unsigned(h >= 'a' ? h - 'a' + 10 : h >= 'A' ? h - 'A' + 10 : h - '0');
                    }
                    // UTF-8 of a BMP code point (names here are ASCII)
                    if (cp < 0x80) s += char(cp);
                    else if (cp < 0x800) { s += char(0xC0 | (cp >> 6)); s += char(0x80 | (cp & 0x3F)); }
                    else {
                        s += char(0xE0 | (cp >> 12));
                        s += char(0x80 | ((cp >> 6) & 0x3F));
                        s += char(0x80 | (cp & 0x3F));
                    }
                    break;
                }
                default: fail("bad escape");
            }
        }
        if (p_ >= e_) fail("unterminated string");
        p_++;
        return s;
    }
    JVal number() {
        const char* b = p_;
        bool frac = false;
        if (p_ < e_ && (*p_ == '-' || *p_ == '+')) p_++;
        while (p_ < e_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' ||
                           *p_ == '-' || *p_ == '+')) {
            if (*p_ == '.' || *p_ == 'e' || *p_ == 'E') frac = true;
            p_++;
        }
        if (p_ == b) fail("unexpected character");
        const std::string t(b, p_);
        JVal v;
        v.type = JVal::kNum;
        v.num = std::strtod(t.c_str(), nullptr);
        if (!frac) {
            v.is_int = true;
            v.inum = std::strtoll(t.c_str(), nullptr, 10);
        }
        return v;
    }
};

JVal parse_json(const char* b, const char* e) { return JParser(b, e).parse(); }

std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    return std::string(std::istreambuf_iterator<char>(f), std::istreambuf_iterator<char>());
}

float bf16_bits_to_f32(uint16_t h) {
    const uint32_t u = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void iq_check(int rc, const char* what) {
    if (rc != IQ_OK) throw std::runtime_error(std::string(what) + ": " + iq_error_string(rc));
}

}  // namespace

const char* qkind_name(QKind k) {
    return k == QKind::kInt8 ? "int8" : k == QKind::kInt4 ? "int4" : "bf16";
}

QTensor QMatrix::view() const {
    QTensor t;
    t.kind = kind;
    t.rows = rows;
    t.cols = cols;
    t.q = q.data();
    t.scales = scales.data();
    t.zeros = zeros.empty() ? nullptr : zeros.data();
    return t;
}

float dequant(const QTensor& t, int64_t r, int64_t c) {
    const int64_t G = t.groups(), g = c / kGroup;
    const float s = bf16_bits_to_f32(t.scales[r * G + g]);
    if (t.kind == QKind::kInt8) return s * float(int8_t(t.q[r * t.cols + c]));
    const uint8_t byte = t.q[(r * t.cols + c) / 2];
    const int v = (c & 1) ? (byte >> 4) : (byte & 0x0F);
    return s * float(v - int(t.zeros[r * G + g]));
}

QMatrix quantize(const uint16_t* w_bf16, int64_t rows, int64_t cols, QKind kind) {
    if (kind != QKind::kInt8 && kind != QKind::kInt4) throw std::runtime_error("quantize: kind must be int8 or int4");
    if (kind == QKind::kInt4 && cols % 2) throw std::runtime_error("int4 quantisation needs an even column count");
    QMatrix m;
    m.kind = kind;
    m.rows = rows;
    m.cols = cols;
    const int64_t G = (cols + kGroup - 1) / kGroup;
    m.q.resize(kind == QKind::kInt4 ? size_t(rows) * cols / 2 : size_t(rows) * cols);
    m.scales.resize(size_t(rows) * G);
    if (kind == QKind::kInt4) m.zeros.resize(size_t(rows) * G);
    const size_t nw = size_t(rows) * cols * 2, nq = m.q.size(), ns = m.scales.size() * 2, nz = m.zeros.size();
    char* d = nullptr;
    hip_check(hipMalloc(&d, nw + nq + ns + nz + 64), "quantize: hipMalloc");
    auto cleanup = [&]() { (void)hipFree(d); };
    try {
        uint16_t* dw = reinterpret_cast<uint16_t*>(d);
        uint8_t* dq = reinterpret_cast<uint8_t*>(d + nw);
        uint16_t* ds = reinterpret_cast<uint16_t*>(d + ((nw + nq + 1) & ~size_t(1)));
        uint8_t* dz = reinterpret_cast<uint8_t*>(reinterpret_cast<char*>(ds) + ns);
        hip_check(hipMemcpy(dw, w_bf16, nw, hipMemcpyHostToDevice), "quantize: upload");
        iq_check(iq_quantize(dw, rows, cols, kind == QKind::kInt4 ? IQ_INT4 : IQ_INT8, dq, ds,
                             kind == QKind::kInt4 ? dz : nullptr, nullptr),
                 "quantize");
        hip_check(hipMemcpy(m.q.data(), dq, nq, hipMemcpyDeviceToHost), "quantize: download");
        hip_check(hipMemcpy(m.scales.data(), ds, ns, hipMemcpyDeviceToHost), "quantize: download");
        if (nz) hip_check(hipMemcpy(m.zeros.data(), dz, nz, hipMemcpyDeviceToHost), "quantize: download");
    } catch (...) {
        cleanup();
        throw;
    }
    cleanup();
    return m;
}

// ------------------------------------------------------------------ model quantiser
namespace {

// Device buffers for one matrix at a time, grown to the largest seen.
class Staging {
public:
    ~Staging() {
        if (d_) (void)hipFree(d_);
    }
    // bf16 input, codes, scales, zero points for a rows x cols matrix
    void fit(int64_t rows, int64_t cols) {
        const size_t G = size_t((cols + kGroup - 1) / kGroup);
        in_ = size_t(rows) * cols * 2;
        q_ = size_t(rows) * cols;  // int8 upper bound
        s_ = size_t(rows) * G * 2;
        z_ = size_t(rows) * G;
        const size_t need = align(in_) + align(q_) + align(s_) + align(z_);
        if (need > cap_) {
            if (d_) (void)hipFree(d_);
            d_ = nullptr;
            cap_ = 0;
            hip_check(hipMalloc(&d_, need), "quantize_model: hipMalloc");
            cap_ = need;
        }
    }
    uint16_t* in() { return reinterpret_cast<uint16_t*>(base(0)); }
    uint8_t* q() { return reinterpret_cast<uint8_t*>(base(align(in_))); }
    uint16_t* s() { return reinterpret_cast<uint16_t*>(base(align(in_) + align(q_))); }
    uint8_t* z() { return reinterpret_cast<uint8_t*>(base(align(in_) + align(q_) + align(s_))); }

private:
    static size_t align(size_t v) { return (v + 255) & ~size_t(255); }
    char* base(size_t off) { return static_cast<char*>(d_) + off; }
    void* d_ = nullptr;
    size_t cap_ = 0, in_ = 0, q_ = 0, s_ = 0, z_ = 0;
};

// Worst |w - dequant(w)| / absmax over the groups of every rows/64-th row
// (zero-absmax groups skipped): the reference's report of
// tools/quantize.cpp:35-45, evaluated the same way on the host.
double sampled_group_error(const uint16_t* w, const QTensor& t) {
    double worst = 0.0;
    const int64_t step = std::max<int64_t>(1, t.rows / 64);
    for (int64_t r = 0; r < t.rows; r += step)
        for (int64_t g = 0; g < t.groups(); g++) {
            float amax = 0.0f, err = 0.0f;
            const int64_t c1 = std::min(t.cols, (g + 1) * kGroup);
            for (int64_t c = g * kGroup; c < c1; c++) {
                const float x = bf16_bits_to_f32(w[r * t.cols + c]);
                amax = std::max(amax, std::fabs(x));
                err = std::max(err, std::fabs(x - dequant(t, r, c)));
            }
            if (amax > 0.0f) worst = std::max(worst, double(err / amax));
        }
    return worst;
}

}  // namespace

QuantizeReport quantize_model(const std::map<std::string, BF16Tensor>& src, const ModelConfig& cfg, QKind kind,
                              QuantWriter& w) {
    if (kind != QKind::kInt8 && kind != QKind::kInt4) throw std::runtime_error("quantize_model: kind must be int8 or int4");
    QuantizeReport rep;
    const auto t0 = std::chrono::steady_clock::now();
    Staging dev;
    auto find = [&](const std::string& name) -> const BF16Tensor* {
        auto it = src.find(name);
        return it == src.end() ? nullptr : &it->second;
    };
    auto need = [&](const std::string& name) -> const BF16Tensor& {
        const BF16Tensor* t = find(name);
        if (!t || !t->data) throw std::runtime_error("quantize_model: missing tensor " + name);
        return *t;
    };
    auto matrix = [&](const std::string& name) {
        const BF16Tensor& t = need(name);
        if (t.shape.size() != 2 || t.shape[0] <= 0 || t.shape[1] <= 0)
            throw std::runtime_error("quantize_model: " + name + " is not a matrix");
        const int64_t rows = t.shape[0], cols = t.shape[1];
        if (kind == QKind::kInt4 && (cols & 1)) throw std::runtime_error("quantize_model: " + name + " has an odd width");
        QMatrix m;
        m.kind = kind;
        m.rows = rows;
        m.cols = cols;
        const int64_t G = (cols + kGroup - 1) / kGroup;
        m.q.resize(kind == QKind::kInt4 ? size_t(rows) * cols / 2 : size_t(rows) * cols);
        m.scales.resize(size_t(rows) * G);
        if (kind == QKind::kInt4) m.zeros.resize(size_t(rows) * G);
        dev.fit(rows, cols);
        hip_check(hipMemcpy(dev.in(), t.data, size_t(rows) * cols * 2, hipMemcpyHostToDevice), "quantize_model: upload");
        iq_check(iq_quantize(dev.in(), rows, cols, kind == QKind::kInt4 ? IQ_INT4 : IQ_INT8, dev.q(), dev.s(),
                             kind == QKind::kInt4 ? dev.z() : nullptr, nullptr),
                 "quantize_model");
        hip_check(hipMemcpy(m.q.data(), dev.q(), m.q.size(), hipMemcpyDeviceToHost), "quantize_model: download");
        hip_check(hipMemcpy(m.scales.data(), dev.s(), m.scales.size() * 2, hipMemcpyDeviceToHost),
                  "quantize_model: download");
        if (!m.zeros.empty())
            hip_check(hipMemcpy(m.zeros.data(), dev.z(), m.zeros.size(), hipMemcpyDeviceToHost), "quantize_model: download");
        rep.worst = std::max(rep.worst, sampled_group_error(t.data, m.view()));
        rep.bytes_in += size_t(rows) * cols * 2;
        rep.bytes_out += m.q.size() + m.scales.size() * 2 + m.zeros.size();
        rep.matrices++;
        w.add(name, m);
    };
    auto copy_vec = [&](const std::string& name, bool required) {
        const BF16Tensor* t = required ? &need(name) : find(name);
        if (!t || !t->data) return;
        int64_t n = 1;
        for (int64_t d : t->shape) n *= d;
        w.add_bf16(name, t->data, t->shape);
        rep.bytes_in += size_t(n) * 2;
        rep.bytes_out += size_t(n) * 2;
        rep.vectors++;
    };
    matrix("model.embed_tokens.weight");
    if (find("lm_head.weight")) matrix("lm_head.weight");
    copy_vec("model.norm.weight", true);
    for (int64_t i = 0; i < cfg.num_hidden_layers; i++) {
        const std::string p = "model.layers." + std::to_string(i) + ".";
        for (const char* m : {"self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
                              "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
                              "mlp.down_proj.weight"})
            matrix(p + m);
        copy_vec(p + "input_layernorm.weight", true);
        copy_vec(p + "post_attention_layernorm.weight", true);
        for (const char* b : {"self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias"})
            copy_vec(p + b, false);
    }
    rep.seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    return rep;
}

// ------------------------------------------------------------------ writer
void QuantWriter::add(const std::string& name, const QMatrix& m) {
    if (m.kind == QKind::kBf16) throw std::runtime_error("QuantWriter::add: " + name + " is not quantised");
    entries_.push_back({name, m.kind, {m.rows, m.cols}, m.q, m.zeros, m.scales});
}

void QuantWriter::add_bf16(const std::string& name, const uint16_t* data, std::vector<int64_t> shape) {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    Entry e{name, QKind::kBf16, std::move(shape), {}, {}, {}};
    e.scales.assign(data, data + n);  // the bf16 payload rides in `scales`
    entries_.push_back(std::move(e));
}

std::vector<uint8_t> QuantWriter::serialize() const {
    // Header: names in sorted order (a JSON object with sorted keys, compact),
    // byte ranges in insertion order; the same bytes the reference's writer
    // produces for the same entries.
    struct Ranges {
        const Entry* e;
        size_t data[2], scales[2], zeros[2];
    };
    std::map<std::string, Ranges> hdr;
    size_t off = 0;
    for (const Entry& e : entries_) {
        Ranges r{&e, {0, 0}, {0, 0}, {0, 0}};
        auto span = [&](size_t (&rg)[2], size_t n) { rg[0] = off; rg[1] = off + n; off += n; };
        if (e.kind == QKind::kBf16) {
            span(r.data, e.scales.size() * 2);
        } else {
            span(r.data, e.q.size());
            span(r.scales, e.scales.size() * 2);
            if (!e.zeros.empty()) span(r.zeros, e.zeros.size());
        }
        if (!hdr.emplace(e.name, r).second) throw std::runtime_error("QuantWriter: duplicate tensor " + e.name);
    }
    std::string h = "{";
    bool first = true;
    for (const auto& kv : hdr) {
        const Ranges& r = kv.second;
        const Entry& e = *r.e;
        auto range = [](const size_t (&rg)[2]) { return "[" + std::to_string(rg[0]) + "," + std::to_string(rg[1]) + "]"; };
        std::string shape = "[";
        for (size_t i = 0; i < e.shape.size(); i++) shape += (i ? "," : "") + std::to_string(e.shape[i]);
        shape += "]";
        std::string esc;
        for (char c : kv.first) {
            if (c == '"' || c == '\\') esc += '\\';
            esc += c;
        }
        h += (first ? "\"" : ",\"") + esc + "\":{\"data\":" + range(r.data) + ",\"dtype\":\"" + qkind_name(e.kind) +
             "\",\"group\":" + std::to_string(kGroup);
        if (e.kind != QKind::kBf16) h += ",\"scales\":" + range(r.scales);
        h += ",\"shape\":" + shape;
        if (e.kind != QKind::kBf16 && !e.zeros.empty()) h += ",\"zeros\":" + range(r.zeros);
        h += "}";
        first = false;
    }
    h += "}";
    std::vector<uint8_t> out;
    out.reserve(16 + h.size() + off);
    const char magic[8] = {'L', 'L', 'M', 'Q', '0', '0', '0', '1'};
    out.insert(out.end(), magic, magic + 8);
    const uint64_t hl = h.size();
    for (int i = 0; i < 8; i++) out.push_back(uint8_t(hl >> (8 * i)));
    out.insert(out.end(), h.begin(), h.end());
    auto put = [&](const void* p, size_t n) {
        const uint8_t* b = static_cast<const uint8_t*>(p);
        out.insert(out.end(), b, b + n);
    };
    for (const Entry& e : entries_) {
        if (e.kind == QKind::kBf16) {
            put(e.scales.data(), e.scales.size() * 2);
            continue;
        }
        put(e.q.data(), e.q.size());
        put(e.scales.data(), e.scales.size() * 2);
        if (!e.zeros.empty()) put(e.zeros.data(), e.zeros.size());
    }
    return out;
}

void QuantWriter::write(const std::string& path) const {
    const std::vector<uint8_t> b = serialize();
    std::ofstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot write " + path);
    f.write(reinterpret_cast<const char*>(b.data()), std::streamsize(b.size()));
    if (!f) throw std::runtime_error("write failed: " + path);
}

// ------------------------------------------------------------------ reader
// A read-only file mapping; the QuantFile keeps it while its views live.
namespace {

struct Span {
    const uint8_t* p = nullptr;
    size_t n = 0;
};

// Maps `path` read-only; returns the mapping (nullptr for an empty file).
Span map_readonly(const std::string& path) {
    const int fd = ::open(path.c_str(), O_RDONLY);
    if (fd < 0) throw std::runtime_error("llmq: " + path + ": cannot be opened");
    struct stat st;
    const bool sized = fstat(fd, &st) == 0;
    void* m = nullptr;
    if (sized && st.st_size > 0) m = mmap(nullptr, size_t(st.st_size), PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (!sized) throw std::runtime_error("llmq: " + path + ": cannot stat");
    if (m == MAP_FAILED) throw std::runtime_error("llmq: " + path + ": cannot be mapped");
    return Span{static_cast<const uint8_t*>(m), size_t(st.st_size)};
}

// The fixed preamble: 8 magic bytes, then the header length (u64 LE).
constexpr size_t kPreamble = 16;

uint64_t le64(const uint8_t* b) {
    uint64_t v = 0;
    for (int i = 7; i >= 0; i--) v = (v << 8) | b[i];
    return v;
}

QKind kind_of_dtype(const std::string& d, const std::string& where) {
    for (QKind k : {QKind::kInt8, QKind::kInt4, QKind::kBf16})
        if (d == qkind_name(k)) return k;
    throw std::runtime_error("llmq: " + where + ": dtype \"" + d + "\" is not int8, int4 or bf16");
}

}  // namespace

QuantFile::~QuantFile() {
    if (map_) munmap(map_, map_size_);
}

void QuantFile::open(const std::string& path) {
    // Parse everything into locals first; the object changes only when the
    // whole file is valid (a failed open leaves the previous file in place).
    Span file = map_readonly(path);
    struct Unmap {
        Span* s;
        ~Unmap() { if (s && s->p) munmap(const_cast<uint8_t*>(s->p), s->n); }
    } guard{&file};
    auto bad = [&](const std::string& why) { return std::runtime_error("llmq: " + path + ": " + why); };

    if (file.n < kPreamble || std::memcmp(file.p, "LLMQ0001", 8) != 0) throw bad("missing LLMQ0001 magic");
    const uint64_t header_len = le64(file.p + 8);
    if (header_len > file.n - kPreamble) throw bad("header runs past the end of the file");
    const char* hb = reinterpret_cast<const char*>(file.p + kPreamble);
    const JVal header = parse_json(hb, hb + header_len);
    if (header.type != JVal::kObj) throw bad("header is not a JSON object");
    const Span blob{file.p + kPreamble + header_len, file.n - kPreamble - header_len};

    // [begin, end) of one payload, checked against the blob and its expected size.
    auto payload = [&](const JVal& r, size_t expect, const std::string& name) -> size_t {
        if (r.type != JVal::kArr || r.arr.size() != 2) throw bad(name + ": a byte range must be [begin, end]");
        const int64_t lo = r.arr[0].as_int(), hi = r.arr[1].as_int();
        if (lo < 0 || hi < lo || uint64_t(hi) > blob.n) throw bad(name + ": byte range outside the data");
        if (uint64_t(hi - lo) != expect) throw bad(name + ": byte range does not match the shape");
        return size_t(lo);
    };

    std::map<std::string, QTensor> tensors;
    std::map<std::string, size_t> first_byte;
    QKind file_kind = QKind::kBf16;
    for (const auto& entry : header.obj) {
        const std::string& name = entry.first;
        const JVal& e = entry.second;
        QTensor t;
        t.kind = kind_of_dtype(e.at("dtype").as_str(), name);
        const JVal& shape = e.at("shape");
        // the reference's writer emits [n] (bf16 vectors) or [rows, cols];
        // every dimension positive, the element count checked against
        // overflow before any payload size is derived from it
        if (shape.type != JVal::kArr || shape.arr.empty() || shape.arr.size() > 2)
            throw bad(name + ": shape must be [n] or [rows, cols]");
        if (t.kind != QKind::kBf16 && shape.arr.size() != 2) throw bad(name + ": a quantised tensor needs [rows, cols]");
        constexpr int64_t kMaxDim = int64_t(1) << 40;
        int64_t count = 1;
        for (const JVal& d : shape.arr) {
            const int64_t v = d.as_int();
            if (v <= 0 || v > kMaxDim) throw bad(name + ": shape dimension out of range");
            if (count > (int64_t(1) << 62) / v) throw bad(name + ": shape too large");
            count *= v;
        }
        t.rows = shape.arr[0].as_int();
        t.cols = shape.arr.size() > 1 ? shape.arr[1].as_int() : 1;
        if (t.kind == QKind::kBf16) {
            const size_t at = payload(e.at("data"), size_t(count) * 2, name);
            t.bf16 = reinterpret_cast<const uint16_t*>(blob.p + at);
            first_byte[name] = at;
        } else {
            if (const JVal* g = e.find("group"); g && g->as_int() != kGroup)
                throw bad(name + ": group size " + std::to_string(g->as_int()) + " (this build reads 128)");
            if (t.kind == QKind::kInt4 && (t.cols & 1)) throw bad(name + ": int4 rows need an even width");
            const size_t meta = size_t(t.rows) * size_t(t.groups());
            const size_t qa = payload(e.at("data"), t.q_bytes(), name);
            t.q = blob.p + qa;
            t.scales = reinterpret_cast<const uint16_t*>(blob.p + payload(e.at("scales"), meta * 2, name));
            const JVal* z = e.find("zeros");
            if (t.kind == QKind::kInt4) {
                if (!z) throw bad(name + ": int4 needs zero points");
                t.zeros = blob.p + payload(*z, meta, name);
            } else if (z) {
                t.zeros = blob.p + payload(*z, meta, name);
            }
            first_byte[name] = qa;
            file_kind = t.kind;
        }
        tensors.emplace(name, t);
    }

    if (map_) munmap(map_, map_size_);
    map_ = const_cast<uint8_t*>(file.p);
    map_size_ = file.n;
    guard.s = nullptr;  // ownership moves to the object
    tensors_ = std::move(tensors);
    offset_ = std::move(first_byte);
    kind_ = file_kind;
}

const QTensor& QuantFile::get(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) throw std::runtime_error("tensor not in .llmq: " + name);
    return it->second;
}

std::vector<std::string> QuantFile::names() const {
    std::vector<std::string> v;
    for (const auto& kv : tensors_) v.push_back(kv.first);
    return v;
}

std::vector<std::string> QuantFile::names_in_file() const {
    std::vector<std::pair<size_t, std::string>> v;
    for (const auto& kv : offset_) v.emplace_back(kv.second, kv.first);
    std::sort(v.begin(), v.end());
    std::vector<std::string> out;
    for (auto& p : v) out.push_back(p.second);
    return out;
}

// ------------------------------------------------------------------ config
// The integer fields are required; the optional ones have the documented
// Hugging Face defaults (head_dim = hidden / heads; attention_bias is true
// for Qwen2, whose config class always uses q/k/v biases).
ModelConfig ModelConfig::from_file(const std::string& path) {
    const std::string text = read_file(path);
    const JVal j = parse_json(text.data(), text.data() + text.size());
    auto bad = [&](const std::string& why) { return std::runtime_error("config " + path + ": " + why); };
    ModelConfig c;

    static const std::pair<const char*, int64_t ModelConfig::*> kInts[] = {
        {"hidden_size", &ModelConfig::hidden_size},
        {"intermediate_size", &ModelConfig::intermediate_size},
        {"num_attention_heads", &ModelConfig::num_attention_heads},
        {"num_hidden_layers", &ModelConfig::num_hidden_layers},
        {"num_key_value_heads", &ModelConfig::num_key_value_heads},
        {"vocab_size", &ModelConfig::vocab_size},
    };
    for (const auto& f : kInts) c.*(f.second) = j.at(f.first).as_int();
    c.rms_norm_eps = j.at("rms_norm_eps").as_double();
    c.rope_theta = j.at("rope_theta").as_double();

    const JVal& archs = j.at("architectures");
    if (archs.type != JVal::kArr || archs.arr.empty()) throw bad("\"architectures\" names no class");
    c.architecture = archs.arr.front().as_str();

    if (c.num_attention_heads <= 0 || c.num_key_value_heads <= 0) throw bad("head counts must be positive");
    if (c.num_attention_heads % c.num_key_value_heads)
        throw bad("query heads must be a multiple of the key/value heads");
    const int64_t per_head = c.hidden_size / c.num_attention_heads;
    const JVal* hd = j.find("head_dim");
    c.head_dim = (hd && hd->type == JVal::kNum) ? hd->as_int() : per_head;
    if (c.head_dim != per_head) throw bad("head_dim differs from hidden_size / num_attention_heads");

    const JVal* tie = j.find("tie_word_embeddings");
    c.tie_word_embeddings = tie && tie->type == JVal::kBool && tie->b;
    const JVal* ab = j.find("attention_bias");
    c.attention_bias = (ab && ab->type == JVal::kBool) ? ab->b : c.architecture == "Qwen2ForCausalLM";
    return c;
}

// ------------------------------------------------------------------ model
std::string QuantModel::file_for(const std::string& dir, QKind kind) {
    return dir + (kind == QKind::kInt4 ? "/model.q4.llmq" : "/model.q8.llmq");
}

namespace {

// Sizes a tensor's rows / cols are checked against.
enum Dim { kHidden, kQOut, kKvOut, kInter, kVocab, kOne };

struct Want {
    const char* suffix;           // tensor name after "model.layers.<i>."
    QTensor QLayer::*field;
    Dim rows, cols;               // cols == kOne: a bf16 vector
    bool bias_only;               // present only with attention biases
};

// Every tensor a decoder layer reads, with the shape it must have.
const Want kLayerTensors[] = {
    {"self_attn.q_proj.weight", &QLayer::q_w, kQOut, kHidden, false},
    {"self_attn.k_proj.weight", &QLayer::k_w, kKvOut, kHidden, false},
    {"self_attn.v_proj.weight", &QLayer::v_w, kKvOut, kHidden, false},
    {"self_attn.o_proj.weight", &QLayer::o_w, kHidden, kQOut, false},
    {"mlp.gate_proj.weight", &QLayer::gate_w, kInter, kHidden, false},
    {"mlp.up_proj.weight", &QLayer::up_w, kInter, kHidden, false},
    {"mlp.down_proj.weight", &QLayer::down_w, kHidden, kInter, false},
    {"input_layernorm.weight", &QLayer::input_ln, kHidden, kOne, false},
    {"post_attention_layernorm.weight", &QLayer::post_attn_ln, kHidden, kOne, false},
    {"self_attn.q_proj.bias", &QLayer::q_b, kQOut, kOne, true},
    {"self_attn.k_proj.bias", &QLayer::k_b, kKvOut, kOne, true},
    {"self_attn.v_proj.bias", &QLayer::v_b, kKvOut, kOne, true},
};

}  // namespace

void QuantModel::load(const std::string& dir, QKind k) {
    const ModelConfig c = ModelConfig::from_file(dir + "/config.json");
    const int64_t size[] = {c.hidden_size, c.num_attention_heads * c.head_dim, c.num_key_value_heads * c.head_dim,
                            c.intermediate_size, c.vocab_size, 1};
    file_.open(file_for(dir, k));
    // One tensor of the file, checked: matrices must be of kind k, vectors bf16.
    auto take = [&](const std::string& name, Dim rows, Dim cols) -> QTensor {
        const QTensor& t = file_.get(name);
        const bool vec = cols == kOne;
        const QKind want = vec ? QKind::kBf16 : k;
        if (t.kind != want)
            throw std::runtime_error(name + ": stored as " + qkind_name(t.kind) + ", expected " + qkind_name(want));
        if (t.rows != size[rows] || (!vec && t.cols != size[cols]))
            throw std::runtime_error(name + ": stored shape " + std::to_string(t.rows) + "x" + std::to_string(t.cols) +
                                     " does not match config.json");
        return t;
    };
    std::vector<QLayer> ls(size_t(c.num_hidden_layers));
    for (size_t i = 0; i < ls.size(); i++) {
        const std::string prefix = "model.layers." + std::to_string(i) + ".";
        ls[i].has_bias = c.attention_bias;
        for (const Want& w : kLayerTensors)
            if (!w.bias_only || c.attention_bias) ls[i].*(w.field) = take(prefix + w.suffix, w.rows, w.cols);
    }
    embed_tokens = take("model.embed_tokens.weight", kVocab, kHidden);
    lm_head = c.tie_word_embeddings ? QTensor{} : take("lm_head.weight", kVocab, kHidden);
    final_norm = take("model.norm.weight", kHidden, kOne);
    layers = std::move(ls);
    cfg = c;
    kind = k;
}

// ------------------------------------------------------------------ device
namespace gpu {

static_assert(sizeof(QuantView) == sizeof(iq_view), "QuantView must match iq_view");
static_assert(offsetof(QuantView, q) == offsetof(iq_view, q), "QuantView must match iq_view");
static_assert(offsetof(QuantView, zeros) == offsetof(iq_view, zeros), "QuantView must match iq_view");

namespace {
const iq_view* as_iq(const QuantView& W) { return reinterpret_cast<const iq_view*>(&W); }
}  // namespace

void launch_gemv_batched_q(const float* x, const QuantView& W, const uint16_t* bias, int B, int64_t in, int64_t out,
                           float* y, hipStream_t stream) {
    iq_check(iq_gemv(x, as_iq(W), bias, B, in, out, y, stream), "launch_gemv_batched_q");
}

void launch_gemm_tiled_q(const float* x, const QuantView& W, const uint16_t* bias, int64_t T, int64_t in,
                         int64_t out, float* y, hipStream_t stream) {
    iq_check(iq_gemm(x, as_iq(W), bias, T, in, out, y, stream), "launch_gemm_tiled_q");
}

void launch_embedding_q(const QuantView& table, const int64_t* ids, int64_t T, int64_t H, float* out,
                        hipStream_t stream) {
    iq_check(iq_embedding(as_iq(table), ids, T, H, out, stream), "launch_embedding_q");
}

void linear_q(const float* x, const QuantView& W, const uint16_t* bias, int64_t T, int64_t in, int64_t out,
              float* y, hipStream_t stream) {
    iq_check(iq_linear(x, as_iq(W), bias, T, in, out, y, stream), "linear_q");
}

DevQuant::DevQuant(const QTensor& t) {
    if (t.kind == QKind::kBf16) {
        const size_t n = size_t(t.rows) * size_t(t.cols) * 2;
        if (!n) return;
        hip_check(hipMalloc(&data_, n), "DevQuant: hipMalloc");
        hip_check(hipMemcpy(data_, t.bf16, n, hipMemcpyHostToDevice), "DevQuant: upload");
        view_ = QuantView{QuantKind::kInt8, t.rows, t.cols, 0, nullptr, nullptr, nullptr};
        return;
    }
    const size_t nq = t.q_bytes(), ns = size_t(t.rows * t.groups()) * 2, nz = t.zeros ? size_t(t.rows * t.groups()) : 0;
    // q | scales | zeros in one allocation; the scales start 256-byte aligned
    const size_t so = (nq + 255) & ~size_t(255), zo = so + ns;
    hip_check(hipMalloc(&data_, zo + nz), "DevQuant: hipMalloc");
    char* d = static_cast<char*>(data_);
    try {
        hip_check(hipMemcpy(d, t.q, nq, hipMemcpyHostToDevice), "DevQuant: upload");
        hip_check(hipMemcpy(d + so, t.scales, ns, hipMemcpyHostToDevice), "DevQuant: upload");
        if (nz) hip_check(hipMemcpy(d + zo, t.zeros, nz, hipMemcpyHostToDevice), "DevQuant: upload");
    } catch (...) {
        release();
        throw;
    }
    view_ = QuantView{t.kind == QKind::kInt4 ? QuantKind::kInt4 : QuantKind::kInt8,
                      t.rows,
                      t.cols,
                      t.groups(),
                      reinterpret_cast<const uint8_t*>(d),
                      reinterpret_cast<const uint16_t*>(d + so),
                      nz ? reinterpret_cast<const uint8_t*>(d + zo) : nullptr};
}

void DevQuant::release() {
    if (data_) (void)hipFree(data_);
    data_ = nullptr;
    view_ = QuantView{};
}

DevQuant::~DevQuant() { release(); }

DevQuant::DevQuant(DevQuant&& o) noexcept : data_(o.data_), view_(o.view_) {
    o.data_ = nullptr;
    o.view_ = QuantView{};
}

DevQuant& DevQuant::operator=(DevQuant&& o) noexcept {
    if (this != &o) {
        release();
        data_ = o.data_;
        view_ = o.view_;
        o.data_ = nullptr;
        o.view_ = QuantView{};
    }
    return *this;
}

DevQuantModel::DevQuantModel(const QuantModel& m)
    : embed_tokens(m.embed_tokens), lm_head(m.lm_head.rows ? DevQuant(m.lm_head) : DevQuant()),
      final_norm(m.final_norm) {
    layers.reserve(m.layers.size());
    for (const QLayer& L : m.layers) {
        DevLayer d;
        d.q_w = DevQuant(L.q_w);
        d.k_w = DevQuant(L.k_w);
        d.v_w = DevQuant(L.v_w);
        d.o_w = DevQuant(L.o_w);
        d.gate_w = DevQuant(L.gate_w);
        d.up_w = DevQuant(L.up_w);
        d.down_w = DevQuant(L.down_w);
        d.input_ln = DevQuant(L.input_ln);
        d.post_attn_ln = DevQuant(L.post_attn_ln);
        if (L.has_bias) {
            d.q_b = DevQuant(L.q_b);
            d.k_b = DevQuant(L.k_b);
            d.v_b = DevQuant(L.v_b);
        }
        layers.push_back(std::move(d));
    }
}

namespace {
iq_view to_iq(const QuantView& v) {
    iq_view r;
    std::memcpy(&r, &v, sizeof(r));
    return r;
}
}  // namespace

DecodeStep::DecodeStep(const DevQuantModel& m, const ModelConfig& cfg, int rows) : m_(m) {
    const int64_t H = cfg.hidden_size, I = cfg.intermediate_size, V = cfg.vocab_size;
    const int64_t hd = cfg.head_dim, nh = cfg.num_attention_heads, nkv = cfg.num_key_value_heads;
    const int64_t qo = nh * hd, kvo = nkv * hd, L = cfg.num_hidden_layers;
    H_ = H;
    V_ = V;
    if (rows < 1 || rows > 32) throw std::runtime_error("DecodeStep: rows must be 1..32");
    B_ = rows;
    if (int64_t(m.layers.size()) != L) throw std::runtime_error("DecodeStep: model and config disagree on layers");
    // arena: h0, per layer q, k, v, h1, act, h2, then logits, each [B][n];
    // each block on its own 1 KiB boundary
    const int64_t B = rows;
    auto pad = [B](int64_t n) { return (B * n + 255) / 256 * 256; };
    int64_t total = pad(H) + L * (pad(qo) + 2 * pad(kvo) + 2 * pad(H) + pad(I)) + pad(V);
    hip_check(hipMalloc(reinterpret_cast<void**>(&arena_), size_t(total) * 4), "DecodeStep: hipMalloc");
    if (hipMalloc(reinterpret_cast<void**>(&ids_), size_t(8 * B)) != hipSuccess) {
        (void)hipFree(arena_);
        throw std::runtime_error("DecodeStep: hipMalloc");
    }
    float* cur = arena_;
    auto take = [&](int64_t n) {
        float* p = cur;
        cur += pad(n);
        return p;
    };
    std::vector<iq_stage> st;
    float* h = take(H);
    h_.push_back(h);
    const float eps = float(cfg.rms_norm_eps);
    for (int64_t l = 0; l < L; l++) {
        const DevLayer& D = m.layers[size_t(l)];
        float *q = take(qo), *k = take(kvo), *v = take(kvo), *h1 = take(H), *act = take(I), *h2 = take(H);
        iq_stage a{};
        a.rows = rows;
        a.in_op = IQ_IN_RMSNORM;
        a.out_op = IQ_OUT_STORE;
        a.n = 3;
        a.eps = eps;
        a.x = h;
        a.norm = D.input_ln.bf16();
        a.W[0] = to_iq(D.q_w.view());
        a.W[1] = to_iq(D.k_w.view());
        a.W[2] = to_iq(D.v_w.view());
        a.bias[0] = D.q_b.empty() ? nullptr : D.q_b.bf16();
        a.bias[1] = D.k_b.empty() ? nullptr : D.k_b.bf16();
        a.bias[2] = D.v_b.empty() ? nullptr : D.v_b.bf16();
        a.y[0] = q;
        a.y[1] = k;
        a.y[2] = v;
        st.push_back(a);
        iq_stage o{};
        o.rows = rows;
        o.in_op = IQ_IN_GQA;
        o.out_op = IQ_OUT_RESIDUAL;
        o.n = 1;
        o.gqa_head_dim = int32_t(hd);
        o.gqa_group = int32_t(nh / nkv);
        o.x = v;
        o.residual = h;
        o.W[0] = to_iq(D.o_w.view());
        o.y[0] = h1;
        st.push_back(o);
        iq_stage g{};
        g.rows = rows;
        g.in_op = IQ_IN_RMSNORM;
        g.out_op = IQ_OUT_SWIGLU;
        g.n = 2;
        g.eps = eps;
        g.x = h1;
        g.norm = D.post_attn_ln.bf16();
        g.W[0] = to_iq(D.gate_w.view());
        g.W[1] = to_iq(D.up_w.view());
        g.y[0] = act;
        st.push_back(g);
        iq_stage d{};
        d.rows = rows;
        d.in_op = IQ_IN_PLAIN;
        d.out_op = IQ_OUT_RESIDUAL;
        d.n = 1;
        d.x = act;
        d.residual = h1;
        d.W[0] = to_iq(D.down_w.view());
        d.y[0] = h2;
        st.push_back(d);
        h = h2;
        h_.push_back(h);
    }
    logits_ = take(V);
    iq_stage f{};
    f.rows = rows;
    f.in_op = IQ_IN_RMSNORM;
    f.out_op = IQ_OUT_STORE;
    f.n = 1;
    f.eps = eps;
    f.x = h;
    f.norm = m.final_norm.bf16();
    f.W[0] = to_iq(m.head());
    f.y[0] = logits_;
    st.push_back(f);
    const int rc = iq_chain_create(st.data(), int(st.size()), &chain_);
    if (rc != IQ_OK) {
        (void)hipFree(arena_);
        (void)hipFree(ids_);
        throw std::runtime_error(std::string("DecodeStep: ") + iq_error_string(rc));
    }
}

DecodeStep::~DecodeStep() {
    if (chain_) iq_chain_destroy(chain_);
    if (arena_) (void)hipFree(arena_);
    if (ids_) (void)hipFree(ids_);
}

void DecodeStep::step(int64_t token, hipStream_t stream) {
    const std::vector<int64_t> t(size_t(B_), token);
    step(t.data(), B_, stream);
}

void DecodeStep::step(const int64_t* tokens, int n, hipStream_t stream) {
    if (n != B_) throw std::runtime_error("DecodeStep: one token per row expected");
    for (int i = 0; i < n; i++)
        if (tokens[i] < 0 || tokens[i] >= V_) throw std::runtime_error("DecodeStep: token id out of range");
    hip_check(hipMemcpyAsync(ids_, tokens, size_t(8 * n), hipMemcpyHostToDevice, stream), "DecodeStep: id upload");
    // (the copy has read the caller's array when this returns)
    hip_check(hipStreamSynchronize(stream), "DecodeStep: id upload");
    run(stream);
}

void DecodeStep::run(hipStream_t stream) {
    iq_check(iq_embedding(reinterpret_cast<const iq_view*>(&m_.embed_tokens.view()), ids_, B_, H_, h_[0], stream),
             "DecodeStep: embedding");
    iq_check(iq_chain_run(chain_, stream), "DecodeStep: chain");
}

const float* DecodeStep::hidden(int layer) const {
    if (layer < 0 || size_t(layer) >= h_.size()) throw std::runtime_error("DecodeStep: no such layer");
    return h_[size_t(layer)];
}

}  // namespace gpu
}  // namespace llm

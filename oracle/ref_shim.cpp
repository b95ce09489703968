// ref_shim.cpp -- C entry points over the reference's OWN quantiser, compiled
// from the reference sources where they lie (/root/reference/src/quant.cpp,
// model_config.cpp, loader.cpp) by oracle/Makefile into oracle/_ref/.
//
// TEST INFRASTRUCTURE ONLY: used in the build container to write the golden
// fixtures under tests/golden/ and to cross-check oracle/iq_oracle.c.  It is
// not part of libiq.so, never built on the GPU box (the reference tree is
// absent there), and its build output (oracle/_ref) is excluded from the
// tree copied to the GPU machines.
#include "quant.h"
#include "f16.h"

#include <cstring>
#include <stdexcept>

extern "C" {

// llm::quantize (src/quant.cpp:34-84).  kind: 0 = int8, 1 = int4.
// Returns 0, or -1 when the reference threw.
int ref_quantize(const uint16_t* w, int64_t rows, int64_t cols, int kind, uint8_t* q,
                 uint16_t* scales, uint8_t* zeros) {
    try {
        llm::QMatrix m = llm::quantize(w, rows, cols, kind == 0 ? llm::QKind::kInt8 : llm::QKind::kInt4);
        std::memcpy(q, m.q.data(), m.q.size());
        std::memcpy(scales, m.scales.data(), m.scales.size() * 2);
        if (!m.zeros.empty()) std::memcpy(zeros, m.zeros.data(), m.zeros.size());
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// llm::dequant (src/quant.cpp:86-93) over a whole matrix.
void ref_dequant_matrix(const uint8_t* q, const uint16_t* scales, const uint8_t* zeros, int kind,
                        int64_t rows, int64_t cols, float* out) {
    llm::QTensor t;
    t.kind = kind == 0 ? llm::QKind::kInt8 : llm::QKind::kInt4;
    t.rows = rows; t.cols = cols; t.q = q; t.scales = scales; t.zeros = zeros;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < cols; c++) out[r * cols + c] = llm::dequant(t, r, c);
}

uint16_t ref_f32_to_bf16(float f) { return f16::f32_to_bf16(f); }

// QuantWriter + QuantFile round trip (src/quant.cpp:96-191): writes one
// quantised matrix `name` and reads it back; returns 0 when the views match.
int ref_llmq_write(const char* path, const char* name, const uint8_t* q, const uint16_t* scales,
                   const uint8_t* zeros, int kind, int64_t rows, int64_t cols) {
    try {
        llm::QMatrix m;
        m.kind = kind == 0 ? llm::QKind::kInt8 : llm::QKind::kInt4;
        m.rows = rows; m.cols = cols;
        const int64_t G = (cols + llm::kGroup - 1) / llm::kGroup;
        m.q.assign(q, q + (kind == 1 ? rows * cols / 2 : rows * cols));
        m.scales.assign(scales, scales + rows * G);
        if (kind == 1) m.zeros.assign(zeros, zeros + rows * G);
        llm::QuantWriter wr;
        wr.add(name, m);
        wr.write(path);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// A QuantWriter (src/quant.h:68-77) behind a handle, for multi-tensor files.
void* ref_writer_new() { return new llm::QuantWriter(); }
void ref_writer_free(void* h) { delete static_cast<llm::QuantWriter*>(h); }

int ref_writer_add(void* h, const char* name, const uint8_t* q, const uint16_t* scales,
                   const uint8_t* zeros, int kind, int64_t rows, int64_t cols) {
    try {
        llm::QMatrix m;
        m.kind = kind == 0 ? llm::QKind::kInt8 : llm::QKind::kInt4;
        m.rows = rows; m.cols = cols;
        const int64_t G = (cols + llm::kGroup - 1) / llm::kGroup;
        m.q.assign(q, q + (kind == 1 ? rows * cols / 2 : rows * cols));
        m.scales.assign(scales, scales + rows * G);
        if (kind == 1) m.zeros.assign(zeros, zeros + rows * G);
        static_cast<llm::QuantWriter*>(h)->add(name, m);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_writer_add_bf16(void* h, const char* name, const uint16_t* data, int64_t n) {
    try {
        static_cast<llm::QuantWriter*>(h)->add_bf16(name, data, {n});
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

int ref_writer_write(void* h, const char* path) {
    try {
        static_cast<llm::QuantWriter*>(h)->write(path);
        return 0;
    } catch (const std::exception&) {
        return -1;
    }
}

// llm::QuantModel::load (src/quant.cpp:198-238): returns the number of layers
// loaded, or -1 when the reference rejected the directory.
int ref_quantmodel_layers(const char* dir, int kind) {
    try {
        llm::QuantModel m;
        m.load(dir, kind == 0 ? llm::QKind::kInt8 : llm::QKind::kInt4);
        return int(m.layers.size());
    } catch (const std::exception&) {
        return -1;
    }
}
}

// GGUF v3 writer and GGML block quantizers (Q4_0, Q8_0, Q4_K, Q6_K).
//
// The reference reads GGUF but never writes it; this module exists so that the
// synthetic benchmark models can be produced offline with any valid encoding.
// The layout written here is exactly what the reader expects
// (core/gguf_parser.cpp:164-324): header, KV metadata, tensor table, data
// section aligned to 32 bytes from the file start, each tensor aligned to 32
// inside the data section (or to `alignment`, declared as general.alignment).
#pragma once
#include "gguf_types.hpp"
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>
#include <functional>

namespace orc {

// Quantize `n` floats (a multiple of the block size) into `out`.
void quantize_q8_0(const float* x, int64_t n, uint8_t* out);
void quantize_q4_0(const float* x, int64_t n, uint8_t* out);
void quantize_q4_k(const float* x, int64_t n, uint8_t* out);
void quantize_q6_k(const float* x, int64_t n, uint8_t* out);
// Dispatch on type (F32 copies, F16 rounds). Returns false on an unsupported type.
bool quantize_any(GGMLType t, const float* x, int64_t n, uint8_t* out);
// Bytes a row of `n` elements of type `t` takes (0 if unsupported).
uint64_t row_bytes(GGMLType t, int64_t n);

struct GGUFWriter {
    struct KV {
        std::string key;
        uint32_t kind;                  // GGUF value type id
        std::string s;                  // kind 8
        uint64_t u = 0;                 // kinds 4, 10
        float f = 0.f;                  // kind 6
        std::vector<std::string> arr;   // kind 9, element type 8 (strings)
        std::vector<int32_t> ai;        // kind 9, element type 5 (int32), when arr is empty
    };
    struct Tensor {
        std::string name;
        std::vector<uint64_t> shape;    // shape[0] is the contiguous dimension
        GGMLType type;
        uint64_t offset = 0;
        uint64_t nbytes = 0;
        // Produces rows [r0, r1) of the tensor already encoded into `dst`.
        std::function<void(int64_t r0, int64_t r1, uint8_t* dst)> fill;
    };
    std::vector<KV> kvs;
    std::vector<Tensor> tensors;
    // Data-section and tensor alignment (a power of two). Other than 32 it is
    // declared as general.alignment, as the GGUF format defines; the
    // reference's reader supports 32 only (core/gguf_parser.cpp:30, 196).
    uint64_t alignment = 32;

    void add_str(const std::string& k, const std::string& v);
    void add_u32(const std::string& k, uint32_t v);
    void add_f32(const std::string& k, float v);
    void add_str_array(const std::string& k, const std::vector<std::string>& v);
    void add_i32_array(const std::string& k, const std::vector<int32_t>& v);
    void add_tensor(const std::string& name, std::vector<uint64_t> shape, GGMLType type,
                    std::function<void(int64_t, int64_t, uint8_t*)> fill);
    // Writes the file; returns false on an I/O error.
    bool write(const std::string& path, bool verbose = false);
};

}  // namespace orc

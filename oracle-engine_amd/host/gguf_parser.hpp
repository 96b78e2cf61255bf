// GGUFParser — the reference's GGUF reader API (core/gguf_parser.hpp:26-176)
// with the weight bytes resident in HBM.
//
// load() maps the file, parses header / KV metadata / tensor table exactly as
// the reference does (core/gguf_parser.cpp:80-324: data section aligned to 32
// bytes from the file start, types restricted to F32/F16/BF16/Q4_0/Q8_0/Q4_K/
// Q6_K) and uploads the whole data section to one HBM allocation unchanged
// (no dequant-to-float expansion). gemv_q / gemv_q_range / gemm_q /
// dequantize_row keep their host-pointer signatures for drop-in callers and
// run on the GPU; the model uses the device pointers directly.
//
// A tensor's HBM bytes may be re-laid out once after load (regroup_q8_0); the
// parser records each tensor's device layout and every device drop-in reads
// the bytes in that layout, so results stay those of the file's tensor.
#pragma once
#include "gguf_types.hpp"

#include <cstdint>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

struct MetaValue {
    enum Kind { U8, I8, U16, I16, U32, I32, F32, BOOL, STR, U64, I64, F64, ARR_STR, ARR_I32, ARR_U32, ARR_F32, SKIP } kind =
        SKIP;
    union {
        uint8_t u8;
        int8_t i8;
        uint16_t u16;
        int16_t i16;
        uint32_t u32;
        int32_t i32;
        float f32;
        bool b;
        uint64_t u64;
        int64_t i64;
        double f64;
    };
    std::string str;
    std::vector<std::string> arr_str;
    std::vector<int32_t> arr_i32;
    std::vector<uint32_t> arr_u32;
    std::vector<float> arr_f32;
    MetaValue() : u64(0) {}
};

struct TensorInfo {
    std::string name;
    std::vector<uint64_t> shape;  // shape[0] is the contiguous dimension
    GGMLType type = GGMLType::UNKNOWN;
    uint64_t offset = 0;          // from the start of the data section
    uint64_t n_elems() const;
    uint64_t n_bytes() const;
};

class GGUFParser {
public:
    GGUFParser() = default;
    ~GGUFParser() { close(); }
    GGUFParser(const GGUFParser&) = delete;
    GGUFParser& operator=(const GGUFParser&) = delete;

    // Parses and uploads; false (with a message on stderr) on any error.
    bool load(const std::string& path);
    // Parses the header, metadata and tensor table only, with the weights
    // left in the file mapping (is_mmap_only(); the device drop-ins then
    // refuse): enough for a Tokenizer, and needs no GPU.
    bool load_meta(const std::string& path);
    void close();
    bool is_open() const { return map_ != nullptr; }

    bool has_meta(const std::string& key) const;
    const MetaValue& meta(const std::string& key) const;
    uint32_t meta_u32(const std::string& key, uint32_t def = 0) const;
    int32_t meta_i32(const std::string& key, int32_t def = 0) const;
    uint64_t meta_u64(const std::string& key, uint64_t def = 0) const;
    float meta_f32(const std::string& key, float def = 0.f) const;
    std::string meta_str(const std::string& key, const std::string& def = "") const;
    const std::vector<std::string>& meta_arr_str(const std::string& key) const;

    bool has_tensor(const std::string& name) const;
    const TensorInfo& tensor_info(const std::string& name) const;
    const uint8_t* tensor_raw(const std::string& name) const;     // host (mapped) bytes
    const uint8_t* tensor_device(const std::string& name) const;  // HBM bytes
    std::vector<std::string> tensor_names() const;

    // Layout of the tensor's HBM bytes as an orc.h type id: the GGML type of
    // the file, or ORC_Q8_0_X8 after regroup_q8_0; -1 for an unknown name.
    int device_type(const std::string& name) const;
    // Rewrites a Q8_0 matrix's HBM bytes in the aligned ORC_Q8_0_X8 layout
    // (same bytes per row, same values; rows of a multiple of 256 values,
    // 16-byte aligned data). Once per tensor; false if not eligible.
    bool regroup_q8_0(const std::string& name);

    // Host-pointer drop-ins of the reference kernels (run on the GPU; host
    // buffers in and out, device scratch reused across calls; thread-safe).
    std::vector<float> dequantize(const std::string& name) const;
    void dequantize_into(const std::string& name, std::vector<float>& out) const;
    void dequantize_row(const std::string& name, int64_t row, float* out) const;
    bool gemv_q(const std::string& name, float* out, const float* x, int n_out, int n_in) const;
    bool gemv_q_range(const std::string& name, float* out, const float* x, int j0, int j1, int n_in) const;
    bool gemm_q(const std::string& name, float* out, const float* x, int n_tokens, int n_out, int n_in) const;

    uint32_t version() const { return version_; }
    uint64_t n_tensors() const { return n_tensors_; }
    uint64_t n_meta() const { return meta_.size(); }
    uint64_t file_size() const { return (uint64_t)fsize_; }
    uint64_t data_bytes() const { return fsize_ - data_start_; }
    // core/gguf_parser.hpp:125: true when the weights were not preloaded and
    // are served from the file mapping (the Engine then skips its warmup).
    // Here the data section always lives in HBM once load() succeeds.
    bool is_mmap_only() const { return d_data_ == nullptr; }

    // Test hooks on synthetic blocks (core/gguf_parser.hpp:128-132), run by
    // the device codecs / GEMV on host buffers.
    static void test_dq_q6_k(const uint8_t* s, uint64_t n, float* out) { dq_hook(14, s, n, out); }
    static void test_dq_q4_k(const uint8_t* s, uint64_t n, float* out) { dq_hook(12, s, n, out); }
    static void test_dq_q4_0(const uint8_t* s, uint64_t n, float* out) { dq_hook(2, s, n, out); }
    static float test_dot_q6k(const uint8_t* row, int n_cols, const float* x) { return dot_hook(14, row, n_cols, x); }
    static float test_dot_q4_0(const uint8_t* row, int n_cols, const float* x) { return dot_hook(2, row, n_cols, x); }

private:
    const uint8_t* map_ = nullptr;
    size_t fsize_ = 0;
    int fd_ = -1;
    uint32_t version_ = 0;
    uint64_t n_tensors_ = 0;
    uint64_t data_start_ = 0;
    uint8_t* d_data_ = nullptr;  // HBM copy of the data section
    std::unordered_map<std::string, MetaValue> meta_;
    std::unordered_map<std::string, TensorInfo> tensors_;
    std::unordered_map<std::string, int> dev_type_;  // tensors whose HBM layout differs from the file's
    mutable std::mutex scr_mu_;                      // guards the drop-ins' device scratch
    mutable void* d_scr_ = nullptr;
    mutable size_t scr_cap_ = 0;

    bool parse();
    bool open_file(const std::string& path, bool upload);
    bool gemm_dev(const std::string& name, const TensorInfo& ti, float* out, const float* x, int n_tokens, int j0,
                  int j1, int n_in) const;
    void* scratch(size_t bytes) const;  // caller holds scr_mu_
    static void dq_hook(int type, const uint8_t* s, uint64_t n, float* out);
    static float dot_hook(int type, const uint8_t* row, int n_cols, const float* x);
};

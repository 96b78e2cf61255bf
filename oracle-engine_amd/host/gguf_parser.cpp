#include "gguf_parser.hpp"

#include "orc.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cstdio>
#include <cstring>

uint64_t TensorInfo::n_elems() const {
    if (shape.empty()) return 0;
    uint64_t n = 1;
    for (uint64_t d : shape) n *= d;
    return n;
}

uint64_t TensorInfo::n_bytes() const {
    uint32_t be, bb;
    if (!ggml_block_geom(type, be, bb)) return 0;
    return n_elems() / be * bb;
}

namespace {
// Bounds-checked little-endian cursor over the mapped file.
struct Cursor {
    const uint8_t* p;
    const uint8_t* end;
    bool ok = true;
    bool need(size_t n) {
        if (!ok || (size_t)(end - p) < n) { ok = false; return false; }
        return true;
    }
    template <typename T> T get() {
        T v{};
        if (need(sizeof(T))) { std::memcpy(&v, p, sizeof(T)); p += sizeof(T); }
        return v;
    }
    std::string str() {
        uint64_t n = get<uint64_t>();
        if (!ok || n > (uint64_t)(end - p)) { ok = false; return {}; }
        std::string s((const char*)p, (size_t)n);
        p += n;
        return s;
    }
};

void read_value(Cursor& c, uint32_t kind, MetaValue& v);

void skip_value(Cursor& c, uint32_t kind) {
    MetaValue tmp;
    read_value(c, kind, tmp);
}

// GGUF value types 0..12 (core/gguf_parser.cpp:232-292).
void read_value(Cursor& c, uint32_t kind, MetaValue& v) {
    switch (kind) {
        case 0: v.kind = MetaValue::U8; v.u8 = c.get<uint8_t>(); break;
        case 1: v.kind = MetaValue::I8; v.i8 = c.get<int8_t>(); break;
        case 2: v.kind = MetaValue::U16; v.u16 = c.get<uint16_t>(); break;
        case 3: v.kind = MetaValue::I16; v.i16 = c.get<int16_t>(); break;
        case 4: v.kind = MetaValue::U32; v.u32 = c.get<uint32_t>(); break;
        case 5: v.kind = MetaValue::I32; v.i32 = c.get<int32_t>(); break;
        case 6: v.kind = MetaValue::F32; v.f32 = c.get<float>(); break;
        case 7: v.kind = MetaValue::BOOL; v.b = c.get<uint8_t>() != 0; break;
        case 8: v.kind = MetaValue::STR; v.str = c.str(); break;
        case 10: v.kind = MetaValue::U64; v.u64 = c.get<uint64_t>(); break;
        case 11: v.kind = MetaValue::I64; v.i64 = c.get<int64_t>(); break;
        case 12: v.kind = MetaValue::F64; v.f64 = c.get<double>(); break;
        case 9: {
            const uint32_t at = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            v.kind = at == 8 ? MetaValue::ARR_STR : at == 5 ? MetaValue::ARR_I32 : at == 4 ? MetaValue::ARR_U32
                   : at == 6 ? MetaValue::ARR_F32 : MetaValue::SKIP;
            for (uint64_t i = 0; i < n && c.ok; ++i) {
                if (at == 8) v.arr_str.push_back(c.str());
                else if (at == 5) v.arr_i32.push_back(c.get<int32_t>());
                else if (at == 4) v.arr_u32.push_back(c.get<uint32_t>());
                else if (at == 6) v.arr_f32.push_back(c.get<float>());
                else skip_value(c, at);
            }
            break;
        }
        default: v.kind = MetaValue::SKIP; c.ok = false; break;  // unknown size: cannot continue
    }
}
}  // namespace

bool GGUFParser::load(const std::string& path) { return open_file(path, true); }

bool GGUFParser::load_meta(const std::string& path) { return open_file(path, false); }

bool GGUFParser::open_file(const std::string& path, bool upload) {
    close();
    fd_ = ::open(path.c_str(), O_RDONLY);
    if (fd_ < 0) { std::fprintf(stderr, "[GGUFParser] cannot open %s\n", path.c_str()); return false; }
    struct stat st;
    if (fstat(fd_, &st) != 0) { close(); return false; }
    fsize_ = (size_t)st.st_size;
    void* m = mmap(nullptr, fsize_, PROT_READ, MAP_PRIVATE, fd_, 0);
    if (m == MAP_FAILED) { map_ = nullptr; close(); return false; }
    map_ = (const uint8_t*)m;
    if (!parse()) { close(); return false; }
    for (const auto& kv : tensors_) {  // fail at load, never silently at inference (gguf_parser.cpp:93-110)
        uint32_t be, bb;
        if (!ggml_block_geom(kv.second.type, be, bb)) {
            std::fprintf(stderr, "[GGUFParser] tensor '%s' has unsupported type %u\n", kv.first.c_str(),
                         (unsigned)kv.second.type);
            close();
            return false;
        }
        if (data_start_ + kv.second.offset + kv.second.n_bytes() > fsize_) {
            std::fprintf(stderr, "[GGUFParser] tensor '%s' extends past the end of the file\n", kv.first.c_str());
            close();
            return false;
        }
    }
    if (!upload) return true;
    void* d = nullptr;
    if (orc_init(0) != 0 || orc_upload(map_ + data_start_, fsize_ - data_start_, &d) != 0) {
        std::fprintf(stderr, "[GGUFParser] upload failed: %s\n", orc_last_error());
        close();
        return false;
    }
    d_data_ = (uint8_t*)d;
    return true;
}

void GGUFParser::close() {
    if (d_data_) orc_free(d_data_);
    d_data_ = nullptr;
    {
        std::lock_guard<std::mutex> lk(scr_mu_);
        if (d_scr_) orc_free(d_scr_);
        d_scr_ = nullptr;
        scr_cap_ = 0;
    }
    dev_type_.clear();
    if (map_) munmap((void*)map_, fsize_);
    map_ = nullptr;
    if (fd_ >= 0) ::close(fd_);
    fd_ = -1;
    meta_.clear();
    tensors_.clear();
    version_ = 0;
    n_tensors_ = data_start_ = 0;
    fsize_ = 0;
}

bool GGUFParser::parse() {
    Cursor c{map_, map_ + fsize_};
    if (fsize_ < 4 || std::memcmp(map_, "GGUF", 4) != 0) {
        std::fprintf(stderr, "[GGUFParser] bad magic\n");
        return false;
    }
    c.p += 4;
    version_ = c.get<uint32_t>();
    n_tensors_ = c.get<uint64_t>();
    const uint64_t n_kv = c.get<uint64_t>();
    for (uint64_t i = 0; i < n_kv && c.ok; ++i) {
        std::string key = c.str();
        const uint32_t kind = c.get<uint32_t>();
        MetaValue v;
        read_value(c, kind, v);
        if (c.ok) meta_.emplace(std::move(key), std::move(v));
    }
    for (uint64_t i = 0; i < n_tensors_ && c.ok; ++i) {
        TensorInfo ti;
        ti.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (nd > 8) { c.ok = false; break; }
        for (uint32_t d = 0; d < nd && c.ok; ++d) ti.shape.push_back(c.get<uint64_t>());
        ti.type = (GGMLType)c.get<uint32_t>();
        ti.offset = c.get<uint64_t>();
        if (c.ok) tensors_.emplace(ti.name, std::move(ti));
    }
    if (!c.ok) {
        std::fprintf(stderr, "[GGUFParser] truncated or corrupt header\n");
        return false;
    }
    // The data section starts at the next multiple of general.alignment (32
    // when absent, the only value the reference supports: gguf_parser.cpp:30,
    // 196, where the key is ignored; for files that declare 32 or nothing the
    // two readers agree).
    uint64_t align = 32;
    auto al = meta_.find("general.alignment");
    if (al != meta_.end() && al->second.kind == MetaValue::U32) align = al->second.u32;
    if (align == 0 || (align & (align - 1)) || align > 65536) {
        std::fprintf(stderr, "[GGUFParser] general.alignment %llu is not a power of two\n", (unsigned long long)align);
        return false;
    }
    data_start_ = ((uint64_t)(c.p - map_) + align - 1) & ~(align - 1);
    if (data_start_ > fsize_) return false;
    return true;
}

bool GGUFParser::has_meta(const std::string& k) const { return meta_.count(k) > 0; }
const MetaValue& GGUFParser::meta(const std::string& k) const {
    static const MetaValue none;
    auto it = meta_.find(k);
    return it == meta_.end() ? none : it->second;
}
uint32_t GGUFParser::meta_u32(const std::string& k, uint32_t def) const {
    auto it = meta_.find(k);
    if (it == meta_.end()) return def;
    switch (it->second.kind) {
        case MetaValue::U32: return it->second.u32;
        case MetaValue::I32: return (uint32_t)it->second.i32;
        case MetaValue::U64: return (uint32_t)it->second.u64;
        default: return def;
    }
}
int32_t GGUFParser::meta_i32(const std::string& k, int32_t def) const {
    auto it = meta_.find(k);
    if (it == meta_.end()) return def;
    if (it->second.kind == MetaValue::I32) return it->second.i32;
    if (it->second.kind == MetaValue::U32) return (int32_t)it->second.u32;
    return def;
}
uint64_t GGUFParser::meta_u64(const std::string& k, uint64_t def) const {
    auto it = meta_.find(k);
    if (it == meta_.end()) return def;
    if (it->second.kind == MetaValue::U64) return it->second.u64;
    if (it->second.kind == MetaValue::U32) return it->second.u32;
    return def;
}
float GGUFParser::meta_f32(const std::string& k, float def) const {
    auto it = meta_.find(k);
    if (it == meta_.end()) return def;
    if (it->second.kind == MetaValue::F32) return it->second.f32;
    if (it->second.kind == MetaValue::F64) return (float)it->second.f64;
    return def;
}
std::string GGUFParser::meta_str(const std::string& k, const std::string& def) const {
    auto it = meta_.find(k);
    return it != meta_.end() && it->second.kind == MetaValue::STR ? it->second.str : def;
}
const std::vector<std::string>& GGUFParser::meta_arr_str(const std::string& k) const {
    static const std::vector<std::string> none;
    auto it = meta_.find(k);
    return it != meta_.end() && it->second.kind == MetaValue::ARR_STR ? it->second.arr_str : none;
}

bool GGUFParser::has_tensor(const std::string& n) const { return tensors_.count(n) > 0; }
const TensorInfo& GGUFParser::tensor_info(const std::string& n) const {
    static const TensorInfo none;
    auto it = tensors_.find(n);
    return it == tensors_.end() ? none : it->second;
}
const uint8_t* GGUFParser::tensor_raw(const std::string& n) const {
    auto it = tensors_.find(n);
    return it == tensors_.end() ? nullptr : map_ + data_start_ + it->second.offset;
}
const uint8_t* GGUFParser::tensor_device(const std::string& n) const {
    auto it = tensors_.find(n);
    return it == tensors_.end() || !d_data_ ? nullptr : d_data_ + it->second.offset;
}
std::vector<std::string> GGUFParser::tensor_names() const {
    std::vector<std::string> v;
    for (const auto& kv : tensors_) v.push_back(kv.first);
    std::sort(v.begin(), v.end());
    return v;
}

// ── device layout ────────────────────────────────────────────────────────────
int GGUFParser::device_type(const std::string& name) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) return -1;
    auto d = dev_type_.find(name);
    return d != dev_type_.end() ? d->second : (int)it->second.type;
}

bool GGUFParser::regroup_q8_0(const std::string& name) {
    auto it = tensors_.find(name);
    if (it == tensors_.end() || !d_data_ || it->second.type != GGMLType::Q8_0 || dev_type_.count(name)) return false;
    const TensorInfo& ti = it->second;
    if (ti.shape.empty() || ti.shape[0] % 256 || ((uintptr_t)tensor_device(name) & 15)) return false;
    if (orc_q8_0_regroup((void*)tensor_device(name), (int64_t)(ti.n_elems() / 256), nullptr) != 0) return false;
    dev_type_[name] = ORC_Q8_0_X8;
    return true;
}

// ── host-pointer drop-ins, executed on the device ────────────────────────────
void* GGUFParser::scratch(size_t bytes) const {
    bytes = (bytes + 255) & ~size_t(255);
    if (bytes > scr_cap_) {
        if (d_scr_) orc_free(d_scr_);
        d_scr_ = nullptr;
        scr_cap_ = 0;
        if (orc_malloc(&d_scr_, bytes) != 0) return nullptr;
        scr_cap_ = bytes;
    }
    return d_scr_;
}

void GGUFParser::dequantize_into(const std::string& name, std::vector<float>& out) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) return;
    const TensorInfo& ti = it->second;
    const uint64_t n = ti.n_elems();
    if (!n) return;
    if (out.size() < n) out.resize(n);
    if (ti.type == GGMLType::BF16) {  // plain widening, no device kernel needed
        const uint16_t* s = (const uint16_t*)tensor_raw(name);
        for (uint64_t i = 0; i < n; ++i) { uint32_t f = (uint32_t)s[i] << 16; std::memcpy(&out[i], &f, 4); }
        return;
    }
    std::lock_guard<std::mutex> lk(scr_mu_);
    void* y = scratch(n * 4);
    if (y && orc_dequant(device_type(name), tensor_device(name), (int64_t)n, (float*)y, nullptr) == 0)
        orc_memcpy_d2h(out.data(), y, n * 4, nullptr);
}

std::vector<float> GGUFParser::dequantize(const std::string& name) const {
    std::vector<float> v;
    dequantize_into(name, v);
    return v;
}

void GGUFParser::dequantize_row(const std::string& name, int64_t row, float* out) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end() || !out) return;
    const TensorInfo& ti = it->second;
    const uint64_t cols = ti.shape.empty() ? 0 : ti.shape[0];
    uint32_t be, bb;
    ggml_block_geom(ti.type, be, bb);
    const uint64_t rb = cols / be * bb;
    if (ti.type == GGMLType::BF16) {
        const uint16_t* s = (const uint16_t*)(tensor_raw(name) + row * rb);
        for (uint64_t i = 0; i < cols; ++i) { uint32_t f = (uint32_t)s[i] << 16; std::memcpy(&out[i], &f, 4); }
        return;
    }
    std::lock_guard<std::mutex> lk(scr_mu_);
    void* y = scratch(cols * 4);
    // a row of a regrouped matrix is as long as the file's row and starts a group
    if (y && orc_dequant(device_type(name), tensor_device(name) + row * rb, (int64_t)cols, (float*)y, nullptr) == 0)
        orc_memcpy_d2h(out, y, cols * 4, nullptr);
}

bool GGUFParser::gemm_dev(const std::string& name, const TensorInfo& ti, float* out, const float* x, int n_tok,
                          int j0, int j1, int n_in) const {
    const int t = (int)ti.type;
    if (t != ORC_Q4_0 && t != ORC_Q8_0 && t != ORC_Q4_K && t != ORC_Q6_K) return false;  // reference: false too
    const int n_out = j1 - j0;
    if (n_out <= 0) return true;
    if (n_tok <= 0 || n_in <= 0 || ti.shape.empty() || (uint64_t)n_in != ti.shape[0] || j0 < 0 ||
        (ti.shape.size() > 1 && (uint64_t)j1 > ti.shape[1]))
        return false;
    const int64_t rb = orc_row_bytes(t, n_in);  // a regrouped row has the same length
    const size_t xb = ((size_t)n_tok * n_in * 4 + 255) & ~size_t(255), yb = (size_t)n_tok * n_out * 4;
    std::lock_guard<std::mutex> lk(scr_mu_);
    uint8_t* s = (uint8_t*)scratch(xb + yb);
    if (!s) return false;
    float *dx = (float*)s, *dy = (float*)(s + xb);
    if (orc_memcpy_h2d(dx, x, (size_t)n_tok * n_in * 4, nullptr)) return false;
    if (orc_gemm(device_type(name), tensor_device(name) + (size_t)j0 * rb, n_tok, n_out, n_in, dx, n_in, dy, n_out,
                 nullptr))
        return false;
    // gemv_q_range writes out[j0..j1); gemm_q (j0 = 0) writes out[t * n_out + j]
    return orc_memcpy_d2h(out + j0, dy, yb, nullptr) == 0;
}

bool GGUFParser::gemv_q(const std::string& name, float* out, const float* x, int n_out, int n_in) const {
    return gemv_q_range(name, out, x, 0, n_out, n_in);
}

bool GGUFParser::gemv_q_range(const std::string& name, float* out, const float* x, int j0, int j1, int n_in) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) return false;
    return gemm_dev(name, it->second, out, x, 1, j0, j1, n_in);
}

bool GGUFParser::gemm_q(const std::string& name, float* out, const float* x, int n_tokens, int n_out,
                        int n_in) const {
    auto it = tensors_.find(name);
    if (it == tensors_.end()) return false;
    return gemm_dev(name, it->second, out, x, n_tokens, 0, n_out, n_in);
}

// ── static test hooks: one-shot device buffers (test code, not a hot path) ───
void GGUFParser::dq_hook(int type, const uint8_t* s, uint64_t n, float* out) {
    if (!s || !out || !n || orc_init(0) != 0) return;
    const int64_t in_bytes = orc_row_bytes(type, (int64_t)n);
    if (in_bytes <= 0) return;
    void *d_in = nullptr, *d_out = nullptr;
    if (orc_malloc(&d_in, (size_t)in_bytes) == 0 && orc_malloc(&d_out, n * 4) == 0 &&
        orc_memcpy_h2d(d_in, s, (size_t)in_bytes, nullptr) == 0 &&
        orc_dequant(type, d_in, (int64_t)n, (float*)d_out, nullptr) == 0)
        orc_memcpy_d2h(out, d_out, n * 4, nullptr);
    orc_free(d_in);
    orc_free(d_out);
}

float GGUFParser::dot_hook(int type, const uint8_t* row, int n_cols, const float* x) {
    if (!row || !x || n_cols <= 0 || orc_init(0) != 0) return 0.f;
    const int64_t rb = orc_row_bytes(type, n_cols);
    if (rb <= 0) return 0.f;
    void *d_w = nullptr, *d_x = nullptr, *d_y = nullptr;
    float y = 0.f;
    if (orc_malloc(&d_w, (size_t)rb) == 0 && orc_malloc(&d_x, (size_t)n_cols * 4) == 0 && orc_malloc(&d_y, 4) == 0 &&
        orc_memcpy_h2d(d_w, row, (size_t)rb, nullptr) == 0 &&
        orc_memcpy_h2d(d_x, x, (size_t)n_cols * 4, nullptr) == 0 &&
        orc_gemm(type, d_w, 1, 1, n_cols, (const float*)d_x, n_cols, (float*)d_y, 1, nullptr) == 0)
        orc_memcpy_d2h(&y, d_y, 4, nullptr);
    orc_free(d_w);
    orc_free(d_x);
    orc_free(d_y);
    return y;
}

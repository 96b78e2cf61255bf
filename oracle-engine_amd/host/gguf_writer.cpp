#include "gguf_writer.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>

namespace orc {

static inline int clampi(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }
static inline int rnd(float v) { return (int)std::nearbyint(v); }

uint64_t row_bytes(GGMLType t, int64_t n) {
    uint32_t be, bb;
    if (!ggml_block_geom(t, be, bb) || n % be) return 0;
    return (uint64_t)(n / be) * bb;
}

// Q8_0: per 32 values one fp16 scale d = max|x|/127 and 32 int8 codes.
void quantize_q8_0(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* v = x + b * 32;
        uint8_t* blk = out + b * 34;
        float amax = 0.f;
        for (int i = 0; i < 32; ++i) amax = std::max(amax, std::fabs(v[i]));
        uint16_t dh = float_to_half(amax / 127.f);
        float d = half_to_float(dh);
        std::memcpy(blk, &dh, 2);
        for (int i = 0; i < 32; ++i)
            blk[2 + i] = (uint8_t)(int8_t)(d > 0.f ? clampi(rnd(v[i] / d), -127, 127) : 0);
    }
}

// Q4_0: per 32 values one fp16 scale; codes 0..15 with an implicit -8 offset.
// Low nibbles hold elements 0..15, high nibbles elements 16..31.
void quantize_q4_0(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 32; ++b) {
        const float* v = x + b * 32;
        uint8_t* blk = out + b * 18;
        float vmax = 0.f;
        for (int i = 0; i < 32; ++i)
            if (std::fabs(v[i]) > std::fabs(vmax)) vmax = v[i];
        uint16_t dh = float_to_half(vmax / -8.f);
        float d = half_to_float(dh);
        std::memcpy(blk, &dh, 2);
        int q[32];
        for (int i = 0; i < 32; ++i) q[i] = d != 0.f ? clampi(rnd(v[i] / d) + 8, 0, 15) : 8;
        for (int l = 0; l < 16; ++l) blk[2 + l] = (uint8_t)(q[l] | (q[l + 16] << 4));
    }
}

// Q4_K: 256-value superblock = fp16 d, fp16 dmin, 12 bytes of packed 6-bit
// (scale, min) pairs for 8 sub-blocks of 32, then 128 bytes of nibbles.
// Value = d*sc*q - dmin*m. Chunk j (64 values) stores values 64j+l in the low
// nibble and 64j+32+l in the high nibble of byte 32j+l.
void quantize_q4_k(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 256; ++b) {
        const float* v = x + b * 256;
        uint8_t* blk = out + b * 144;
        float scale[8], minv[8];
        for (int s = 0; s < 8; ++s) {
            float mn = 0.f, mx = -INFINITY;
            for (int i = 0; i < 32; ++i) { mn = std::min(mn, v[32 * s + i]); mx = std::max(mx, v[32 * s + i]); }
            if (mx < mn) mx = mn;
            scale[s] = (mx - mn) / 15.f;
            minv[s] = -mn;
        }
        float smax = 0.f, mmax = 0.f;
        for (int s = 0; s < 8; ++s) { smax = std::max(smax, scale[s]); mmax = std::max(mmax, minv[s]); }
        uint16_t dh = float_to_half(smax / 63.f), mh = float_to_half(mmax / 63.f);
        float d = half_to_float(dh), dmin = half_to_float(mh);
        int sc[8], mq[8];
        for (int s = 0; s < 8; ++s) {
            sc[s] = d > 0.f ? clampi(rnd(scale[s] / d), 0, 63) : 0;
            mq[s] = dmin > 0.f ? clampi(rnd(minv[s] / dmin), 0, 63) : 0;
        }
        std::memcpy(blk, &dh, 2);
        std::memcpy(blk + 2, &mh, 2);
        uint8_t* sp = blk + 4;
        for (int j = 0; j < 4; ++j) {
            sp[j] = (uint8_t)((sc[j] & 63) | ((sc[j + 4] >> 4) << 6));
            sp[j + 4] = (uint8_t)((mq[j] & 63) | ((mq[j + 4] >> 4) << 6));
            sp[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mq[j + 4] & 15) << 4));
        }
        int q[256];
        for (int s = 0; s < 8; ++s) {
            float d1 = d * (float)sc[s], m1 = dmin * (float)mq[s];
            for (int i = 0; i < 32; ++i)
                q[32 * s + i] = d1 > 0.f ? clampi(rnd((v[32 * s + i] + m1) / d1), 0, 15) : 0;
        }
        uint8_t* qs = blk + 16;
        for (int j = 0; j < 4; ++j)
            for (int l = 0; l < 32; ++l)
                qs[32 * j + l] = (uint8_t)(q[64 * j + l] | (q[64 * j + 32 + l] << 4));
    }
}

// Q6_K: 256-value superblock = ql[128] (low 4 bits), qh[64] (high 2 bits),
// int8 scales[16] (one per 16 consecutive values), fp16 d. Value =
// d*sc[e/16]*(q-32). For half h and l<32 the four values 128h+l+32g (g=0..3)
// share ql[64h+l], ql[64h+l+32] and qh[32h+l].
void quantize_q6_k(const float* x, int64_t n, uint8_t* out) {
    for (int64_t b = 0; b < n / 256; ++b) {
        const float* v = x + b * 256;
        uint8_t* blk = out + b * 210;
        float scale[16], smax = 0.f;
        for (int s = 0; s < 16; ++s) {
            float amax = 0.f;
            for (int i = 0; i < 16; ++i) amax = std::max(amax, std::fabs(v[16 * s + i]));
            scale[s] = amax / 31.f;
            smax = std::max(smax, scale[s]);
        }
        uint16_t dh = float_to_half(smax / 127.f);
        float d = half_to_float(dh);
        int8_t sc[16];
        int q[256];
        for (int s = 0; s < 16; ++s) {
            sc[s] = (int8_t)(d > 0.f ? clampi(rnd(scale[s] / d), -128, 127) : 0);
            float step = d * (float)sc[s];
            for (int i = 0; i < 16; ++i)
                q[16 * s + i] = step > 0.f ? clampi(rnd(v[16 * s + i] / step), -32, 31) + 32 : 32;
        }
        uint8_t* ql = blk;
        uint8_t* qh = blk + 128;
        for (int h = 0; h < 2; ++h)
            for (int l = 0; l < 32; ++l) {
                int q1 = q[128 * h + l], q2 = q[128 * h + l + 32];
                int q3 = q[128 * h + l + 64], q4 = q[128 * h + l + 96];
                ql[64 * h + l] = (uint8_t)((q1 & 15) | ((q3 & 15) << 4));
                ql[64 * h + l + 32] = (uint8_t)((q2 & 15) | ((q4 & 15) << 4));
                qh[32 * h + l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
            }
        std::memcpy(blk + 192, sc, 16);
        std::memcpy(blk + 208, &dh, 2);
    }
}

bool quantize_any(GGMLType t, const float* x, int64_t n, uint8_t* out) {
    switch (t) {
        case GGMLType::F32: std::memcpy(out, x, (size_t)n * 4); return true;
        case GGMLType::F16:
            for (int64_t i = 0; i < n; ++i) {
                uint16_t h = float_to_half(x[i]);
                std::memcpy(out + 2 * i, &h, 2);
            }
            return true;
        case GGMLType::BF16:  // round to nearest even (finite inputs)
            for (int64_t i = 0; i < n; ++i) {
                uint32_t u;
                std::memcpy(&u, &x[i], 4);
                u += 0x7FFFu + ((u >> 16) & 1u);
                const uint16_t h = (uint16_t)(u >> 16);
                std::memcpy(out + 2 * i, &h, 2);
            }
            return true;
        case GGMLType::Q8_0: quantize_q8_0(x, n, out); return true;
        case GGMLType::Q4_0: quantize_q4_0(x, n, out); return true;
        case GGMLType::Q4_K: quantize_q4_k(x, n, out); return true;
        case GGMLType::Q6_K: quantize_q6_k(x, n, out); return true;
        default: return false;
    }
}

void GGUFWriter::add_str(const std::string& k, const std::string& v) {
    KV kv; kv.key = k; kv.kind = 8; kv.s = v; kvs.push_back(kv);
}
void GGUFWriter::add_u32(const std::string& k, uint32_t v) {
    KV kv; kv.key = k; kv.kind = 4; kv.u = v; kvs.push_back(kv);
}
void GGUFWriter::add_f32(const std::string& k, float v) {
    KV kv; kv.key = k; kv.kind = 6; kv.f = v; kvs.push_back(kv);
}
void GGUFWriter::add_str_array(const std::string& k, const std::vector<std::string>& v) {
    KV kv; kv.key = k; kv.kind = 9; kv.arr = v; kvs.push_back(kv);
}
void GGUFWriter::add_i32_array(const std::string& k, const std::vector<int32_t>& v) {
    KV kv; kv.key = k; kv.kind = 9; kv.ai = v; kvs.push_back(kv);
}
void GGUFWriter::add_tensor(const std::string& name, std::vector<uint64_t> shape, GGMLType type,
                            std::function<void(int64_t, int64_t, uint8_t*)> fill) {
    Tensor t;
    t.name = name;
    t.shape = std::move(shape);
    t.type = type;
    t.fill = std::move(fill);
    uint64_t rows = 1;
    for (size_t i = 1; i < t.shape.size(); ++i) rows *= t.shape[i];
    t.nbytes = row_bytes(type, (int64_t)t.shape[0]) * rows;
    tensors.push_back(std::move(t));
}

namespace {
struct Out {
    FILE* f;
    uint64_t pos = 0;
    bool ok = true;
    void raw(const void* p, size_t n) {
        if (ok && n && std::fwrite(p, 1, n, f) != n) ok = false;
        pos += n;
    }
    void u32(uint32_t v) { raw(&v, 4); }
    void u64(uint64_t v) { raw(&v, 8); }
    void str(const std::string& s) { u64(s.size()); raw(s.data(), s.size()); }
    void pad_to(uint64_t align) {
        static const uint8_t z[64] = {0};
        uint64_t want = (pos + align - 1) / align * align;
        while (pos < want) raw(z, (size_t)std::min<uint64_t>(64, want - pos));
    }
};
}  // namespace

bool GGUFWriter::write(const std::string& path, bool verbose) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) return false;
    std::vector<char> buf(1 << 22);
    std::setvbuf(f, buf.data(), _IOFBF, buf.size());
    const uint64_t al = alignment ? alignment : 32;
    std::vector<KV> all = kvs;
    if (al != 32) {
        KV kv;
        kv.key = "general.alignment";
        kv.kind = 4;
        kv.u = al;
        all.push_back(kv);
    }
    Out o{f};
    o.raw("GGUF", 4);
    o.u32(3);
    o.u64(tensors.size());
    o.u64(all.size());
    for (const KV& kv : all) {
        o.str(kv.key);
        o.u32(kv.kind);
        switch (kv.kind) {
            case 8: o.str(kv.s); break;
            case 4: o.u32((uint32_t)kv.u); break;
            case 6: o.raw(&kv.f, 4); break;
            case 9:
                if (kv.arr.empty() && !kv.ai.empty()) {
                    o.u32(5);
                    o.u64(kv.ai.size());
                    o.raw(kv.ai.data(), kv.ai.size() * 4);
                } else {
                    o.u32(8);
                    o.u64(kv.arr.size());
                    for (const auto& s : kv.arr) o.str(s);
                }
                break;
        }
    }
    uint64_t off = 0;
    for (Tensor& t : tensors) {
        t.offset = off;
        off = (off + t.nbytes + al - 1) / al * al;
    }
    for (const Tensor& t : tensors) {
        o.str(t.name);
        o.u32((uint32_t)t.shape.size());
        for (uint64_t d : t.shape) o.u64(d);
        o.u32((uint32_t)t.type);
        o.u64(t.offset);
    }
    o.pad_to(al);
    const uint64_t data_start = o.pos;
    std::vector<uint8_t> chunk;
    for (const Tensor& t : tensors) {
        while (o.pos < data_start + t.offset) { uint8_t z = 0; o.raw(&z, 1); }
        uint64_t rows = t.shape.size() > 1 ? t.nbytes / row_bytes(t.type, (int64_t)t.shape[0]) : 1;
        uint64_t rb = t.nbytes / rows;
        const int64_t step = std::max<int64_t>(1, (int64_t)((64ull << 20) / std::max<uint64_t>(rb, 1)));
        for (int64_t r0 = 0; r0 < (int64_t)rows; r0 += step) {
            int64_t r1 = std::min<int64_t>((int64_t)rows, r0 + step);
            chunk.resize((size_t)((r1 - r0) * rb));
            t.fill(r0, r1, chunk.data());
            o.raw(chunk.data(), chunk.size());
        }
        if (verbose) std::fprintf(stderr, "  %-28s %-5s %10.2f MB\n", t.name.c_str(), ggml_type_name(t.type), t.nbytes / 1e6);
    }
    o.pad_to(32);
    bool ok = o.ok;
    if (std::fclose(f) != 0) ok = false;
    return ok;
}

}  // namespace orc

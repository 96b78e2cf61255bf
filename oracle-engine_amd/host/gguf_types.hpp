// GGUF on-disk tensor types and GGML block geometry shared by the reader, the
// writer and the device upload path.
//
// The enum values are the GGUF/GGML on-disk type ids; they must stay equal to
// the reference's `GGMLType` (core/gguf_parser.hpp:9-24) so the same file means
// the same thing to both implementations. Block sizes follow
// `TensorInfo::n_bytes` (core/gguf_parser.cpp:61-75).
#pragma once
#include <cstdint>
#include <cstring>

enum class GGMLType : uint32_t {
    F32 = 0,
    F16 = 1,
    Q4_0 = 2,
    Q4_1 = 3,
    Q5_0 = 6,
    Q5_1 = 7,
    Q8_0 = 8,
    Q8_1 = 9,
    Q4_K = 12,
    Q5_K = 13,
    Q6_K = 14,
    Q8_K = 15,
    BF16 = 30,
    UNKNOWN = 0xFFFFFFFF,
};

// Elements per block and bytes per block for every type this engine decodes.
// Returns false for types the hot path does not support (the reference rejects
// them at load time, core/gguf_parser.cpp:96-110).
inline bool ggml_block_geom(GGMLType t, uint32_t& blk_elems, uint32_t& blk_bytes) {
    switch (t) {
        case GGMLType::F32:  blk_elems = 1;   blk_bytes = 4;   return true;
        case GGMLType::F16:
        case GGMLType::BF16: blk_elems = 1;   blk_bytes = 2;   return true;
        case GGMLType::Q4_0: blk_elems = 32;  blk_bytes = 18;  return true;
        case GGMLType::Q8_0: blk_elems = 32;  blk_bytes = 34;  return true;
        case GGMLType::Q4_K: blk_elems = 256; blk_bytes = 144; return true;
        case GGMLType::Q6_K: blk_elems = 256; blk_bytes = 210; return true;
        default: blk_elems = 0; blk_bytes = 0; return false;
    }
}

inline const char* ggml_type_name(GGMLType t) {
    switch (t) {
        case GGMLType::F32: return "F32";
        case GGMLType::F16: return "F16";
        case GGMLType::BF16: return "BF16";
        case GGMLType::Q4_0: return "Q4_0";
        case GGMLType::Q8_0: return "Q8_0";
        case GGMLType::Q4_K: return "Q4_K";
        case GGMLType::Q6_K: return "Q6_K";
        default: return "?";
    }
}

// IEEE binary16 -> binary32, exact for every input (subnormals, inf, NaN).
inline float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t e = (h >> 10) & 0x1F, m = h & 0x3FF, f;
    if (e == 0) {
        if (m == 0) {
            f = sign;
        } else {
            int sh = 0;
            while (!(m & 0x400)) { m <<= 1; ++sh; }
            f = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3FF) << 13);
        }
    } else if (e == 31) {
        f = sign | 0x7F800000u | (m << 13);
    } else {
        f = sign | ((e + 112) << 23) | (m << 13);
    }
    float r;
    std::memcpy(&r, &f, 4);
    return r;
}

// IEEE binary32 -> binary16, round to nearest even (overflow -> inf).
inline uint16_t float_to_half(float v) {
    uint32_t x;
    std::memcpy(&x, &v, 4);
    uint32_t sign = (x >> 16) & 0x8000;
    uint32_t ax = x & 0x7FFFFFFF;
    if (ax >= 0x7F800000) return (uint16_t)(sign | 0x7C00 | (ax > 0x7F800000 ? 0x200 : 0));
    if (ax >= 0x477FF000) return (uint16_t)(sign | 0x7C00);  // rounds past 65504
    if (ax < 0x38800000) {                                   // result is subnormal or zero
        if (ax < 0x33000000) return (uint16_t)sign;           // below half of the smallest subnormal
        uint32_t m = (ax & 0x7FFFFF) | 0x800000;
        int shift = 126 - (int)(ax >> 23);                    // 14..24
        uint32_t q = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = ((ax >> 13) - (112u << 10));
    uint32_t rem = ax & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (q & 1))) ++q;
    return (uint16_t)(sign | q);
}

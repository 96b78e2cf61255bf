// Bit-exact dequant codecs and the embedding-row gather (gfx950).
//
// Replaces the block codecs and dequantize_row / dequantize_into of the
// reference (core/gguf_parser.cpp:420-482, 1002-1154) and the embedding
// lookups of Model::forward / forward_prefill (core/model.cpp:349-358, 549-558).
#include "orc_internal.hpp"

// ── bit-exact dequant (core/gguf_parser.cpp:1029-1154) ───────────────────────
namespace orc {
// One thread per 32 consecutive output values; rounding exactly as the
// reference build: Q4_0/Q8_0/F16/BF16 one product or exact conversion, Q4_K
// fma(d*sc, q, -(dmin*m)) (the reference's d1*q - m1f contracts to one FMA),
// Q6_K (d*sc)*q with two roundings.
__device__ __forceinline__ void dequant32(int type, const uint8_t* w, int64_t g, float* out) {
    switch (type) {
        case ORC_F32:
            for (int i = 0; i < 32; ++i) out[i] = ((const float*)w)[g * 32 + i];
            break;
        case ORC_F16:
            for (int i = 0; i < 32; ++i) out[i] = h2f(ld2(w + (g * 32 + i) * 2));
            break;
        case ORC_BF16:  // the high half of an fp32 (core/gguf_parser.cpp:1034-1040)
            for (int i = 0; i < 32; ++i) out[i] = __builtin_bit_cast(float, ld2(w + (g * 32 + i) * 2) << 16);
            break;
        case ORC_Q8_0: {
            const uint8_t* b = w + g * 34;
            const float d = h2f(ld2(b));
            for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)b[2 + i];
            break;
        }
        case ORC_Q8_0_X8: {  // block g&7 of the 272-byte group g>>3: scale at 2*(g&7), codes at 16+32*(g&7)
            const uint8_t* grp = w + (g >> 3) * 272;
            const float d = h2f(ld2(grp + 2 * (g & 7)));
            const uint8_t* q = grp + 16 + 32 * (g & 7);
            for (int i = 0; i < 32; ++i) out[i] = d * (float)(int8_t)q[i];
            break;
        }
        case ORC_Q4_0: {
            const uint8_t* b = w + g * 18;
            const float d = h2f(ld2(b));
            for (int l = 0; l < 16; ++l) {
                out[l] = d * (float)((int)(b[2 + l] & 0xF) - 8);
                out[l + 16] = d * (float)((int)(b[2 + l] >> 4) - 8);
            }
            break;
        }
        case ORC_Q4_K: {  // 32 values = one sub-block
            const int64_t sb = g >> 3;
            const int s = (int)(g & 7), j = s >> 1, hi = s & 1;
            const uint8_t* b = w + sb * 144;
            const float d = h2f(ld2(b)), dmin = h2f(ld2(b + 2));
            uint32_t sc, mn;
            q4k_scale_min(s, ld4(b + 4), ld4(b + 8), ld4(b + 12), sc, mn);
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            const uint8_t* qs = b + 16 + 32 * j;
            for (int l = 0; l < 32; ++l) {
                const uint32_t q = hi ? (qs[l] >> 4) : (qs[l] & 0xF);
                out[l] = __builtin_fmaf(d1, (float)q, -m1);
            }
            break;
        }
        case ORC_Q6_K: {  // 32 values = values 128hh+32gg+[0,32) of superblock sb
            const int64_t sb = g >> 3;
            const int s = (int)(g & 7), hh = s >> 2, gg = s & 3;
            const uint8_t* b = w + sb * 210;
            const uint8_t* ql = b + 64 * hh;
            const uint8_t* qh = b + 128 + 32 * hh;
            const int8_t* sc = (const int8_t*)(b + 192 + 8 * hh);
            const float d = h2f(ld2(b + 208));
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                int q;
                if (gg == 0) q = (ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4);
                else if (gg == 1) q = (ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4);
                else if (gg == 2) q = (ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4);
                else q = (ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4);
                out[l] = (d * (float)sc[is + 2 * gg]) * (float)(q - 32);
            }
            break;
        }
    }
}

__global__ void k_dequant(int type, const uint8_t* w, int64_t n_groups, float* y) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    float v[32];
    dequant32(type, w, g, v);
    float4* o = (float4*)(y + g * 32);
    for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

__global__ void k_embed(int type, const uint8_t* table, int n_in, int n_rows, uint64_t row_bytes, const int32_t* ids,
                        float* y, int ldy) {
    const int t = blockIdx.y;
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g * 32 >= n_in) return;
    int id = ids[t];
    if (id < 0 || id >= n_rows) id = 0;
    float v[32];
    dequant32(type, table + (uint64_t)id * row_bytes, g, v);
    float4* o = (float4*)(y + (size_t)t * ldy + g * 32);
    for (int i = 0; i < 8; ++i) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}
}  // namespace orc

using namespace orc;

static bool dq_type_ok(int t) {
    return t == ORC_F32 || t == ORC_F16 || t == ORC_BF16 || t == ORC_Q4_0 || t == ORC_Q8_0 || t == ORC_Q4_K ||
           t == ORC_Q6_K;
}

extern "C" int orc_dequant(int type, const void* d_w, int64_t n_el, float* d_y, orc_stream_t stream) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!dq_type_ok(type) && type != ORC_Q8_0_X8)
        return set_error(ORC_E_UNSUPPORTED, "dequant: unsupported type " + std::to_string(type));
    const int be = (type == ORC_Q4_K || type == ORC_Q6_K || type == ORC_Q8_0_X8) ? 256 : 32;
    if (n_el <= 0 || n_el % be || !d_w || !d_y) return set_error(ORC_E_INVALID, "dequant: bad size or pointer");
    if ((uintptr_t)d_y & 15) return set_error(ORC_E_INVALID, "dequant: output must be 16-byte aligned");
    const int64_t groups = n_el / 32;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, resolve_stream(stream), type,
                       (const uint8_t*)d_w, groups, d_y);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_embed(int type, const void* d_table, int n_in, int n_rows, const int32_t* d_ids, int n_tok,
                         float* d_y, int ldy, orc_stream_t stream) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!dq_type_ok(type)) return set_error(ORC_E_UNSUPPORTED, "embed: unsupported type " + std::to_string(type));
    const int be = (type == ORC_Q4_K || type == ORC_Q6_K) ? 256 : 32;
    if (n_in <= 0 || n_in % be || n_rows <= 0 || n_tok < 0 || ldy < n_in || ldy % 4 || !d_table || !d_ids || !d_y)
        return set_error(ORC_E_INVALID, "embed: bad arguments");
    if (n_tok == 0) return ORC_OK;
    const int groups = n_in / 32;
    hipLaunchKernelGGL(k_embed, dim3((groups + 63) / 64, n_tok), dim3(64), 0, resolve_stream(stream), type,
                       (const uint8_t*)d_table, n_in, n_rows, (uint64_t)orc_row_bytes(type, n_in), d_ids, d_y, ldy);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

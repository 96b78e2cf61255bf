// Quantized GEMV / GEMM on raw GGML blocks (gfx950).
//
// Replaces gemv_q / gemv_q_range / gemm_q (core/gguf_parser.cpp:496-997) and
// the projection sequences of Model::forward / forward_prefill that surround
// them (RMSNorm, QKV bias, residual add, SwiGLU; core/model.cpp:366-473,
// 565-643).
//
// Two kernel families. Q4_K and Q6_K matrices (a Q4_K_M target's) run on the
// matrix cores (k_mmq, orc_mmq.hip); Q8_0 and Q4_0 on the vector ALUs (k_qmv,
// below). Either way one matrix always uses one family and one reduction
// order, so n-token results equal n decode results bit for bit.
//
// k_qmv design (n_tok = 1 is the decode GEMV):
//  * Persistent 512-thread workgroups (one or two per CU). A workgroup stages
//    the activations of all n_tok tokens in LDS once (fp32, 4 floats of
//    padding every 32/64 values so the lanes of a slot hit distinct banks,
//    plus per-16-value sums for the Q4_K minimum and the code offsets), then
//    its waves walk row groups spread over every CU.
//  * A wave holds G = 64/LPR slots of ROWS rows. A slot's LPR lanes split the
//    row into units (a 16-byte Q4_K nibble chunk = 32 values, a 64-value
//    quarter of a Q6_K superblock, one Q8_0 / Q4_0 block); lane li owns units
//    li, li+LPR, ... and walks them in batches of UPL whose loads are all in
//    flight at once, straight from the as-uploaded GGUF bytes with 128-bit
//    loads. The first batch of a wave's first row group is issued before the
//    activations are staged.
//  * Each weight code is converted once and applied to every token, 8 codes
//    at a time against 8 activations read from LDS; fp32 FMA chains.
//  * RMSNorm prologue: x is staged multiplied by the norm weight and the
//    per-token 1/rms (reduced while staging) scales the finished dot product:
//    sum_i w_i (x_i s g_i) = s * sum_i w_i (x_i g_i).
//  * Batch invariance: LPR depends on the type only; a lane's partial sum
//    runs over its units in a fixed order, the slot reduction is a fixed xor
//    butterfly and the RMS sum uses a fixed thread mapping, so a (token, row)
//    result is bit-identical for every n_tok and every launch shape: the
//    (k+1)-token verify pass equals k+1 decode GEMVs.
#include "orc_gemm.hpp"

#include <algorithm>
#include <type_traits>
#include <vector>

namespace orc {

// LPR: lanes per row slot; EPU: values per unit; PP: LDS padding period.
template <int QT> struct QTr;
template <> struct QTr<ORC_Q8_0> { static constexpr int EPU = 32, PP = 32, LPR = 32; };
template <> struct QTr<ORC_Q8_0_X8> { static constexpr int EPU = 32, PP = 32, LPR = 32; };
template <> struct QTr<ORC_Q4_0> { static constexpr int EPU = 32, PP = 32, LPR = 32; };
template <> struct QTr<ORC_Q4_K> { static constexpr int EPU = 32, PP = 64, LPR = 32; };
template <> struct QTr<ORC_Q6_K> { static constexpr int EPU = 64, PP = 64, LPR = 16; };
// dense rows (F32 / F16 / BF16): a unit is 32 consecutive values
template <> struct QTr<ORC_F32> { static constexpr int EPU = 32, PP = 32, LPR = 32; };
template <> struct QTr<ORC_F16> { static constexpr int EPU = 32, PP = 32, LPR = 32; };
template <> struct QTr<ORC_BF16> { static constexpr int EPU = 32, PP = 32, LPR = 32; };
// one-token mixed launches (Q4_K segments, then Q6_K segments): each row
// group takes its own type's unit, LPR and row count; both pad every 64 values
template <> struct QTr<kMixK> { static constexpr int EPU = 32, PP = 64, LPR = 32; };

template <int PP> __device__ __forceinline__ int padx(int k) { return k + 4 * (k / PP); }

// Segment pointers held in scalar registers: readfirstlane keeps the
// compiler from turning a lane-dependent choice between them back into a
// vector load from the parameter block (and a wait on it).
template <class T> __device__ __forceinline__ T* spin(T* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T*)(((uint64_t)hi << 32) | lo);
}

struct XCtx {
    const float* xs;  // staged x (times the norm weight), token 0, element 0, padded
    int xs_stride;    // floats between tokens
    const float* sx;  // per-16 sums of the staged x, token 0
    int sx_stride;
    int k0;           // first element staged
};

// Bytes of two dwords as 8 floats: byte k of a -> w[k], of b -> w[4+k].
// v unchanged, but opaque to the optimiser: a nibble word masked with
// 0x0F0F0F0F then converted byte by byte stays one AND per word and one
// v_cvt_f32_ubyteN per value, instead of the mask folded into a v_bfe_u32
// per value in front of a v_cvt_f32_ubyte0 (twice the conversion work).
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm("" : "+v"(v));
    return v;
}

__device__ __forceinline__ void to_f8(uint32_t a, uint32_t b, float* w) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        w[k] = ubyte_f(a, k);
        w[4 + k] = ubyte_f(b, k);
    }
}

// S[r][t] += sum_{i<8} w[r][i] * x_t[e+i] (sequential FMA chain), x from LDS
// at padded offset pe. The 8 activations of a token are read once for all rows.
template <int ROWS, int NT>
__device__ __forceinline__ void dot8(const float (&w)[ROWS][8], const XCtx& c, int pe, float (&S)[ROWS][NT]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const float4 a = *(const float4*)(c.xs + t * c.xs_stride + pe);
        const float4 b = *(const float4*)(c.xs + t * c.xs_stride + pe + 4);
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            float s = S[r][t];
            s = __builtin_fmaf(w[r][0], a.x, s);
            s = __builtin_fmaf(w[r][1], a.y, s);
            s = __builtin_fmaf(w[r][2], a.z, s);
            s = __builtin_fmaf(w[r][3], a.w, s);
            s = __builtin_fmaf(w[r][4], b.x, s);
            s = __builtin_fmaf(w[r][5], b.y, s);
            s = __builtin_fmaf(w[r][6], b.z, s);
            s = __builtin_fmaf(w[r][7], b.w, s);
            S[r][t] = s;
        }
    }
}

template <int ROWS, int NT> __device__ __forceinline__ void zero(float (&S)[ROWS][NT]) {
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) S[r][t] = 0.f;
}

// ── per-type units: load() issues the loads, compute() does the arithmetic ───
template <int QT, int ROWS> struct Unit;

template <int ROWS> struct Unit<ORC_Q4_K, ROWS> {
    // unit u: superblock u/8, 16-byte nibble chunk c = u%8 of it. Chunk c
    // holds values 64j+16h+[0,16) (low nibbles, sub-block 2j) and
    // 64j+32+16h+[0,16) (high nibbles, sub-block 2j+1), j = c/2, h = c%2.
    // Per sub-block: d*sc * sum(q x) - dmin*m * sum(x)  (core/gguf_parser.cpp:1096-1121).
    u32x4 hdr[ROWS], q[ROWS];
    __device__ __forceinline__ void load(const uint8_t* const (&rp)[ROWS], int u) {
        const int b = u >> 3, ch = u & 7;
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint8_t* blk = rp[r] + (size_t)b * 144;
            hdr[r] = ld16(blk);
            q[r] = ld16(blk + 16 + 16 * ch);
        }
    }
    // the nibbles of the chunk words at bit sh (0: low, 4: high), masked right
    // before their conversion
    template <int NT>
    __device__ __forceinline__ void half(int sh, int e, const float (&dd)[ROWS], const float (&mm)[ROWS],
                                         const XCtx& c, float (&acc)[ROWS][NT]) const {
        float S[ROWS][NT];
        zero(S);
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            float w[ROWS][8];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const uint32_t a = k ? q[r].z : q[r].x, b = k ? q[r].w : q[r].y;
                to_f8(opaque((a >> sh) & 0x0F0F0F0Fu), opaque((b >> sh) & 0x0F0F0F0Fu), w[r]);
            }
            dot8(w, c, padx<64>(e + 8 * k), S);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float sxv = c.sx[t * c.sx_stride + e / 16];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                acc[r][t] = __builtin_fmaf(dd[r], S[r][t], acc[r][t]);
                acc[r][t] = __builtin_fmaf(-mm[r], sxv, acc[r][t]);
            }
        }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const XCtx& c, float (&acc)[ROWS][NT]) const {
        const int b = u >> 3, ch = u & 7, j = ch >> 1, h = ch & 1;
        const int eA = b * 256 + 64 * j + 16 * h - c.k0;
        float dA[ROWS], mA[ROWS], dB[ROWS], mB[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const float d = h2f(hdr[r].x & 0xFFFFu), dmin = h2f(hdr[r].x >> 16);
            uint32_t s0, m0, s1, m1;
            q4k_scale_min(2 * j, hdr[r].y, hdr[r].z, hdr[r].w, s0, m0);
            q4k_scale_min(2 * j + 1, hdr[r].y, hdr[r].z, hdr[r].w, s1, m1);
            dA[r] = d * (float)s0;
            mA[r] = dmin * (float)m0;
            dB[r] = d * (float)s1;
            mB[r] = dmin * (float)m1;
        }
        half<NT>(0, eA, dA, mA, c, acc);
        half<NT>(4, eA + 32, dB, mB, c, acc);
    }
};

template <int ROWS> struct Unit<ORC_Q6_K, ROWS> {
    // unit u: superblock u/4, quarter v = u%4: half hh = v/2, l0 = 16*(v%2).
    // Group g (0..3) holds values 128hh+32g+l0+[0,16) with scale sc[8hh+2g+v%2];
    // codes are stored +32 (core/gguf_parser.cpp:1124-1154).
    u32x4 qa[ROWS], qb[ROWS], qh[ROWS];
    u32x2 sc[ROWS];
    uint32_t dh[ROWS];
    __device__ __forceinline__ void load(const uint8_t* const (&rp)[ROWS], int u) {
        const int b = u >> 2, v = u & 3, hh = v >> 1, l0 = 16 * (v & 1);
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint8_t* blk = rp[r] + (size_t)b * 210;
            qa[r] = ld16(blk + 64 * hh + l0);
            qb[r] = ld16(blk + 64 * hh + 32 + l0);
            qh[r] = ld16(blk + 128 + 32 * hh + l0);
            sc[r] = ld8(blk + 192 + 8 * hh);
            dh[r] = ld2(blk + 208);
        }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const XCtx& c, float (&acc)[ROWS][NT]) const {
        const int b = u >> 2, v = u & 3, hh = v >> 1, odd = v & 1, l0 = 16 * odd;
        const int e0 = b * 256 + 128 * hh + l0 - c.k0;
        float d[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) d[r] = h2f(dh[r]);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float sg[ROWS];
            uint32_t qq[ROWS][4];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const int si = 2 * g + odd;  // byte index inside the 8 scale bytes of this half
                const uint32_t sw = si < 4 ? sc[r].x : sc[r].y;
                sg[r] = d[r] * (float)(int8_t)((sw >> (8 * (si & 3))) & 0xFFu);
                const uint32_t a4[4] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w};
                const uint32_t b4[4] = {qb[r].x, qb[r].y, qb[r].z, qb[r].w};
                const uint32_t h4[4] = {qh[r].x, qh[r].y, qh[r].z, qh[r].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t nib, hb;
                    if (g == 0) { nib = a4[i] & 0x0F0F0F0Fu; hb = (h4[i] << 4) & 0x30303030u; }
                    else if (g == 1) { nib = b4[i] & 0x0F0F0F0Fu; hb = (h4[i] << 2) & 0x30303030u; }
                    else if (g == 2) { nib = (a4[i] >> 4) & 0x0F0F0F0Fu; hb = h4[i] & 0x30303030u; }
                    else { nib = (b4[i] >> 4) & 0x0F0F0F0Fu; hb = (h4[i] >> 2) & 0x30303030u; }
                    qq[r][i] = nib | hb;
                }
            }
            const int eg = e0 + 32 * g;
            float S[ROWS][NT];
            zero(S);
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                float w[ROWS][8];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) to_f8(qq[r][2 * k], qq[r][2 * k + 1], w[r]);
                dot8(w, c, padx<64>(eg + 8 * k), S);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float sxg = c.sx[t * c.sx_stride + eg / 16];
#pragma unroll
                for (int r = 0; r < ROWS; ++r)  // sum (q-32) x = sum q x - 32 sum x
                    acc[r][t] = __builtin_fmaf(sg[r], __builtin_fmaf(-32.f, sxg, S[r][t]), acc[r][t]);
            }
        }
    }
};

template <int ROWS> struct Unit<ORC_Q8_0, ROWS> {
    // unit u: block u (fp16 d + 32 int8 codes), acc += d * sum(q x)
    // (core/gguf_parser.cpp:1073-1082). Codes are converted as unsigned q+128
    // (one xor per 4 codes) and the offset removed with the block sum of x.
    u32x4 q0[ROWS], q1[ROWS];
    uint32_t dh[ROWS];
    __device__ __forceinline__ void load(const uint8_t* const (&rp)[ROWS], int u) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint8_t* blk = rp[r] + (size_t)u * 34;
            dh[r] = ld2(blk);
            q0[r] = ld16(blk + 2);
            q1[r] = ld16(blk + 18);
        }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const XCtx& c, float (&acc)[ROWS][NT]) const {
        const int e0 = u * 32 - c.k0;
        const int p0 = padx<32>(e0);
        float S[ROWS][NT];
        zero(S);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float w[ROWS][8];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const uint32_t qq[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
                to_f8(qq[2 * k] ^ 0x80808080u, qq[2 * k + 1] ^ 0x80808080u, w[r]);
            }
            dot8(w, c, p0 + 8 * k, S);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float sx32 = c.sx[t * c.sx_stride + e0 / 16] + c.sx[t * c.sx_stride + e0 / 16 + 1];
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
                acc[r][t] = __builtin_fmaf(h2f(dh[r]), __builtin_fmaf(-128.f, sx32, S[r][t]), acc[r][t]);
        }
    }
};

// ORC_Q8_0_X8: block u is code run u % 8 of the 272-byte group u / 8 (8
// fp16 scales, then 8 x 32 codes): the same values as Q8_0, loaded with
// aligned 16-byte reads; the arithmetic is Q8_0's.
// Loads through the global address space (not flat), so the x staging's LDS
// waits (lgkmcnt) never wait for them: this type's first batch is in flight
// during the staging.
template <int ROWS> struct Unit<ORC_Q8_0_X8, ROWS> : Unit<ORC_Q8_0, ROWS> {
    typedef const __attribute__((address_space(1))) u32x4* g16;
    typedef const __attribute__((address_space(1))) uint16_t* g2;
    __device__ __forceinline__ void load(const uint8_t* const (&rp)[ROWS], int u) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint8_t* grp = rp[r] + (size_t)(u >> 3) * 272;
            this->dh[r] = *(g2)(grp + 2 * (u & 7));
            const g16 q = (g16)(grp + 16 + 32 * (u & 7));
            this->q0[r] = q[0];
            this->q1[r] = q[1];
        }
    }
};

template <int ROWS> struct Unit<ORC_Q4_0, ROWS> {
    // unit u: block u (fp16 d + 16 bytes: low nibble -> value l, high -> l+16),
    // codes stored +8 (core/gguf_parser.cpp:1058-1070).
    u32x4 q[ROWS];
    uint32_t dh[ROWS];
    __device__ __forceinline__ void load(const uint8_t* const (&rp)[ROWS], int u) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint8_t* blk = rp[r] + (size_t)u * 18;
            dh[r] = ld2(blk);
            q[r] = ld16(blk + 2);
        }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const XCtx& c, float (&acc)[ROWS][NT]) const {
        const int e0 = u * 32 - c.k0;
        const int p0 = padx<32>(e0);
        float S[ROWS][NT];
        zero(S);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float w[ROWS][8];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                const uint32_t qq[4] = {q[r].x, q[r].y, q[r].z, q[r].w};
                const uint32_t a = qq[2 * (k & 1)], b = qq[2 * (k & 1) + 1];
                if (k < 2) to_f8(opaque(a & 0x0F0F0F0Fu), opaque(b & 0x0F0F0F0Fu), w[r]);
                else to_f8(opaque((a >> 4) & 0x0F0F0F0Fu), opaque((b >> 4) & 0x0F0F0F0Fu), w[r]);
            }
            dot8(w, c, p0 + 8 * k, S);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float sx32 = c.sx[t * c.sx_stride + e0 / 16] + c.sx[t * c.sx_stride + e0 / 16 + 1];
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
                acc[r][t] = __builtin_fmaf(h2f(dh[r]), __builtin_fmaf(-8.f, sx32, S[r][t]), acc[r][t]);
        }
    }
};

// Dense rows: F32, F16 or BF16 values widened exactly to fp32. The reference
// runs such matrices through its fallback, dequantize + ops::matmul
// (core/model.cpp:370-381 and the same pattern for o / gate / up / down /
// head; core/gguf_parser.cpp:1029-1055 for the conversions).
template <int QT, int ROWS> struct DenseUnit {
    static constexpr int WB = QT == ORC_F32 ? 4 : 2;  // bytes per value
    static constexpr int NV = 2 * WB;                 // 16-byte loads per 32-value unit
    u32x4 v[ROWS][NV];
    __device__ __forceinline__ void load(const uint8_t* const (&rp)[ROWS], int u) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const uint8_t* p = rp[r] + (size_t)u * 32 * WB;
#pragma unroll
            for (int i = 0; i < NV; ++i) v[r][i] = ld16(p + 16 * i);
        }
    }
    // values 8k .. 8k + 7 of the unit of row r
    __device__ __forceinline__ void vals8(int r, int k, float* w) const {
        if constexpr (QT == ORC_F32) {
            const u32x4 a = v[r][2 * k], b = v[r][2 * k + 1];
            const uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) w[i] = __builtin_bit_cast(float, q[i]);
        } else {
            const u32x4 a = v[r][k];
            const uint32_t q[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (QT == ORC_F16) {
                    w[2 * i] = h2f(q[i] & 0xFFFFu);
                    w[2 * i + 1] = h2f(q[i] >> 16);
                } else {  // BF16: the high half of an fp32
                    w[2 * i] = __builtin_bit_cast(float, q[i] << 16);
                    w[2 * i + 1] = __builtin_bit_cast(float, q[i] & 0xFFFF0000u);
                }
            }
        }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const XCtx& c, float (&acc)[ROWS][NT]) const {
        const int p0 = padx<32>(u * 32 - c.k0);
        float S[ROWS][NT];
        zero(S);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float w[ROWS][8];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) vals8(r, k, w[r]);
            dot8(w, c, p0 + 8 * k, S);
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[r][t] += S[r][t];
    }
};
template <int ROWS> struct Unit<ORC_F32, ROWS> : DenseUnit<ORC_F32, ROWS> {};
template <int ROWS> struct Unit<ORC_F16, ROWS> : DenseUnit<ORC_F16, ROWS> {};
template <int ROWS> struct Unit<ORC_BF16, ROWS> : DenseUnit<ORC_BF16, ROWS> {};

// kMixK instantiates the generic row-group loops, which its launches never
// run (the mixed loop below takes every group)
template <int ROWS> struct Unit<kMixK, ROWS> : Unit<ORC_Q4_K, ROWS> {};

// ── the kernel ───────────────────────────────────────────────────────────────

constexpr int kQWG = 512, kQWaves = kQWG / 64;
constexpr int kMaxNT = 5;  // tokens per launch; larger batches are chunked (results unchanged)

template <int ROWS> struct RowSet {
    const uint8_t* rp[ROWS];
    float* y[ROWS];
    const float* bias[ROWS];
    bool ok[ROWS];
    int jl0;  // first logical row of the slot
};

// Logical rows of a slot. SwiGLU: the first ROWS/2 are gate rows, the rest the
// up rows of the same indices. Rows past the end are clamped to row 0 so every
// load stays in bounds; their results are dropped.
template <int ROWS, int RG>
__device__ __forceinline__ void map_rows(const QmvParams& p, int g, int slot, RowSet<ROWS>& R) {
    const int jl0 = g * RG + slot * ROWS;
    R.jl0 = jl0;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        // segments by comparisons and constant indices (see mrow)
        constexpr int H = ROWS >= 2 ? ROWS / 2 : 1;  // SwiGLU launches use an even ROWS
        int j;
        bool s1, s2 = false;
        if (p.epi == ORC_EPI_SWIGLU) {
            j = jl0 / 2 + r % H;
            s1 = r / H == 1;  // compile-time per r
            R.ok[r] = j < p.rows[0];
        } else {
            j = jl0 + r;
            R.ok[r] = j < p.n_rows;
            s1 = p.n_seg > 1 && j >= p.rows[0];
            s2 = p.n_seg > 2 && j >= p.rows[0] + p.rows[1];
            j = s2 ? j - p.rows[0] - p.rows[1] : (s1 ? j - p.rows[0] : j);
        }
        if (!R.ok[r]) {
            s1 = s2 = false;
            j = 0;
        }
        const uint8_t* w = s2 ? spin(p.w[2]) : (s1 ? spin(p.w[1]) : spin(p.w[0]));
        float* yb = s2 ? spin(p.y[2]) : (s1 ? spin(p.y[1]) : spin(p.y[0]));
        const float* bb = s2 ? spin(p.bias[2]) : (s1 ? spin(p.bias[1]) : spin(p.bias[0]));
        R.rp[r] = w + (size_t)j * p.row_bytes;
        R.y[r] = yb + j;
        R.bias[r] = bb ? bb + j : nullptr;
    }
}

// Rows of a slot from its first logical row jl0 (store / accumulate
// epilogues) with rows of rb bytes; rows of the launch past the end, or past
// jlim, are clamped to row 0 of segment 0 and marked not ok.
template <int ROWS>
__device__ __forceinline__ void map_rows_at(const QmvParams& p, int jl0, int jlim, uint64_t rb, RowSet<ROWS>& R) {
    R.jl0 = jl0;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        int j = jl0 + r;
        R.ok[r] = j < jlim;
        bool s1 = R.ok[r] && p.n_seg > 1 && j >= p.rows[0];
        bool s2 = R.ok[r] && p.n_seg > 2 && j >= p.rows[0] + p.rows[1];
        j = !R.ok[r] ? 0 : (s2 ? j - p.rows[0] - p.rows[1] : (s1 ? j - p.rows[0] : j));
        const uint8_t* w = s2 ? spin(p.w[2]) : (s1 ? spin(p.w[1]) : spin(p.w[0]));
        float* yb = s2 ? spin(p.y[2]) : (s1 ? spin(p.y[1]) : spin(p.y[0]));
        const float* bb = s2 ? spin(p.bias[2]) : (s1 ? spin(p.bias[1]) : spin(p.bias[0]));
        R.rp[r] = w + (size_t)j * (R.ok[r] ? rb : 0);
        R.y[r] = yb + j;
        R.bias[r] = bb ? bb + j : nullptr;
    }
}

// PIPE (rows of one batch, many row groups per wave): the next row group's
// loads go out before the current group's arithmetic, two register sets
// taking turns.
template <int QT, int NT, int ROWS, int UPL, int WPE, bool PIPE>
__global__ __launch_bounds__(kQWG) __attribute__((amdgpu_waves_per_eu(WPE))) void k_qmv(QmvParams p) {
    // token block blockIdx.y: tokens [NT y, NT y + NT) of the launch (every block full)
    if (blockIdx.y) {
        const size_t ox = (size_t)blockIdx.y * NT * p.ldx, oy = (size_t)blockIdx.y * NT * p.ldy;
        p.x += ox;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            if (p.y[i]) p.y[i] += oy;
    }
    using T = QTr<QT>;
    constexpr int LPR = T::LPR, G = 64 / LPR, RG = G * ROWS;
    extern __shared__ float smem[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int slot = lane / LPR, li = lane % LPR;
    const int kn = p.n_in;
    const int xs_stride = padx<T::PP>(kn) + 4;
    const int sx_stride = kn / 16;
    float* xs = smem;
    float* sx = xs + NT * xs_stride;
    float* red = sx + NT * sx_stride;  // kQWaves x NT wave sums of x^2

    // A lane owns units li, li + LPR, li + 2 LPR, ... of each of its rows and
    // walks them in batches of UPL (all loads of a batch in flight at once).
    // Units past the end are clamped to unit 0 so loads stay in bounds.
    const int n_batches = (p.units + LPR * UPL - 1) / (LPR * UPL);
    const int gstride = gridDim.x * kQWaves;
    int g = blockIdx.x + gridDim.x * wave;
    Unit<QT, ROWS> U[UPL];
    RowSet<ROWS> R;

    // stage x: the loads of a pass of x (and of the norm weights) go out
    // first; x is stored to LDS with its per-16 sums (4-lane shuffle). The
    // first batch of weights goes out after the staging barrier (late_w):
    // issued earlier, the weight stream of the CU's waves delays the x reads
    // queued behind it (measured: 0.4-1.3 us per launch on 1-30 MB
    // matrices); or (large matrices, row-group pipelining) right after the
    // first pass of x loads, in flight while x is stored.
    // the regrouped Q8_0 layout: the first batch goes out with the x loads,
    // before x is stored, at every size. Its loads are global (the staging's
    // LDS waits skip them) and unconditional (the waits for x count past
    // them instead of draining them at a branch's join); measured against
    // the late order below: C3 269.2 -> 271.2 tok/s. The other types keep
    // the late order for launches under 40 MB: issued early, their weights
    // delay x (C2 greedy 693 -> 663, C4 113.6 -> 111.4 tok/s with the same
    // exact waits)
    constexpr bool kEarly = QT == ORC_Q8_0_X8;
    const bool norm = p.norm_w != nullptr;
    float ss[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) ss[t] = 0.f;
    const int q4 = kn / 4;
    auto load_pass = [&](int b0, float4 (&v)[NT][4], float4 (&gw)[4]) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int i = b0 + m * kQWG + tid;
                v[t][m] = i < q4 ? *(const float4*)(p.x + (size_t)t * p.ldx + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        if (norm) {
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int i = b0 + m * kQWG + tid;
                gw[m] = i < q4 ? *(const float4*)(p.norm_w + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
            }
        }
    };
    auto store_pass = [&](int b0, const float4 (&v)[NT][4], const float4 (&gw)[4]) {
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                const int i = b0 + m * kQWG + tid;
                float4 a = v[t][m];
                if (norm && i < q4) {
                    ss[t] = __builtin_fmaf(a.x, a.x, ss[t]);
                    ss[t] = __builtin_fmaf(a.y, a.y, ss[t]);
                    ss[t] = __builtin_fmaf(a.z, a.z, ss[t]);
                    ss[t] = __builtin_fmaf(a.w, a.w, ss[t]);
                    a.x *= gw[m].x;
                    a.y *= gw[m].y;
                    a.z *= gw[m].z;
                    a.w *= gw[m].w;
                }
                float s16 = (a.x + a.y) + (a.z + a.w);
                s16 += __shfl_xor(s16, 1, 64);
                s16 += __shfl_xor(s16, 2, 64);
                if (i < q4) {
                    *(float4*)(xs + t * xs_stride + padx<T::PP>(4 * i)) = a;
                    if ((tid & 3) == 0) sx[t * sx_stride + i / 4] = s16;
                }
            }
    };
    {
        float4 v[NT][4], gw[4];
        load_pass(0, v, gw);
        if constexpr (kEarly) {  // every wave, no branch: idle waves load group 0's rows
            map_rows<ROWS, RG>(p, g < p.n_groups ? g : 0, slot, R);
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                const int u = li + LPR * i;
                U[i].load(R.rp, u < p.units ? u : 0);
            }
        } else if (!p.late_w && g < p.n_groups) {  // first batch of the first row group
            map_rows<ROWS, RG>(p, g, slot, R);
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                const int u = li + LPR * i;
                U[i].load(R.rp, u < p.units ? u : 0);
            }
        }
        store_pass(0, v, gw);
        for (int b0 = 4 * kQWG; b0 < q4; b0 += 4 * kQWG) {
            load_pass(b0, v, gw);
            store_pass(b0, v, gw);
        }
    }
    if (norm) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float v = ss[t];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            if (lane == 0) red[t * kQWaves + wave] = v;
        }
    }
    __syncthreads();
    if (QT != kMixK && !kEarly && p.late_w && g < p.n_groups) {
        map_rows<ROWS, RG>(p, g, slot, R);
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const int u = li + LPR * i;
            U[i].load(R.rp, u < p.units ? u : 0);
        }
    }
    float inv[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        inv[t] = 1.f;
        if (norm) {
            const float* rw = red + t * kQWaves;
            const float tot = ((rw[0] + rw[1]) + (rw[2] + rw[3])) + ((rw[4] + rw[5]) + (rw[6] + rw[7]));
            inv[t] = 1.f / sqrtf(tot / (float)p.n_in + p.eps);
        }
    }

    const XCtx c{xs, xs_stride, sx, sx_stride, 0};
    // slot reduction (fixed xor butterfly over the LPR lanes) and epilogue
    auto finish = [&](float (&acc)[ROWS][NT], const RowSet<ROWS>& R) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float v = acc[r][t];
#pragma unroll
                for (int o = LPR / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
                acc[r][t] = v;
            }
        if (p.epi == ORC_EPI_SWIGLU) {
#pragma unroll
            for (int r = 0; r < ROWS / 2; ++r)
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    if (li == (r * NT + t) % LPR && R.ok[r]) {
                        const float gv = acc[r][t] * inv[t], uv = acc[r + ROWS / 2][t] * inv[t];
                        R.y[r][(size_t)t * p.ldy] = (gv / (1.f + expf(-gv))) * uv;
                    }
        } else {
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
#pragma unroll
                for (int t = 0; t < NT; ++t)
                    if (li == (r * NT + t) % LPR && R.ok[r]) {
                        float v = acc[r][t] * inv[t];
                        if (R.bias[r]) v += *R.bias[r];
                        float* dst = R.y[r] + (size_t)t * p.ldy;
                        if (p.epi == ORC_EPI_ACCUM) *dst += v;
                        else *dst = v;
                    }
        }
    };
    if constexpr (QT == kMixK) {
        // groups [0, g4): Q4_K rows [0, split_rows), 64 / 32 slots of ROWS
        // rows; then Q6_K rows [split_rows, n_rows), 64 / 16 slots. A group's
        // type is wave-uniform; each keeps its type's unit, lane split and
        // slot reduction, so its rows equal the single-type launches' bit
        // for bit.
        const int rows4 = p.split_rows, g4 = rows4 / (2 * ROWS);
        const uint64_t rb4 = (uint64_t)(kn / 256) * 144, rb6 = (uint64_t)(kn / 256) * 210;
        auto run = [&](auto tag, int gl, int jbase, int jlim, uint64_t rb) {
            constexpr int UT = decltype(tag)::value, L = QTr<UT>::LPR, RGU = (64 / L) * ROWS;
            const int sl = lane / L, lli = lane % L, units = kn / QTr<UT>::EPU;
            RowSet<ROWS> Rr;
            map_rows_at<ROWS>(p, jbase + gl * RGU + sl * ROWS, jlim, rb, Rr);
            Unit<UT, ROWS> Uu[UPL];
            float acc[ROWS][NT];
            zero(acc);
            const int nbt = (units + L * UPL - 1) / (L * UPL);
            for (int bt = 0; bt < nbt; ++bt) {
#pragma unroll
                for (int i = 0; i < UPL; ++i) {
                    const int u = lli + L * (bt * UPL + i);
                    Uu[i].load(Rr.rp, u < units ? u : 0);
                }
#pragma unroll
                for (int i = 0; i < UPL; ++i) {
                    const int u = lli + L * (bt * UPL + i);
                    if (u < units) Uu[i].template compute<NT>(u, c, acc);
                }
            }
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    float v = acc[r][t];
#pragma unroll
                    for (int o = L / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
                    if (lli == (r * NT + t) % L && Rr.ok[r]) {
                        v *= inv[t];
                        if (Rr.bias[r]) v += *Rr.bias[r];
                        float* dst = Rr.y[r] + (size_t)t * p.ldy;
                        if (p.epi == ORC_EPI_ACCUM) *dst += v;
                        else *dst = v;
                    }
                }
        };
        for (; g < p.n_groups; g += gstride) {
            if (g < g4) run(std::integral_constant<int, ORC_Q4_K>{}, g, 0, rows4, rb4);
            else run(std::integral_constant<int, ORC_Q6_K>{}, g - g4, rows4, p.n_rows, rb6);
        }
        return;
    }
    if constexpr (PIPE) {
        Unit<QT, ROWS> V[UPL];
        RowSet<ROWS> R2;
        // computes group gc from cur (rows Rc) after issuing group gc + gstride into nxt (rows Rn)
        auto step = [&](Unit<QT, ROWS> (&cur)[UPL], Unit<QT, ROWS> (&nxt)[UPL], const RowSet<ROWS>& Rc,
                        RowSet<ROWS>& Rn, int gc) {
            const int gn = gc + gstride;
            if (gn < p.n_groups) {
                map_rows<ROWS, RG>(p, gn, slot, Rn);
#pragma unroll
                for (int i = 0; i < UPL; ++i) {
                    const int u = li + LPR * i;
                    nxt[i].load(Rn.rp, u < p.units ? u : 0);
                }
            }
            float acc[ROWS][NT];
            zero(acc);
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                const int u = li + LPR * i;
                if (u < p.units) cur[i].template compute<NT>(u, c, acc);
            }
            finish(acc, Rc);
        };
        while (g < p.n_groups) {
            step(U, V, R, R2, g);
            g += gstride;
            if (g >= p.n_groups) break;
            step(V, U, R2, R, g);
            g += gstride;
        }
        return;
    }
    while (g < p.n_groups) {
        float acc[ROWS][NT];
        zero(acc);
        for (int bt = 0; bt < n_batches; ++bt) {
            if (bt > 0) {
#pragma unroll
                for (int i = 0; i < UPL; ++i) {
                    const int u = li + LPR * (bt * UPL + i);
                    U[i].load(R.rp, u < p.units ? u : 0);
                }
            }
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                const int u = li + LPR * (bt * UPL + i);
                if (u < p.units) U[i].template compute<NT>(u, c, acc);
            }
        }
        finish(acc, R);
        g += gstride;
        if (g < p.n_groups) {
            map_rows<ROWS, RG>(p, g, slot, R);
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                const int u = li + LPR * i;
                U[i].load(R.rp, u < p.units ? u : 0);
            }
        }
    }
}

// ── host side ────────────────────────────────────────────────────────────────
int g_n_cu = 256;
size_t g_lds_max = 64 * 1024;

int gemm_device_init(int device) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess && v > 0) g_n_cu = v;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, device) == hipSuccess && v > 0)
        g_lds_max = std::min<size_t>((size_t)v, 160 * 1024);
    return ORC_OK;
}

void gemm_device_release() {}

static int elems_per_unit(int type) { return type == ORC_Q6_K ? 64 : 32; }
static int block_elems(int type) { return type == ORC_Q4_K || type == ORC_Q6_K || type == ORC_Q8_0_X8 ? 256 : 32; }
static int pad_period(int type) { return type == ORC_Q4_K || type == ORC_Q6_K ? 64 : 32; }

static size_t qmv_lds(int type, int nt, int kn) {
    const int pp = pad_period(type);
    return ((size_t)nt * ((kn + 4 * (kn / pp) + 4) + kn / 16) + (size_t)kQWaves * nt) * sizeof(float);
}

// Tokens per launch: as many as fit the LDS of one workgroup (multi-token
// launches run one workgroup per CU), at most kMaxNT. Chunking never changes a
// (token, row) result.
static int max_tokens(int type, int n_in) {
    int nt = kMaxNT;
    while (nt > 1 && qmv_lds(type, nt, n_in) > g_lds_max) --nt;
    return qmv_lds(type, nt, n_in) <= g_lds_max ? nt : 0;
}


template <int QT, int NT, int ROWS, int UPL, int WPE, bool PIPE = false>
static int launch_shape(const QmvParams& p0, hipStream_t s, const LaunchEvents& ev) {
    QmvParams p = p0;
    const int rg = (64 / QTr<QT>::LPR) * ROWS;
    p.n_groups = (p.n_rows + rg - 1) / rg;
    // mixed: whole groups of two (Q4_K) and four (Q6_K) rows per slot set
    if constexpr (QT == kMixK) p.n_groups = p.split_rows / (2 * ROWS) + (p.n_rows - p.split_rows) / (4 * ROWS);
    // persistent grid: WPE/2 workgroups per CU, at most one per row group,
    // times the launch's blocks of exactly NT tokens (the kernel stages and
    // writes NT rows per block)
    if (p.tok_block != NT || p.n_tok % NT) return set_error(ORC_E_INVALID, "gemm: token blocks must be whole");
    const dim3 grid(std::max(1, std::min(p.n_groups, (WPE / 2) * g_n_cu)), p.n_tok / NT);
    const size_t lds = qmv_lds(QT, NT, p.n_in);
    if (lds > g_lds_max) return set_error(ORC_E_UNSUPPORTED, "gemm: activations do not fit LDS");
    // weights after the staging (one ordering or the other: results are the
    // same); a 53 MB Q8_0 gate+up and the pipelined LM heads keep them early
    double wbytes = 0;
    for (int i = 0; i < p.n_seg; ++i) wbytes += (double)p.seg_rb[i] * p.rows[i];
    p.late_w = QT == kMixK || (!PIPE && wbytes < 40e6);
    if (ev.start)
        hipExtLaunchKernelGGL((k_qmv<QT, NT, ROWS, UPL, WPE, PIPE>), grid, dim3(kQWG), lds, s, ev.start, ev.stop, 0, p);
    else
        hipLaunchKernelGGL((k_qmv<QT, NT, ROWS, UPL, WPE, PIPE>), grid, dim3(kQWG), lds, s, p);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

// Rows per slot, units per lane per batch and waves per SIMD (WPE) per type,
// token count and matrix height, from a sweep of the C1-C3 matrix shapes on
// MI355X (none of them changes a (token, row) result). SwiGLU pairs gate and
// up rows inside a slot and needs an even ROWS.
template <int QT, int NT>
static int launch_nt(const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    const bool pair = p.epi == ORC_EPI_SWIGLU;
    const bool tall = p.n_rows >= 32768;  // LM heads
    if constexpr (QT == ORC_F32 || QT == ORC_F16 || QT == ORC_BF16) {
        // dense units hold 64-128 bytes per row: one unit per lane in flight
        // (two for 2-byte values), no row pipelining
        const int per_lane = (p.units + 31) / 32;
        if constexpr (NT == 1) {
            if (pair) return launch_shape<QT, NT, 2, 1, 4>(p, s, ev);
            if (QT != ORC_F32 && per_lane >= 2) return launch_shape<QT, NT, 1, 2, 4>(p, s, ev);
            return launch_shape<QT, NT, 1, 1, 4>(p, s, ev);
        } else {
            if (pair) return launch_shape<QT, NT, 2, 1, 2>(p, s, ev);
            return launch_shape<QT, NT, 1, 1, 2>(p, s, ev);
        }
    }
    if constexpr (NT == 1) {
        if ((QT == ORC_Q6_K && tall) || pair) return launch_shape<QT, NT, 2, 1, 4>(p, s, ev);
        // units per lane per batch: at most what a row gives a lane (the
        // clamped extra loads of a shorter row only cost: a 151936 x 896
        // Q8_0 head took 80 us with three per batch, 41 us with one)
        const int per_lane = (p.units + QTr<QT>::LPR - 1) / QTr<QT>::LPR;
        if (tall && per_lane <= 3) {  // rows of one batch: row groups double-buffered
            if (per_lane == 1) return launch_shape<QT, NT, 1, 1, 4, true>(p, s, ev);
            if (per_lane == 2) return launch_shape<QT, NT, 1, 2, 4, true>(p, s, ev);
            return launch_shape<QT, NT, 1, 3, 4, true>(p, s, ev);
        }
        if (per_lane == 1) return launch_shape<QT, NT, 1, 1, 4>(p, s, ev);
        if (per_lane == 2) return launch_shape<QT, NT, 1, 2, 4>(p, s, ev);
        // long rows (4+ units per lane): byte-code types take four units per
        // batch, Q4_K two rows of two (16384 x 8192 over rotating weights:
        // Q8_0_X8 28.2 -> 26.7 us, Q4_K 26.0 -> 24.5, Q4_0 24.0 -> 23.3; the
        // C1-C3 streams and rates unchanged); Q6_K keeps three (four: 27.6 ->
        // 35.9 us)
        if constexpr (QT == ORC_Q8_0 || QT == ORC_Q8_0_X8 || QT == ORC_Q4_0) {
            if (per_lane >= 4) return launch_shape<QT, NT, 1, 4, 4>(p, s, ev);
        }
        if constexpr (QT == ORC_Q4_K) {
            if (per_lane >= 4) return launch_shape<QT, NT, 2, 2, 4>(p, s, ev);
        }
        return launch_shape<QT, NT, 1, 3, 4>(p, s, ev);
    } else {
        if (pair || tall) return launch_shape<QT, NT, 2, 1, 2>(p, s, ev);
        return launch_shape<QT, NT, 1, 1, 2>(p, s, ev);
    }
}

template <int QT>
static int launch_type(const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    if constexpr (QT == ORC_Q4_K || QT == ORC_Q6_K) {  // K-quants: one-token calls only
        if (p.n_tok != 1 || p.tok_block != 1) return set_error(ORC_E_UNSUPPORTED, "gemm: K-quant vector path takes one token");
        return launch_nt<QT, 1>(p, s, ev);
    }
    switch (p.tok_block) {
        case 1: return launch_nt<QT, 1>(p, s, ev);
        case 2: return launch_nt<QT, 2>(p, s, ev);
        case 3: return launch_nt<QT, 3>(p, s, ev);
        case 4: return launch_nt<QT, 4>(p, s, ev);
        case 5: return launch_nt<QT, 5>(p, s, ev);
        default: return set_error(ORC_E_UNSUPPORTED, "n_tok chunk must be 1..5");
    }
}

// ── live kernel timing (orc_prof_*) ─────────────────────────────────────────
struct ProfRec {
    hipEvent_t a, b;
    int type, nt;
    double bytes;
    double sum_ms = 0;  // accumulated over orc_prof_accumulate calls
    int64_t n = 0;
};
static bool g_prof_on = false;
static std::vector<ProfRec> g_prof;
static std::vector<hipEvent_t> g_evpool;
static size_t g_evnext = 0;

static hipEvent_t prof_event() {
    if (g_evnext == g_evpool.size()) {
        hipEvent_t e;
        if (hipEventCreate(&e) != hipSuccess) return nullptr;
        g_evpool.push_back(e);
    }
    return g_evpool[g_evnext++];
}

// Algorithmic HBM bytes of one launch: weight blocks + activations read +
// outputs written (read too when accumulating) + norm weights and biases.
static double gemm_bytes(const QmvParams& p, int nt) {
    const int n_y = p.epi == ORC_EPI_SWIGLU ? p.rows[0] : p.n_rows;
    double b = 4.0 * nt * p.n_in + 4.0 * nt * n_y * (p.epi == ORC_EPI_ACCUM ? 2 : 1);
    for (int i = 0; i < p.n_seg; ++i) b += (double)p.seg_rb[i] * p.rows[i];
    if (p.norm_w) b += 4.0 * p.n_in;
    for (int i = 0; i < p.n_seg; ++i)
        if (p.bias[i]) b += 4.0 * p.rows[i];
    return b;
}

static int gemm_dispatch(QmvParams p, int type, hipStream_t s);

// A one-token launch over Q4_K and Q6_K segments: one vector launch per run
// of segments of one type, each with the norm prologue.
static int dispatch_mixed_decode(const QmvParams& p, hipStream_t s) {
    // Q4_K segments followed by Q6_K segments (a Q4_K_M layer's Q|K|V): one
    // launch whose row groups take their own type (whole groups of each)
    int n4 = 0;
    while (n4 < p.n_seg && p.seg_type[n4] == ORC_Q4_K) ++n4;
    bool ordered = n4 > 0 && n4 < p.n_seg && p.epi != ORC_EPI_SWIGLU;
    int rows4 = 0;
    for (int i = 0; i < p.n_seg; ++i) {
        if (i >= n4 && p.seg_type[i] != ORC_Q6_K) ordered = false;
        if (i < n4) rows4 += p.rows[i];
    }
    if (ordered && rows4 % 2 == 0 && (p.n_rows - rows4) % 4 == 0 && max_tokens(ORC_Q4_K, p.n_in) >= 1) {
        QmvParams q = p;
        q.split_rows = rows4;
        q.tok_block = 1;
        LaunchEvents ev;
        if (g_prof_on) prof_arm(s, kMixK, 1, gemm_bytes(q, 1), &ev.start, &ev.stop);
        const int per_lane = (p.n_in / 32 + 31) / 32;  // Q4_K units per lane; Q6_K's are no more
        if (per_lane == 1) return launch_shape<kMixK, 1, 1, 1, 4>(q, s, ev);
        if (per_lane == 2) return launch_shape<kMixK, 1, 1, 2, 4>(q, s, ev);
        return launch_shape<kMixK, 1, 1, 3, 4>(q, s, ev);
    }
    for (int i0 = 0; i0 < p.n_seg;) {
        int i1 = i0 + 1;
        while (i1 < p.n_seg && p.seg_type[i1] == p.seg_type[i0]) ++i1;
        QmvParams q = p;
        q.n_seg = i1 - i0;
        q.n_rows = 0;
        for (int i = 0; i < 3; ++i) {
            const int j = i0 + i;
            const bool in = i < q.n_seg;
            q.w[i] = in ? p.w[j] : nullptr;
            q.y[i] = in ? p.y[j] : nullptr;
            q.bias[i] = in ? p.bias[j] : nullptr;
            q.rows[i] = in ? p.rows[j] : 0;
            q.seg_type[i] = in ? p.seg_type[j] : 0;
            q.seg_rb[i] = in ? p.seg_rb[j] : 0;
            q.n_rows += q.rows[i];
        }
        q.row_bytes = q.seg_rb[0];
        if (int rc = gemm_dispatch(q, q.seg_type[0], s)) return rc;
        i0 = i1;
    }
    return ORC_OK;
}

static int gemm_dispatch(QmvParams p, int type, hipStream_t s) {
    // a one-token call (decode) runs on the vector ALUs for every type; the
    // K-quants take the matrix cores from two tokens up. The choice follows
    // the call's token count, never a chunk's, so chunking keeps results.
    const bool decode = p.n_tok == 1;
    if (decode && type == kMixK) return dispatch_mixed_decode(p, s);
    p.units = p.n_in / elems_per_unit(type);
    const bool mm = mmq_type(type) && !decode;
    // a prefill pass (K-quant and Q8_0 calls of kPfMinTok tokens or more):
    // every token in one launch on the matrix cores
    if (!decode && (mm || type == ORC_Q8_0 || type == ORC_Q8_0_X8) && mmq_prefill(type, p)) {
        LaunchEvents ev;
        if (g_prof_on) prof_arm(s, type, p.n_tok, gemm_bytes(p, p.n_tok), &ev.start, &ev.stop);
        return mmq_prefill_launch(type, p, s, ev);
    }
    const int ntmax = mm ? mmq_max_tokens(type, p) : max_tokens(type, p.n_in);
    if (ntmax < 1) return set_error(ORC_E_UNSUPPORTED, "gemm: n_in too large for the activations to fit LDS");
    // Tokens go in blocks of ntmax (the second grid dimension of one launch:
    // every kernel computes exactly its instantiated token count per block),
    // and the remainder in a second launch of its own size. Blocking never
    // changes a (token, row) result: the reduction order is independent of
    // the token count.
    for (int t0 = 0; t0 < p.n_tok;) {
        const int left = p.n_tok - t0;
        QmvParams q = p;
        q.tok_block = std::min(ntmax, left);
        q.n_tok = left >= ntmax ? left / ntmax * ntmax : left;
        q.x = p.x + (size_t)t0 * p.ldx;
        for (int i = 0; i < 3; ++i) q.y[i] = p.y[i] ? p.y[i] + (size_t)t0 * p.ldy : nullptr;
        t0 += q.n_tok;
        LaunchEvents ev;
        if (g_prof_on) prof_arm(s, type, q.n_tok, gemm_bytes(q, q.n_tok), &ev.start, &ev.stop);
        int rc;
        switch (type) {
            case ORC_Q4_K: rc = mm ? mmq_launch(type, q, s, ev) : launch_type<ORC_Q4_K>(q, s, ev); break;
            case ORC_Q6_K: rc = mm ? mmq_launch(type, q, s, ev) : launch_type<ORC_Q6_K>(q, s, ev); break;
            case kMixK: rc = mmq_launch(type, q, s, ev); break;
            case ORC_Q8_0: rc = launch_type<ORC_Q8_0>(q, s, ev); break;
            case ORC_Q8_0_X8: rc = launch_type<ORC_Q8_0_X8>(q, s, ev); break;
            case ORC_Q4_0: rc = launch_type<ORC_Q4_0>(q, s, ev); break;
            case ORC_F32: rc = launch_type<ORC_F32>(q, s, ev); break;
            case ORC_F16: rc = launch_type<ORC_F16>(q, s, ev); break;
            case ORC_BF16: rc = launch_type<ORC_BF16>(q, s, ev); break;
            default: return set_error(ORC_E_UNSUPPORTED, "gemm: unsupported weight type " + std::to_string(type));
        }
        if (rc) return rc;
    }
    return ORC_OK;
}

bool prof_arm(hipStream_t s, int family, int n_tok, double bytes, hipEvent_t* start, hipEvent_t* stop) {
    if (!g_prof_on) return false;  // host launches only: a captured launch carries no events
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    (void)hipStreamIsCapturing(s, &cs);
    ProfRec rec{};
    if (cs != hipStreamCaptureStatusNone || !(rec.a = prof_event()) || !(rec.b = prof_event())) return false;
    rec.type = family;
    rec.nt = n_tok;
    rec.bytes = bytes;
    g_prof.push_back(rec);
    *start = rec.a;
    *stop = rec.b;
    return true;
}

}  // namespace orc

using namespace orc;

extern "C" int orc_prof_enable(int on) {
    const int prev = g_prof_on ? 1 : 0;
    g_prof_on = on != 0;
    if (on == 1) {
        g_prof.clear();
        g_evnext = 0;
    }
    return prev;
}

extern "C" int orc_prof_accumulate(void) {
    if (!g_prof_on) return ORC_OK;
    for (ProfRec& r : g_prof) {
        ORC_HIP_CHECK(hipEventSynchronize(r.b));
        float e = 0.f;
        ORC_HIP_CHECK(hipEventElapsedTime(&e, r.a, r.b));
        r.sum_ms += e;
        ++r.n;
    }
    return ORC_OK;
}

extern "C" int orc_prof_read(int type, int n_tok, int64_t* launches, double* total_ms, double* total_bytes) {
    int64_t n = 0;
    double ms = 0, by = 0;
    for (const ProfRec& r : g_prof) {
        if ((type >= 0 && r.type != type) || (n_tok > 0 && r.nt != n_tok)) continue;
        n += r.n;
        ms += r.sum_ms;
        by += r.bytes * (double)r.n;
    }
    if (launches) *launches = n;
    if (total_ms) *total_ms = ms;
    if (total_bytes) *total_bytes = by;
    return ORC_OK;
}

extern "C" int64_t orc_row_bytes(int type, int64_t n) {
    switch (type) {
        case ORC_F32: return n * 4;
        case ORC_F16: return n * 2;
        case ORC_BF16: return n * 2;
        case ORC_Q4_0: return n % 32 ? -1 : n / 32 * 18;
        case ORC_Q8_0: return n % 32 ? -1 : n / 32 * 34;
        case ORC_Q8_0_X8: return n % 256 ? -1 : n / 32 * 34;
        case ORC_Q4_K: return n % 256 ? -1 : n / 256 * 144;
        case ORC_Q6_K: return n % 256 ? -1 : n / 256 * 210;
        default: return -1;
    }
}

// One thread per 272-byte group: the 8 blocks are read whole before the
// group is rewritten, and no other thread touches it, so the change is in
// place.
__global__ __launch_bounds__(256) void k_q8_0_regroup(uint8_t* w, int64_t n8) {
    const int64_t gi = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gi >= n8) return;
    uint8_t* g = w + gi * 272;
    uint16_t d[8];
    u32x4 q[16];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const uint8_t* blk = g + 34 * b;
        d[b] = (uint16_t)ld2(blk);
        q[2 * b] = ld16(blk + 2);
        q[2 * b + 1] = ld16(blk + 18);
    }
    asm volatile("" ::: "memory");  // every read of the group before the first write
    uint16_t* ds = (uint16_t*)g;
#pragma unroll
    for (int b = 0; b < 8; ++b) ds[b] = d[b];
    u32x4* qs = (u32x4*)(g + 16);
#pragma unroll
    for (int i = 0; i < 16; ++i) qs[i] = q[i];
}

static int check_gemm_shape(int type, int n_tok, int n_in, const float* x, int ldx, int ldy, const void* w) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (type != ORC_Q4_K && type != ORC_Q6_K && type != ORC_Q8_0 && type != ORC_Q8_0_X8 && type != ORC_Q4_0 &&
        type != ORC_F32 && type != ORC_F16 && type != ORC_BF16)
        return set_error(ORC_E_UNSUPPORTED, "gemm: unsupported weight type " + std::to_string(type));
    if (n_tok < 1 || n_in <= 0 || n_in % block_elems(type))
        return set_error(ORC_E_INVALID, "gemm: n_in must be a positive multiple of the block size");
    if (!x || !w || ldx < n_in || ldx % 4 || ldy < 1)
        return set_error(ORC_E_INVALID, "gemm: bad pointers or strides (ldx >= n_in, ldx % 4 == 0)");
    if (((uintptr_t)x & 15) != 0) return set_error(ORC_E_INVALID, "gemm: x must be 16-byte aligned");
    if (type == ORC_Q8_0_X8 && ((uintptr_t)w & 15))
        return set_error(ORC_E_INVALID, "gemm: Q8_0_X8 weights must be 16-byte aligned");
    if (type == ORC_F32 && ((uintptr_t)w & 3))
        return set_error(ORC_E_INVALID, "gemm: F32 weights must be 4-byte aligned");
    return ORC_OK;
}

extern "C" int orc_gemm(int type, const void* d_w, int n_tok, int n_out, int n_in, const float* d_x, int ldx,
                        float* d_y, int ldy, orc_stream_t stream) {
    if (int rc = check_gemm_shape(type, n_tok, n_in, d_x, ldx, ldy, d_w)) return rc;
    if (n_out <= 0 || !d_y || (n_tok > 1 && ldy < n_out)) return set_error(ORC_E_INVALID, "gemm: bad output");
    QmvParams p{};
    p.w[0] = (const uint8_t*)d_w;
    p.y[0] = d_y;
    p.rows[0] = n_out;
    p.n_seg = 1;
    p.n_rows = n_out;
    p.n_in = n_in;
    p.row_bytes = (uint64_t)orc_row_bytes(type, n_in);
    p.seg_rb[0] = p.row_bytes;
    p.seg_type[0] = type;
    p.x = d_x;
    p.ldx = ldx;
    p.ldy = ldy;
    p.n_tok = n_tok;
    p.epi = ORC_EPI_STORE;
    return gemm_dispatch(p, type, resolve_stream(stream));
}

extern "C" int orc_gemm_fused(int type, const orc_seg* segs, int n_segs, int n_tok, int n_in, const float* d_x,
                              int ldx, int ldy, const float* d_norm_w, float eps, int epilogue, orc_stream_t stream) {
    if (int rc = check_gemm_shape(type, n_tok, n_in, d_x, ldx, ldy, segs ? segs[0].d_w : nullptr)) return rc;
    if (n_segs < 1 || n_segs > 3) return set_error(ORC_E_INVALID, "gemm_fused: 1..3 segments");
    if (epilogue == ORC_EPI_SWIGLU && (n_segs != 2 || segs[0].n_out != segs[1].n_out))
        return set_error(ORC_E_INVALID, "gemm_fused: SwiGLU needs gate and up segments of equal rows");
    if (epilogue < ORC_EPI_STORE || epilogue > ORC_EPI_SWIGLU) return set_error(ORC_E_INVALID, "bad epilogue");
    if (d_norm_w && ((uintptr_t)d_norm_w & 15)) return set_error(ORC_E_INVALID, "norm weights must be 16-byte aligned");
    QmvParams p{};
    int total = 0;
    for (int i = 0; i < n_segs; ++i) {
        if (!segs[i].d_w || !segs[i].d_y || segs[i].n_out <= 0) return set_error(ORC_E_INVALID, "gemm_fused: bad segment");
        if (type == ORC_Q8_0_X8 && ((uintptr_t)segs[i].d_w & 15))
            return set_error(ORC_E_INVALID, "gemm: Q8_0_X8 weights must be 16-byte aligned");
        p.w[i] = (const uint8_t*)segs[i].d_w;
        p.y[i] = segs[i].d_y;
        p.bias[i] = segs[i].d_bias;
        p.rows[i] = segs[i].n_out;
        total += segs[i].n_out;
    }
    p.n_seg = n_segs;
    p.n_rows = epilogue == ORC_EPI_SWIGLU ? 2 * segs[0].n_out : total;
    p.n_in = n_in;
    p.row_bytes = (uint64_t)orc_row_bytes(type, n_in);
    for (int i = 0; i < n_segs; ++i) {
        p.seg_rb[i] = p.row_bytes;
        p.seg_type[i] = type;
    }
    p.x = d_x;
    p.ldx = ldx;
    p.ldy = ldy;
    p.n_tok = n_tok;
    p.norm_w = d_norm_w;
    p.eps = eps;
    p.epi = epilogue;
    return gemm_dispatch(p, type, resolve_stream(stream));
}

extern "C" int orc_gemm_fused_mixed(const int* types, const orc_seg* segs, int n_segs, int n_tok, int n_in,
                                    const float* d_x, int ldx, int ldy, const float* d_norm_w, float eps, int epilogue,
                                    orc_stream_t stream) {
    if (!types || !segs || n_segs < 1 || n_segs > 3) return set_error(ORC_E_INVALID, "gemm_fused_mixed: 1..3 segments");
    if (epilogue != ORC_EPI_STORE && epilogue != ORC_EPI_ACCUM)
        return set_error(ORC_E_INVALID, "gemm_fused_mixed: store or accumulate epilogue");
    if (d_norm_w && ((uintptr_t)d_norm_w & 15)) return set_error(ORC_E_INVALID, "norm weights must be 16-byte aligned");
    QmvParams p{};
    int total = 0;
    for (int i = 0; i < n_segs; ++i) {
        if (types[i] != ORC_Q4_K && types[i] != ORC_Q6_K)
            return set_error(ORC_E_UNSUPPORTED, "gemm_fused_mixed: segments must be Q4_K or Q6_K");
        if (int rc = check_gemm_shape(types[i], n_tok, n_in, d_x, ldx, ldy, segs[i].d_w)) return rc;
        if (!segs[i].d_y || segs[i].n_out <= 0 || segs[i].n_out % 16)
            return set_error(ORC_E_INVALID, "gemm_fused_mixed: segment rows must be a positive multiple of 16");
        if (segs[i].n_out >= 65536)
            return set_error(ORC_E_UNSUPPORTED, "gemm_fused_mixed: a segment of 65536 rows or more runs alone");
        p.w[i] = (const uint8_t*)segs[i].d_w;
        p.y[i] = segs[i].d_y;
        p.bias[i] = segs[i].d_bias;
        p.rows[i] = segs[i].n_out;
        p.seg_type[i] = types[i];
        p.seg_rb[i] = (uint64_t)orc_row_bytes(types[i], n_in);
        total += segs[i].n_out;
    }
    p.n_seg = n_segs;
    p.n_rows = total;
    p.n_in = n_in;
    p.row_bytes = p.seg_rb[0];
    p.x = d_x;
    p.ldx = ldx;
    p.ldy = ldy;
    p.n_tok = n_tok;
    p.norm_w = d_norm_w;
    p.eps = eps;
    p.epi = epilogue;
    return gemm_dispatch(p, kMixK, resolve_stream(stream));
}

extern "C" int orc_q8_0_regroup(void* d_w, int64_t n_blocks8, orc_stream_t stream) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_w || n_blocks8 < 0 || ((uintptr_t)d_w & 15))
        return set_error(ORC_E_INVALID, "q8_0_regroup: null or not 16-byte aligned weights");
    if (n_blocks8 == 0) return ORC_OK;
    const int64_t nb = (n_blocks8 + 255) / 256;
    if (nb > 0x7fffffff) return set_error(ORC_E_INVALID, "q8_0_regroup: too many groups");
    hipLaunchKernelGGL(k_q8_0_regroup, dim3((unsigned)nb), dim3(256), 0, resolve_stream(stream), (uint8_t*)d_w,
                       n_blocks8);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

// Quantized GEMV / GEMM on raw GGML blocks (gfx950).
//
// Replaces gemv_q / gemv_q_range / gemm_q (core/gguf_parser.cpp:496-997) and
// the projection sequences of Model::forward / forward_prefill that surround
// them (RMSNorm, QKV bias, residual add, SwiGLU; core/model.cpp:366-473,
// 565-643).
//
// Design (one kernel family; n_tok = 1 is the decode GEMV):
//  * A 256-thread workgroup owns a tile of weight rows. A "row group" of
//    KS*LPR lanes (LPR lanes in each of KS waves) owns ROWS rows and walks
//    their row bytes in units: 16 B of Q4_K nibbles (32 values), a 64-value
//    quarter of a Q6_K superblock, one Q8_0 / Q4_0 block. Blocks are read
//    straight from the as-uploaded GGUF bytes with (unaligned) 128-bit loads.
//  * Latency: each lane issues the loads of its first unit before the
//    activations are staged, and the loads of unit i+1 before computing unit
//    i, so HBM latency overlaps the L2 staging and the arithmetic.
//  * The activations of all n_tok tokens for one K tile are staged in LDS
//    (fp32, 4 floats of padding every 32/64 values so the lanes of a group hit
//    distinct banks) with every load in flight at once; per-16-value sums of x
//    (for the Q4_K minimum and the Q6_K / Q4_0 code offsets) come from a
//    4-lane shuffle in the same pass. One barrier per K tile.
//  * RMSNorm prologue: x is staged multiplied by the norm weight and the
//    per-token 1/rms (reduced while staging) scales the finished dot product:
//    sum_i w_i (x_i s g_i) = s * sum_i w_i (x_i g_i).
//  * Each weight code is decoded once per row and applied to every token in
//    LDS; accumulation is fp32. A lane's partial sum depends only on the units
//    it owns, the group reduction is a fixed xor butterfly plus a fixed-order
//    sum over waves, and the RMS reduction uses a fixed thread mapping per
//    token, so a (token, row) result is bit-identical for every n_tok: the
//    (k+1)-token verify pass equals k+1 separate decode GEMVs.
#include "orc_internal.hpp"

#include <algorithm>
#include <vector>

namespace orc {

template <int QT> struct QTr;
template <> struct QTr<ORC_Q8_0> { static constexpr int BLK_EL = 32, UPB = 1, PP = 32; };
template <> struct QTr<ORC_Q4_0> { static constexpr int BLK_EL = 32, UPB = 1, PP = 32; };
template <> struct QTr<ORC_Q4_K> { static constexpr int BLK_EL = 256, UPB = 8, PP = 64; };
template <> struct QTr<ORC_Q6_K> { static constexpr int BLK_EL = 256, UPB = 4, PP = 64; };

template <int PP> __device__ __forceinline__ int padx(int k) { return k + 4 * (k / PP); }

// Σ_{i<16} w[i] * x[i] with x read from LDS as 4 float4 (sequential FMA chain).
__device__ __forceinline__ float dot16(const float* w, const float* xl) {
    const float4* x4 = (const float4*)xl;
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 v = x4[i];
        s = __builtin_fmaf(w[4 * i + 0], v.x, s);
        s = __builtin_fmaf(w[4 * i + 1], v.y, s);
        s = __builtin_fmaf(w[4 * i + 2], v.z, s);
        s = __builtin_fmaf(w[4 * i + 3], v.w, s);
    }
    return s;
}

// Bytes of 4 dwords as 16 floats, byte k of dword i -> w[4i+k].
__device__ __forceinline__ void bytes_to_f(uint32_t a, uint32_t b, uint32_t c, uint32_t d, float* w) {
    const uint32_t q[4] = {a, b, c, d};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int k = 0; k < 4; ++k) w[4 * i + k] = ubyte_f(q[i], k);
}

struct UnitCtx {
    const float* xs;  // LDS x (times the norm weight when fused), token 0, tile element 0, padded
    int xs_stride;    // floats between tokens
    const float* sx;  // LDS per-16 sums of the staged x, token 0
    int sx_stride;
    int k0;           // first element of the tile
};

// ── per-type units: load() issues the loads, compute() does the arithmetic ───
template <int QT, int ROWS> struct Unit;

template <int ROWS> struct Unit<ORC_Q4_K, ROWS> {
    // unit u: superblock u/8, 16-byte nibble chunk c = u%8 of it. Chunk c
    // holds values 64j+16h+[0,16) (low nibbles, sub-block 2j) and
    // 64j+32+16h+[0,16) (high nibbles, sub-block 2j+1), j = c/2, h = c%2.
    u32x4 hdr[ROWS], q[ROWS];
    __device__ __forceinline__ void load(const uint8_t* const (&rows)[ROWS], const bool (&ok)[ROWS], int u) {
        const int b = u >> 3, ch = u & 7;
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            if (ok[r]) {
                const uint8_t* blk = rows[r] + (size_t)b * 144;
                hdr[r] = ld16(blk);
                q[r] = ld16(blk + 16 + 16 * ch);
            }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const UnitCtx& c, const bool (&ok)[ROWS],
                                            float (&acc)[ROWS][NT]) const {
        const int b = u >> 3, ch = u & 7, j = ch >> 1, h = ch & 1;
        const int eA = b * 256 + 64 * j + 16 * h - c.k0, eB = eA + 32;
        const int pA = padx<64>(eA), pB = padx<64>(eB);
        float dA[ROWS], mA[ROWS], dB[ROWS], mB[ROWS], wa[ROWS][16], wb[ROWS][16];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            if (!ok[r]) continue;
            const float d = h2f(hdr[r].x & 0xFFFFu), dmin = h2f(hdr[r].x >> 16);
            uint32_t s0, m0, s1, m1;
            q4k_scale_min(2 * j, hdr[r].y, hdr[r].z, hdr[r].w, s0, m0);
            q4k_scale_min(2 * j + 1, hdr[r].y, hdr[r].z, hdr[r].w, s1, m1);
            dA[r] = d * (float)s0;
            mA[r] = dmin * (float)m0;
            dB[r] = d * (float)s1;
            mB[r] = dmin * (float)m1;
            bytes_to_f(q[r].x & 0x0F0F0F0Fu, q[r].y & 0x0F0F0F0Fu, q[r].z & 0x0F0F0F0Fu, q[r].w & 0x0F0F0F0Fu, wa[r]);
            bytes_to_f((q[r].x >> 4) & 0x0F0F0F0Fu, (q[r].y >> 4) & 0x0F0F0F0Fu, (q[r].z >> 4) & 0x0F0F0F0Fu,
                       (q[r].w >> 4) & 0x0F0F0F0Fu, wb[r]);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float* xt = c.xs + t * c.xs_stride;
            const float sxA = c.sx[t * c.sx_stride + eA / 16], sxB = c.sx[t * c.sx_stride + eB / 16];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                if (!ok[r]) continue;
                const float sA = dot16(wa[r], xt + pA), sB = dot16(wb[r], xt + pB);
                acc[r][t] += dA[r] * sA - mA[r] * sxA + dB[r] * sB - mB[r] * sxB;
            }
        }
    }
};

template <int ROWS> struct Unit<ORC_Q6_K, ROWS> {
    // unit u: superblock u/4, quarter v = u%4: half hh = v/2, l0 = 16*(v%2).
    // Group g (0..3) holds values 128hh+32g+l0+[0,16) with scale sc[8hh+2g+v%2].
    u32x4 qa[ROWS], qb[ROWS], qh[ROWS];
    u32x2 sc[ROWS];
    uint32_t dh[ROWS];
    __device__ __forceinline__ void load(const uint8_t* const (&rows)[ROWS], const bool (&ok)[ROWS], int u) {
        const int b = u >> 2, v = u & 3, hh = v >> 1, l0 = 16 * (v & 1);
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            if (ok[r]) {
                const uint8_t* blk = rows[r] + (size_t)b * 210;
                qa[r] = ld16(blk + 64 * hh + l0);
                qb[r] = ld16(blk + 64 * hh + 32 + l0);
                qh[r] = ld16(blk + 128 + 32 * hh + l0);
                sc[r] = ld8(blk + 192 + 8 * hh);
                dh[r] = ld2(blk + 208);
            }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const UnitCtx& c, const bool (&ok)[ROWS],
                                            float (&acc)[ROWS][NT]) const {
        const int b = u >> 2, v = u & 3, hh = v >> 1, odd = v & 1, l0 = 16 * odd;
        const int e0 = b * 256 + 128 * hh + l0 - c.k0;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float w[ROWS][16], sg[ROWS];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                if (!ok[r]) continue;
                const int si = 2 * g + odd;  // byte index inside the 8 scale bytes of this half
                const uint32_t sw = si < 4 ? sc[r].x : sc[r].y;
                sg[r] = h2f(dh[r]) * (float)(int8_t)((sw >> (8 * (si & 3))) & 0xFFu);
                const uint32_t a4[4] = {qa[r].x, qa[r].y, qa[r].z, qa[r].w};
                const uint32_t b4[4] = {qb[r].x, qb[r].y, qb[r].z, qb[r].w};
                const uint32_t h4[4] = {qh[r].x, qh[r].y, qh[r].z, qh[r].w};
                uint32_t qq[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t nib, hb;
                    if (g == 0) { nib = a4[i] & 0x0F0F0F0Fu; hb = (h4[i] << 4) & 0x30303030u; }
                    else if (g == 1) { nib = b4[i] & 0x0F0F0F0Fu; hb = (h4[i] << 2) & 0x30303030u; }
                    else if (g == 2) { nib = (a4[i] >> 4) & 0x0F0F0F0Fu; hb = h4[i] & 0x30303030u; }
                    else { nib = (b4[i] >> 4) & 0x0F0F0F0Fu; hb = (h4[i] >> 2) & 0x30303030u; }
                    qq[i] = nib | hb;
                }
                bytes_to_f(qq[0], qq[1], qq[2], qq[3], w[r]);
            }
            const int eg = e0 + 32 * g;
            const int pg = padx<64>(eg);
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float* xt = c.xs + t * c.xs_stride;
                const float sxg = c.sx[t * c.sx_stride + eg / 16];
#pragma unroll
                for (int r = 0; r < ROWS; ++r) {
                    if (!ok[r]) continue;
                    // codes are stored +32: Σ (q-32) x = Σ q x - 32 Σ x
                    acc[r][t] += sg[r] * (dot16(w[r], xt + pg) - 32.f * sxg);
                }
            }
        }
    }
};

template <int ROWS> struct Unit<ORC_Q8_0, ROWS> {
    // unit u: block u (fp16 d + 32 int8 codes): acc += d * Σ q x.
    u32x4 q0[ROWS], q1[ROWS];
    uint32_t dh[ROWS];
    __device__ __forceinline__ void load(const uint8_t* const (&rows)[ROWS], const bool (&ok)[ROWS], int u) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            if (ok[r]) {
                const uint8_t* blk = rows[r] + (size_t)u * 34;
                dh[r] = ld2(blk);
                q0[r] = ld16(blk + 2);
                q1[r] = ld16(blk + 18);
            }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const UnitCtx& c, const bool (&ok)[ROWS],
                                            float (&acc)[ROWS][NT]) const {
        const int e0 = u * 32 - c.k0;
        const int p0 = padx<32>(e0);
        float w[ROWS][32], d[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            if (!ok[r]) continue;
            d[r] = h2f(dh[r]);
            const uint32_t qq[8] = {q0[r].x, q0[r].y, q0[r].z, q0[r].w, q1[r].x, q1[r].y, q1[r].z, q1[r].w};
#pragma unroll
            for (int i = 0; i < 8; ++i)
#pragma unroll
                for (int k = 0; k < 4; ++k) w[r][4 * i + k] = (float)(int8_t)((qq[i] >> (8 * k)) & 0xFFu);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float* xt = c.xs + t * c.xs_stride + p0;
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                if (!ok[r]) continue;
                acc[r][t] += d[r] * (dot16(w[r], xt) + dot16(w[r] + 16, xt + 16));
            }
        }
    }
};

template <int ROWS> struct Unit<ORC_Q4_0, ROWS> {
    // unit u: block u (fp16 d + 16 bytes: low nibble -> value l, high -> l+16), codes stored +8.
    u32x4 q[ROWS];
    uint32_t dh[ROWS];
    __device__ __forceinline__ void load(const uint8_t* const (&rows)[ROWS], const bool (&ok)[ROWS], int u) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
            if (ok[r]) {
                const uint8_t* blk = rows[r] + (size_t)u * 18;
                dh[r] = ld2(blk);
                q[r] = ld16(blk + 2);
            }
    }
    template <int NT>
    __device__ __forceinline__ void compute(int u, const UnitCtx& c, const bool (&ok)[ROWS],
                                            float (&acc)[ROWS][NT]) const {
        const int e0 = u * 32 - c.k0;
        const int p0 = padx<32>(e0);
        float wl[ROWS][16], wh[ROWS][16], d[ROWS];
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            if (!ok[r]) continue;
            d[r] = h2f(dh[r]);
            bytes_to_f(q[r].x & 0x0F0F0F0Fu, q[r].y & 0x0F0F0F0Fu, q[r].z & 0x0F0F0F0Fu, q[r].w & 0x0F0F0F0Fu, wl[r]);
            bytes_to_f((q[r].x >> 4) & 0x0F0F0F0Fu, (q[r].y >> 4) & 0x0F0F0F0Fu, (q[r].z >> 4) & 0x0F0F0F0Fu,
                       (q[r].w >> 4) & 0x0F0F0F0Fu, wh[r]);
        }
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float* xt = c.xs + t * c.xs_stride + p0;
            const float sxs = c.sx[t * c.sx_stride + e0 / 16] + c.sx[t * c.sx_stride + e0 / 16 + 1];
#pragma unroll
            for (int r = 0; r < ROWS; ++r) {
                if (!ok[r]) continue;
                acc[r][t] += d[r] * ((dot16(wl[r], xt) + dot16(wh[r], xt + 16)) - 8.f * sxs);
            }
        }
    }
};

// ── the GEMM kernel ──────────────────────────────────────────────────────────
struct GemmParams {
    const uint8_t* w[3];
    float* y[3];
    const float* bias[3];
    int rows[3];
    int n_seg;
    int tile_rows_total;  // rows (or gate/up pairs) covered by the grid
    int n_in;
    int units_per_row;
    uint64_t row_bytes;
    const float* x;
    int ldx, ldy, n_tok;
    const float* norm_w;
    float eps;
    int epi;
    int kt_el;     // K tile in elements (a multiple of 1024 when n_in is split)
    int n_ktiles;
};

constexpr int kWG = 256;
constexpr int kMaxNT = 5;  // tokens per launch; larger batches are chunked (results unchanged)

template <int QT, int NT, int LPR, int KS, int ROWS>
__global__ __launch_bounds__(kWG) void k_gemm(GemmParams p) {
    using T = QTr<QT>;
    extern __shared__ float smem[];
    constexpr int G = 64 / LPR;     // groups per wave
    constexpr int GR = 4 / KS;      // wave rows
    constexpr int LT = KS * LPR;    // lanes per group
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wsub = wave % KS, wrow = wave / KS;
    const int li = wsub * LPR + lane % LPR, gl = wrow * G + lane / LPR;
    const int xs_stride = padx<T::PP>(p.kt_el) + 4;
    const int sx_stride = p.kt_el / 16;
    float* xs = smem;
    float* sx = smem + NT * xs_stride;
    float* red = sx + NT * sx_stride;  // 4*NT wave partials of sum x^2, then KS partial sums
    float* part = red + 4 * NT;

    // rows owned by this lane group
    const uint8_t* rows[ROWS];
    bool ok[ROWS];
    float* yout[ROWS];
    const float* bias[ROWS];
    const int base = (blockIdx.x * GR * G + gl) * ROWS;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        int seg = 0, j;
        if (p.epi == ORC_EPI_SWIGLU) {  // slot 0 = gate row, slot 1 = up row of the same index
            j = base / ROWS;
            seg = r;
            ok[r] = j < p.rows[0];
        } else {
            j = base + r;
            ok[r] = j < p.tile_rows_total;
            while (seg + 1 < p.n_seg && j >= p.rows[seg]) { j -= p.rows[seg]; ++seg; }
        }
        rows[r] = p.w[seg] + (size_t)(ok[r] ? j : 0) * p.row_bytes;
        yout[r] = p.y[seg] + j;
        bias[r] = p.bias[seg] ? p.bias[seg] + j : nullptr;
    }

    float acc[ROWS][NT], ss[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        ss[t] = 0.f;
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc[r][t] = 0.f;
    }
    const bool norm = p.norm_w != nullptr;
    const int units_per_tile = p.kt_el / T::BLK_EL * T::UPB;
    Unit<QT, ROWS> cur, nxt;
    for (int kt = 0; kt < p.n_ktiles; ++kt) {
        const int k0 = kt * p.kt_el;
        const int kn = min(p.kt_el, p.n_in - k0);
        const int u1 = min(p.units_per_row, kt * units_per_tile + units_per_tile);
        int u = kt * units_per_tile + li;
        if (u < u1) cur.load(rows, ok, u);  // in flight while x is staged
        if (kt) __syncthreads();            // previous tile fully consumed
        // stage the tile: all loads first, then LDS stores and per-16 sums (4-lane shuffle)
        const int q4 = kn / 4;
        for (int t = 0; t < NT; ++t) {
            const float* src = p.x + (size_t)t * p.ldx + k0;
            for (int b0 = 0; b0 < q4; b0 += 4 * kWG) {
                float4 v[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int i = b0 + s * kWG + tid;
                    v[s] = i < q4 ? *(const float4*)(src + 4 * i) : make_float4(0.f, 0.f, 0.f, 0.f);
                }
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int i = b0 + s * kWG + tid;
                    float4 a = v[s];
                    if (norm && i < q4) {
                        ss[t] = __builtin_fmaf(a.x, a.x, ss[t]);
                        ss[t] = __builtin_fmaf(a.y, a.y, ss[t]);
                        ss[t] = __builtin_fmaf(a.z, a.z, ss[t]);
                        ss[t] = __builtin_fmaf(a.w, a.w, ss[t]);
                        const float4 g = *(const float4*)(p.norm_w + k0 + 4 * i);
                        a.x *= g.x; a.y *= g.y; a.z *= g.z; a.w *= g.w;
                    }
                    float s16 = (a.x + a.y) + (a.z + a.w);
                    s16 += __shfl_xor(s16, 1, 64);
                    s16 += __shfl_xor(s16, 2, 64);
                    if (i < q4) {
                        *(float4*)(xs + t * xs_stride + padx<T::PP>(4 * i)) = a;
                        if ((tid & 3) == 0) sx[t * sx_stride + i / 4] = s16;
                    }
                }
            }
        }
        __syncthreads();
        const UnitCtx c{xs, xs_stride, sx, sx_stride, k0};
        for (; u < u1; u += LT) {
            const int un = u + LT;
            if (un < u1) nxt.load(rows, ok, un);
            cur.template compute<NT>(u, c, ok, acc);
            cur = nxt;
        }
    }

    // 1/rms per token: a fixed reduction order for every n_tok (as orc_rmsnorm)
    float inv[NT];
    if (norm) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float v = ss[t];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            if (lane == 0) red[4 * t + wave] = v;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < NT; ++t)
            inv[t] = 1.f / sqrtf(((red[4 * t] + red[4 * t + 1]) + (red[4 * t + 2] + red[4 * t + 3])) / (float)p.n_in +
                                 p.eps);
    }

    // reduction: xor butterfly over the LPR lanes of a wave, then the KS waves in fixed order
#pragma unroll
    for (int r = 0; r < ROWS; ++r)
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float v = acc[r][t];
#pragma unroll
            for (int o = LPR / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
            acc[r][t] = v;
        }
    if (KS > 1) {
        const int slot = (gl * ROWS) * NT, st = GR * G * ROWS * NT;
        if (lane % LPR == 0)
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
#pragma unroll
                for (int t = 0; t < NT; ++t) part[wsub * st + slot + r * NT + t] = acc[r][t];
        __syncthreads();
        if (wsub != 0) return;
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int o = slot + r * NT + t;
                if (KS == 2) acc[r][t] = part[o] + part[st + o];
                else acc[r][t] = (part[o] + part[st + o]) + (part[2 * st + o] + part[3 * st + o]);
            }
    }
    if (lane % LPR != 0) return;
    if (norm)
#pragma unroll
        for (int r = 0; r < ROWS; ++r)
#pragma unroll
            for (int t = 0; t < NT; ++t) acc[r][t] *= inv[t];
    if (p.epi == ORC_EPI_SWIGLU) {
        if (!ok[0]) return;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const float g = acc[0][t], u = acc[1][t];
            yout[0][(size_t)t * p.ldy] = (g / (1.f + expf(-g))) * u;
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        if (!ok[r]) continue;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            float v = acc[r][t];
            if (bias[r]) v += *bias[r];
            float* dst = yout[r] + (size_t)t * p.ldy;
            if (p.epi == ORC_EPI_ACCUM) *dst += v;
            else *dst = v;
        }
    }
}

// ── host-side launch ────────────────────────────────────────────────────────
static int units_per_block(int type) {
    switch (type) {
        case ORC_Q8_0: case ORC_Q4_0: return 1;
        case ORC_Q4_K: return 8;
        case ORC_Q6_K: return 4;
        default: return 0;
    }
}
static int block_elems(int type) { return type == ORC_Q4_K || type == ORC_Q6_K ? 256 : 32; }

constexpr int kRows = 2;
static size_t g_lds_budget = 64 * 1024;  // set from the device limit at first use

static size_t lds_bytes(int type, int nt, int kt, int ks, int lpr) {
    const int PP = (type == ORC_Q4_K || type == ORC_Q6_K) ? 64 : 32;
    const size_t part = (size_t)ks * (4 / ks) * (64 / lpr) * kRows * nt;
    return (size_t)nt * ((kt + 4 * (kt / PP) + 4) + kt / 16) * 4 + (4 * nt + part) * 4;
}

struct GemmShape { int lpr, ks; };

// Lanes per row group (LPR) and waves per group (KS) depend on (type, n_in,
// n_out) only, never on n_tok, so every token sees the same reduction order.
// Narrow matrices get more lanes per row (more workgroups in flight); the
// smallest K tile must fit the LDS budget for kMaxNT tokens.
static GemmShape choose_shape(int type, int units, int n_out) {
    const int el_per_unit = block_elems(type) / units_per_block(type);
    int cap = 64;
    while (cap > 8 && lds_bytes(type, kMaxNT, std::max(1024, cap * el_per_unit), 1, 64) > g_lds_budget) cap /= 2;
    int lt;
    if (n_out >= 12288) lt = units >= 96 ? 32 : units >= 32 ? 16 : 8;  // many rows: 1 wave per group
    else {
        lt = 8;
        while (lt * 2 <= units && lt * 2 <= 64) lt *= 2;  // up to one unit per lane
    }
    lt = std::min(lt, cap);
    GemmShape g;
    if (n_out >= 12288 || lt < 16) { g.ks = 1; g.lpr = std::min(lt, 32); }
    else if (lt == 16) { g.ks = 2; g.lpr = 8; }
    else { g.ks = 4; g.lpr = lt / 4; }
    return g;
}

template <int QT, int NT>
static int launch_nt(const GemmParams& p0, GemmShape sh, hipStream_t s) {
    GemmParams p = p0;
    const int lpr = sh.lpr, ks = sh.ks;
    const int tile = (4 / ks) * (64 / lpr) * kRows;
    const int n_items = p.epi == ORC_EPI_SWIGLU ? p.rows[0] * kRows : p.tile_rows_total;
    const int grid = (n_items + tile - 1) / tile;
    // K tile: the whole row when it fits; otherwise a multiple of lcm(1024, KS*LPR units)
    // so that every lane owns the same units and every thread the same x elements.
    const int be = QTr<QT>::BLK_EL, upb = QTr<QT>::UPB;
    const int type = QT;
    int kt = p.n_in;
    if (lds_bytes(type, NT, kt, ks, lpr) > g_lds_budget) {
        const int step = std::max(1024, ks * lpr / upb * be);
        kt = step;
        while (kt + step < p.n_in && lds_bytes(type, NT, kt + step, ks, lpr) <= g_lds_budget) kt += step;
    }
    p.kt_el = kt;
    p.n_ktiles = (p.n_in + kt - 1) / kt;
    const size_t lds = lds_bytes(type, NT, kt, ks, lpr);
    if (lds > g_lds_budget) return set_error(ORC_E_UNSUPPORTED, "gemm: K tile does not fit LDS");
#define L(LPR_, KS_)                                                                              \
    if (lpr == LPR_ && ks == KS_) {                                                               \
        hipLaunchKernelGGL((k_gemm<QT, NT, LPR_, KS_, kRows>), dim3(grid), dim3(kWG), lds, s, p); \
        ORC_LAUNCH_CHECK();                                                                       \
        return ORC_OK;                                                                            \
    }
    L(8, 1) L(16, 1) L(32, 1) L(8, 2) L(8, 4) L(16, 4)
#undef L
    return set_error(ORC_E_INVALID, "gemm: no kernel for this shape");
}

template <int QT>
static int launch_type(const GemmParams& p, GemmShape sh, hipStream_t s) {
    switch (p.n_tok) {
        case 1: return launch_nt<QT, 1>(p, sh, s);
        case 2: return launch_nt<QT, 2>(p, sh, s);
        case 3: return launch_nt<QT, 3>(p, sh, s);
        case 4: return launch_nt<QT, 4>(p, sh, s);
        case 5: return launch_nt<QT, 5>(p, sh, s);
        default: return set_error(ORC_E_UNSUPPORTED, "n_tok chunk must be 1..5");
    }
}

// ── live kernel timing (orc_prof_*) ─────────────────────────────────────────
struct ProfRec {
    hipEvent_t a, b;
    int type, nt;
    double bytes;
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
static double gemm_bytes(const GemmParams& p, int nt) {
    const int n_w = p.epi == ORC_EPI_SWIGLU ? 2 * p.rows[0] : p.tile_rows_total;
    const int n_y = p.epi == ORC_EPI_SWIGLU ? p.rows[0] : p.tile_rows_total;
    double b = (double)p.row_bytes * n_w + 4.0 * nt * p.n_in + 4.0 * nt * n_y * (p.epi == ORC_EPI_ACCUM ? 2 : 1);
    if (p.norm_w) b += 4.0 * p.n_in;
    for (int i = 0; i < p.n_seg; ++i)
        if (p.bias[i]) b += 4.0 * p.rows[i];
    return b;
}

static int gemm_dispatch(GemmParams p, int type, hipStream_t s) {
    static bool lds_init = false;
    if (!lds_init) {
        int dev = 0, v = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0)
            g_lds_budget = std::min<size_t>((size_t)v, 160 * 1024);
        lds_init = true;
    }
    p.units_per_row = p.n_in / block_elems(type) * units_per_block(type);
    const int n_out = p.epi == ORC_EPI_SWIGLU ? p.rows[0] : p.tile_rows_total;
    const GemmShape sh = choose_shape(type, p.units_per_row, n_out);
    // tokens are processed in chunks of at most kMaxNT; chunking never changes a
    // (token,row) result because the reduction order is independent of n_tok
    for (int t0 = 0; t0 < p.n_tok; t0 += kMaxNT) {
        GemmParams q = p;
        q.n_tok = std::min(kMaxNT, p.n_tok - t0);
        q.x = p.x + (size_t)t0 * p.ldx;
        for (int i = 0; i < 3; ++i) q.y[i] = p.y[i] ? p.y[i] + (size_t)t0 * p.ldy : nullptr;
        ProfRec rec{};
        bool prof = false;
        if (g_prof_on) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            (void)hipStreamIsCapturing(s, &cs);
            if (cs == hipStreamCaptureStatusNone && (rec.a = prof_event()) && (rec.b = prof_event())) {
                prof = hipEventRecord(rec.a, s) == hipSuccess;
                rec.type = type;
                rec.nt = q.n_tok;
                rec.bytes = gemm_bytes(q, q.n_tok);
            }
        }
        int rc;
        switch (type) {
            case ORC_Q4_K: rc = launch_type<ORC_Q4_K>(q, sh, s); break;
            case ORC_Q6_K: rc = launch_type<ORC_Q6_K>(q, sh, s); break;
            case ORC_Q8_0: rc = launch_type<ORC_Q8_0>(q, sh, s); break;
            case ORC_Q4_0: rc = launch_type<ORC_Q4_0>(q, sh, s); break;
            default: return set_error(ORC_E_UNSUPPORTED, "gemm: unsupported weight type " + std::to_string(type));
        }
        if (prof && hipEventRecord(rec.b, s) == hipSuccess) g_prof.push_back(rec);
        if (rc) return rc;
    }
    return ORC_OK;
}

}  // namespace orc

using namespace orc;

extern "C" int orc_prof_enable(int on) {
    g_prof_on = on != 0;
    if (on) {
        g_prof.clear();
        g_evnext = 0;
    }
    return ORC_OK;
}

extern "C" int orc_prof_read(int type, int n_tok, int64_t* launches, double* total_ms, double* total_bytes) {
    int64_t n = 0;
    double ms = 0, by = 0;
    for (const ProfRec& r : g_prof) {
        if ((type >= 0 && r.type != type) || (n_tok > 0 && r.nt != n_tok)) continue;
        ORC_HIP_CHECK(hipEventSynchronize(r.b));
        float e = 0.f;
        ORC_HIP_CHECK(hipEventElapsedTime(&e, r.a, r.b));
        ++n;
        ms += e;
        by += r.bytes;
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
        case ORC_Q4_0: return n % 32 ? -1 : n / 32 * 18;
        case ORC_Q8_0: return n % 32 ? -1 : n / 32 * 34;
        case ORC_Q4_K: return n % 256 ? -1 : n / 256 * 144;
        case ORC_Q6_K: return n % 256 ? -1 : n / 256 * 210;
        default: return -1;
    }
}

static int check_gemm_shape(int type, int n_tok, int n_in, const float* x, int ldx, int ldy, const void* w) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (type != ORC_Q4_K && type != ORC_Q6_K && type != ORC_Q8_0 && type != ORC_Q4_0)
        return set_error(ORC_E_UNSUPPORTED, "gemm: unsupported weight type " + std::to_string(type));
    if (n_tok < 1 || n_in <= 0 || n_in % block_elems(type))
        return set_error(ORC_E_INVALID, "gemm: n_in must be a positive multiple of the block size");
    if (!x || !w || ldx < n_in || ldx % 4 || ldy < 1)
        return set_error(ORC_E_INVALID, "gemm: bad pointers or strides (ldx >= n_in, ldx % 4 == 0)");
    if (((uintptr_t)x & 15) != 0) return set_error(ORC_E_INVALID, "gemm: x must be 16-byte aligned");
    return ORC_OK;
}

extern "C" int orc_gemm(int type, const void* d_w, int n_tok, int n_out, int n_in, const float* d_x, int ldx,
                        float* d_y, int ldy, orc_stream_t stream) {
    if (int rc = check_gemm_shape(type, n_tok, n_in, d_x, ldx, ldy, d_w)) return rc;
    if (n_out <= 0 || !d_y || (n_tok > 1 && ldy < n_out)) return set_error(ORC_E_INVALID, "gemm: bad output");
    GemmParams p{};
    p.w[0] = (const uint8_t*)d_w;
    p.y[0] = d_y;
    p.rows[0] = n_out;
    p.n_seg = 1;
    p.tile_rows_total = n_out;
    p.n_in = n_in;
    p.row_bytes = (uint64_t)orc_row_bytes(type, n_in);
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
    GemmParams p{};
    int total = 0;
    for (int i = 0; i < n_segs; ++i) {
        if (!segs[i].d_w || !segs[i].d_y || segs[i].n_out <= 0) return set_error(ORC_E_INVALID, "gemm_fused: bad segment");
        p.w[i] = (const uint8_t*)segs[i].d_w;
        p.y[i] = segs[i].d_y;
        p.bias[i] = segs[i].d_bias;
        p.rows[i] = segs[i].n_out;
        total += segs[i].n_out;
    }
    p.n_seg = n_segs;
    p.tile_rows_total = total;
    p.n_in = n_in;
    p.row_bytes = (uint64_t)orc_row_bytes(type, n_in);
    p.x = d_x;
    p.ldx = ldx;
    p.ldy = ldy;
    p.n_tok = n_tok;
    p.norm_w = d_norm_w;
    p.eps = eps;
    p.epi = epilogue;
    return gemm_dispatch(p, type, resolve_stream(stream));
}


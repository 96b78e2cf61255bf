// Quantized GEMM / GEMV on the matrix cores for Q4_K and Q6_K blocks (gfx950).
//
// Replaces gemv_q / gemv_q_range / gemm_q (core/gguf_parser.cpp:868-997) for
// the K-quant types of a Q4_K_M / Q6_K model, with the RMSNorm prologue and
// the bias / residual / SwiGLU epilogues of Model::forward / forward_prefill
// (core/model.cpp:366-473, 565-643) fused in.
//
// Numerics. Activations are the MFMA's A operand, weights the B operand (16
// weight rows of a tile), so D[A row][weight row] lands with one weight row
// per lane: lane l holds D[4 (l/16) + e][l % 16]. Each activation x' (x
// times the norm weight times a power of two per (unit, token) that keeps
// it below 2^14) is split as hi = fp16(x'), lo = fp16(x' - hi); hi + lo
// carries ~22 bits and every product with a weight code is exact in fp32.
// Up to 8 tokens, A row t holds token t's hi halves and row 8 + t its lo
// halves: one MFMA takes both and the two rows' sums are added once per tile
// (lanes l and l + 32). 9 to 16 tokens use two A tiles (all tokens' hi
// halves, all tokens' lo halves) against the same B: every (token, row) sum
// is formed by the same operations in the same order either way. A unit is
// 128 consecutive values of a row, in four 32-value slices of one
// v_mfma_f32_16x16x32_f16 each; lane group c (lanes 16c .. 16c + 15) holds
// values 8c .. 8c + 7 of a slice for its row (B) or token (A).
//  * Q4_K: a slice is one sub-block. Low-nibble codes become fp16 1024 + q
//    (one v_and_or_b32 per two codes), high-nibble codes 1024 + 16 q without
//    a shift (the nibble already sits at mantissa bits 4-7); one packed FMA
//    per two codes folds the 6-bit scale: (1024 + q) sc - 1024 sc and
//    (1024 + 16 q) sc / 16 - 64 sc are sc q, exact in fp16 (<= 945). d scales
//    the unit's chain; the minimum term dmin m sum(x g) of the unit's four
//    sub-blocks is one 16x16x4 fp32 MFMA per tile.
//  * Q6_K: a slice spans two 16-value sub-blocks whose int8 scales do not fit
//    the code exactly (sc (q - 32) up to 4096), so the scaled code is split
//    into hi = fp16(sc (q - 32)) and lo = sc (q - 32) - hi (exact, |lo| <= 1):
//    one MFMA per code half and slice.
// Products are exact in fp32; results are within a few 1e-6 of the float64
// dot product.
//
// Structure. One 1024-thread workgroup per CU (16 waves, four per SIMD, at
// most 128 VGPRs each). Its waves first stage the activations of all
// tokens: each 16-lane row converts one (unit, token) item (128 values) to
// the A layout with its power of two, the item's sum of x^2 (for the norm)
// and, for Q4_K, its per-sub-block sums of x g. A tile-group is TR tiles of
// 16 rows (a SwiGLU launch pairs gate tile i with up tile i); KS waves split
// a tile-group's units into fixed contiguous ranges, so a round computes
// 16 / KS tile-groups at once. A wave loads its range of units in batches
// of UW whose loads all go out before the batch's arithmetic (the first
// batch before the activations are staged); after each round the waves'
// partial sums meet in the LDS and are added in wave order
// (double-buffered, one barrier per round). The
// staging of a (unit, token), the K split of a shape and every reduction
// order depend on the shape only, never on the token count, so a (token,
// row) result is bit-identical for every token count: a (k+1)-token verify
// equals k+1 decode GEMVs.
//  * FULL mode: every unit of a row is staged once by all waves, one barrier.
//  * Windowed mode (rows too long for the LDS, KS = 16): each wave stages
//    only the units of its own range, a window at a time, and reads only what
//    it wrote; the windows are restaged for each round.
#include "orc_gemm.hpp"

#include <algorithm>

namespace orc {

typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));

constexpr int kWG = 1024, kWv = kWG / 64;  // threads, waves per workgroup
template <int NT> constexpr bool wide() { return NT > 8; }
template <int NT> constexpr int ntp() { return (NT + 3) & ~3; }

// code permutation of one 8-value run (bytes 0,2 / 1,3 / 4,6 / 5,7 land in
// consecutive halves when two dwords are unpacked into fp16 pairs)
__device__ __forceinline__ int perm8(int j) { return (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1); }

// Byte offset of A entry (slice i, lane group c, half hl, token t) in a unit
// (16 bytes: 8 halves); a unit holds 512 NT bytes.
template <int NT> __device__ __forceinline__ int a_off(int i, int c, int hl, int t) {
    return (((i * 4 + c) * 2 + hl) * NT + t) * 16;
}

// Loads through the global address space (a generic pointer would make
// them flat loads, which LDS waits also have to drain).
typedef const __attribute__((address_space(1))) u32x2_u* g8p;
typedef const __attribute__((address_space(1))) u32x4_u* g16p;
typedef const __attribute__((address_space(1))) u16_u* g2p;
__device__ __forceinline__ u32x4 ldg16(const uint8_t* p) { return *(g16p)p; }
__device__ __forceinline__ u32x2 ldg8(const uint8_t* p) { return *(g8p)p; }
__device__ __forceinline__ uint32_t ldg2(const uint8_t* p) { return *(g2p)p; }

// Constants in registers: a VOP3 operation such as v_and_or_b32 takes no
// literal, so (x & mask) | magic is one operation only with both in registers.
__device__ __forceinline__ uint32_t sreg(uint32_t c) {
    uint32_t r;
    asm("s_mov_b32 %0, %1" : "=s"(r) : "n"(c));
    return r;
}
__device__ __forceinline__ uint32_t vreg(uint32_t c) {
    uint32_t r;
    asm("v_mov_b32 %0, %1" : "=v"(r) : "n"(c));
    return r;
}

__device__ __forceinline__ h2v as_h2(uint32_t v) { return __builtin_bit_cast(h2v, v); }
__device__ __forceinline__ uint32_t as_u32(h2v v) { return __builtin_bit_cast(uint32_t, v); }

// Segment pointers held in scalar registers (readfirstlane), so that a
// lane-dependent choice between them stays a register select.
template <class T> __device__ __forceinline__ T* spin(T* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T*)(((uint64_t)hi << 32) | lo);
}

// DPP reductions inside one 16-lane row in a fixed order: the quad, then the
// half-row and row mirrors.
__device__ __forceinline__ float row_sum(float v) {
    v = quad_sum(v);
    v += dpp<0x141>(v);  // row_half_mirror
    v += dpp<0x140>(v);  // row_mirror
    return v;
}
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp<0xB1>(v));
    v = fmaxf(v, dpp<0x4E>(v));
    v = fmaxf(v, dpp<0x141>(v));
    v = fmaxf(v, dpp<0x140>(v));
    return v;
}

// Q4_K 6-bit scales and minimums of sub-blocks 4h .. 4h + 3 (h = 0, 1), one
// per byte of sc4 / mn4, from the 12 scale bytes s0 | s1 | s2
// (core/gguf_parser.cpp:1085-1093); branch-free, h selects by mask.
__device__ __forceinline__ void q4k_unit_sm(int h, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc4,
                                            uint32_t& mn4) {
    const uint32_t sc_lo = s0 & 0x3F3F3F3Fu, mn_lo = s1 & 0x3F3F3F3Fu;
    const uint32_t sc_hi = (s2 & 0x0F0F0F0Fu) | ((s0 >> 2) & 0x30303030u);
    const uint32_t mn_hi = ((s2 >> 4) & 0x0F0F0F0Fu) | ((s1 >> 2) & 0x30303030u);
    const uint32_t msk = 0u - (uint32_t)(h & 1);
    sc4 = sc_lo ^ ((sc_lo ^ sc_hi) & msk);
    mn4 = mn_lo ^ ((mn_lo ^ mn_hi) & msk);
}

// Loaded bytes of one unit of one row for lane group c.
//  Q4_K (core/gguf_parser.cpp:1096-1121): a, b = d, dmin and the 12 scale
//    bytes; c, d = code bytes 8c.. of the unit's first 32 (slices 0, 1: low,
//    high nibbles) and of its next 32 (slices 2, 3).
//  Q6_K (core/gguf_parser.cpp:1124-1154): a, b = low 4 bits of slices 0, 2
//    (ql bytes 8c..) and 1, 3 (ql bytes 32 + 8c..); c = high 2 bits (qh
//    bytes 8c.., bits 2i of slice i); d = the half's 8 int8 scales; e = d.
struct MUnit {
    u32x2 a, b, c, d;
    uint32_t e;
    __device__ __forceinline__ void load(int type, const uint8_t* row, int u, int cg) {
        if (type == ORC_Q4_K) {
            const uint8_t* blk = row + (size_t)(u >> 1) * 144;
            const u32x4 hdr = ldg16(blk);
            a = u32x2{hdr.x, hdr.y};
            b = u32x2{hdr.z, hdr.w};
            const uint8_t* qs = blk + 16 + 64 * (u & 1) + 8 * cg;
            c = ldg8(qs);
            d = ldg8(qs + 32);
        } else {
            const uint8_t* blk = row + (size_t)(u >> 1) * 210;
            const int hh = u & 1;
            a = ldg8(blk + 64 * hh + 8 * cg);
            b = ldg8(blk + 64 * hh + 32 + 8 * cg);
            c = ldg8(blk + 128 + 32 * hh + 8 * cg);
            d = ldg8(blk + 192 + 8 * hh);
            e = ldg2(blk + 208);
        }
    }
};

// Where a unit's activations live in LDS.
struct MCtx {
    const uint8_t* abase;  // A entries, one unit after another
    const float* sx;       // Q4_K: sums of x g over each 32-value sub-block, [token][sub-block]
    int sx_stride;
    const float* esc;      // 2^-e of each (unit, token), [unit][NTP]
};

// The lane's A entries of the unit in LDS slot ua (all four slices; lane row
// r = lane % 16) and the 2^-e of the tokens of its D rows. Up to 8 tokens:
// row r is the hi half of token r or the lo half of token r - 8, D rows are
// tokens 4 (c % 2) + e. 9 to 16 tokens: a holds the hi and al the lo half of
// token r, D rows are tokens 4 c + e. Rows of tokens past n_tok read
// whatever the neighbouring entries hold (always inside the allocation: the
// A region is padded): an MFMA's D row depends only on the same A row, and
// every epilogue drops rows of tokens >= n_tok.
template <int NT>
__device__ __forceinline__ void a_load(int u, int ua, int lane, const MCtx& m, h8v (&a)[4], h8v (&al)[4], float4& es) {
    constexpr bool W = wide<NT>();
    const int c = lane >> 4, r = lane & 15, t = W ? r : r & 7, tb = W ? 4 * c : 4 * (c & 1);
    const uint8_t* ap = m.abase + (size_t)ua * 512 * NT + a_off<NT>(0, c, W ? 0 : r >> 3, t);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = __builtin_bit_cast(h8v, *(const u32x4*)(ap + a_off<NT>(i, 0, 0, 0)));
        if constexpr (W) al[i] = __builtin_bit_cast(h8v, *(const u32x4*)(ap + a_off<NT>(i, 0, 1, 0)));
    }
    es = *(const float4*)(m.esc + u * ntp<NT>() + tb);
}

// D entries e of a lane that can hold a token below n_tok: below 4 tokens
// entries e >= n_tok belong to no token and are not scaled.
template <int NT> constexpr int kDRows = (!wide<NT>() && NT < 4) ? NT : 4;

// Q4_K unit of TR tiles with the lane's A entries given; acc += d 2^-e D
// minus, on the hi rows only, the sum over the unit's sub-blocks of
// dmin m sum(x g) (one 16x16x4 fp32 MFMA per tile).
template <int NT, int TR>
__device__ __forceinline__ void core_q4k(const MUnit (&M)[TR], int u, int lane, const MCtx& m, const h8v (&a)[4],
                                         const h8v (&al)[4], float4 es, f4v (&acc)[TR], f4v (&acl)[TR]) {
    constexpr bool W = wide<NT>();
    const int c = lane >> 4, h = u & 1, r = lane & 15;
    // A of the minimum term: lane (c, r) holds token r's sum of x g over
    // sub-block 4u + c; zero on the lo rows of stacked launches and past the
    // last token
    constexpr int NA = W ? NT : (NT < 8 ? NT : 8);
    const float sxa = r < NA ? m.sx[r * m.sx_stride + 4 * u + c] : 0.f;
    const float esv[4] = {es.x, es.y, es.z, es.w};
    const uint32_t G = vreg(0x64006400u), M8 = sreg(0x00FF00FFu), ML = sreg(0x000F000Fu), MH = sreg(0x00F000F0u);
#pragma unroll
    for (int tr = 0; tr < TR; ++tr) {
        uint32_t sc4, mn4;
        q4k_unit_sm(h, M[tr].a.y, M[tr].b.x, M[tr].b.y, sc4, mn4);
        // fp16 scales: (sc0, sc2) for the low-nibble slices 0, 2 and
        // (sc1 / 16, sc3 / 16) for the high-nibble slices 1, 3 (exact), and
        // the offsets that remove 1024 x scale
        const h2v k1024{(_Float16)-1024.f, (_Float16)-1024.f};
        const h2v s02 = as_h2((sc4 & M8) | G) + k1024;
        const h2v s13 = (as_h2(((sc4 >> 8) & M8) | G) + k1024) * h2v{(_Float16)0.0625f, (_Float16)0.0625f};
        const h2v o02 = s02 * k1024, o13 = s13 * k1024;
        const float dmin = h2f(M[tr].a.x >> 16);
        const float bm = -(dmin * (float)((mn4 >> (8 * c)) & 0xFFu));
        f4v D = f4v{0.f, 0.f, 0.f, 0.f}, Dl = D;  // even and odd slices in independent chains
        f4v E = D, El = D;                         // the same for the lo tile (9-16 tokens)
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            const u32x2 src = half ? M[tr].d : M[tr].c;
            const uint32_t x8 = src.x >> 8, y8 = src.y >> 8;
            const _Float16 sl = half ? s02.y : s02.x, ol = half ? o02.y : o02.x;
            const _Float16 sh = half ? s13.y : s13.x, oh = half ? o13.y : o13.x;
            u32x4 bl, bh;
            const uint32_t wl[4] = {(src.x & ML) | G, (x8 & ML) | G, (src.y & ML) | G, (y8 & ML) | G};
            const uint32_t wh[4] = {(src.x & MH) | G, (x8 & MH) | G, (src.y & MH) | G, (y8 & MH) | G};
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                bl[k] = as_u32(__builtin_elementwise_fma(as_h2(wl[k]), h2v{sl, sl}, h2v{ol, ol}));
                bh[k] = as_u32(__builtin_elementwise_fma(as_h2(wh[k]), h2v{sh, sh}, h2v{oh, oh}));
            }
            const h8v blo = __builtin_bit_cast(h8v, bl), bhi = __builtin_bit_cast(h8v, bh);
            D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2 * half], blo, D, 0, 0, 0);
            Dl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[2 * half + 1], bhi, Dl, 0, 0, 0);
            if constexpr (W) {
                E = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[2 * half], blo, E, 0, 0, 0);
                El = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[2 * half + 1], bhi, El, 0, 0, 0);
            }
        }
        const float d = h2f(M[tr].a.x & 0xFFFFu);
        f4v t = acc[tr];
#pragma unroll
        for (int e = 0; e < kDRows<NT>; ++e) {
            const float de = d * esv[e];
            t[e] = __builtin_fmaf(de, D[e], __builtin_fmaf(de, Dl[e], t[e]));
            if constexpr (W) acl[tr][e] = __builtin_fmaf(de, E[e], __builtin_fmaf(de, El[e], acl[tr][e]));
        }
        acc[tr] = __builtin_amdgcn_mfma_f32_16x16x4f32(sxa, bm, t, 0, 0, 0);
    }
}

// Q6_K unit of TR tiles with the lane's A entries given: scale-folded hi /
// lo codes in two chains, acc += d 2^-e D.
template <int NT, int TR>
__device__ __forceinline__ void core_q6k(const MUnit (&M)[TR], int lane, const h8v (&a)[4], const h8v (&al)[4],
                                         float4 es, f4v (&acc)[TR], f4v (&acl)[TR]) {
    constexpr bool W = wide<NT>();
    const int c = lane >> 4;
    const float esv[4] = {es.x, es.y, es.z, es.w};
    const uint32_t G = vreg(0x64006400u), M8 = sreg(0x00FF00FFu);
#pragma unroll
    for (int tr = 0; tr < TR; ++tr) {
        f4v D = f4v{0.f, 0.f, 0.f, 0.f}, Dl = D;  // hi and lo code halves in independent chains
        f4v E = D, El = D;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // 6-bit codes of the lane's 8 values of slice i (stored + 32)
            const u32x2 src = (i & 1) ? M[tr].b : M[tr].a;
            const int sh = 4 * (i >> 1);
            const uint32_t q0 = ((src.x >> sh) & 0x0F0F0F0Fu) | (((M[tr].c.x >> (2 * i)) & 0x03030303u) << 4);
            const uint32_t q1 = ((src.y >> sh) & 0x0F0F0F0Fu) | (((M[tr].c.y >> (2 * i)) & 0x03030303u) << 4);
            // scale of the lane's 16-value sub-block 2i + c/2
            const int si = 2 * i + (c >> 1);
            const uint32_t sw = si < 4 ? M[tr].d.x : M[tr].d.y;
            const _Float16 sf = (_Float16)(float)(int8_t)((sw >> (8 * (si & 3))) & 0xFFu);
            const h2v sc2{sf, sf}, off{(_Float16)-1056.f, (_Float16)-1056.f};  // 1024 + 32
            const uint32_t r[4] = {(q0 & M8) | G, ((q0 >> 8) & M8) | G, (q1 & M8) | G, ((q1 >> 8) & M8) | G};
            u32x4 bh, bl;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const h2v v = as_h2(r[k]) + off;  // q - 32, exact
                const h2v hi = v * sc2;
                bh[k] = as_u32(hi);
                bl[k] = as_u32(__builtin_elementwise_fma(v, sc2, -hi));  // exact remainder
            }
            const h8v bhi = __builtin_bit_cast(h8v, bh), blo = __builtin_bit_cast(h8v, bl);
            D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], bhi, D, 0, 0, 0);
            Dl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], blo, Dl, 0, 0, 0);
            if constexpr (W) {
                E = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], bhi, E, 0, 0, 0);
                El = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], blo, El, 0, 0, 0);
            }
        }
        const float d = h2f(M[tr].e);
#pragma unroll
        for (int e = 0; e < kDRows<NT>; ++e) {
            const float de = d * esv[e];
            acc[tr][e] = __builtin_fmaf(de, D[e], __builtin_fmaf(de, Dl[e], acc[tr][e]));
            if constexpr (W) acl[tr][e] = __builtin_fmaf(de, E[e], __builtin_fmaf(de, El[e], acl[tr][e]));
        }
    }
}

// Row -> segment by comparisons over values passed by value (scalar
// registers), so a lane-dependent choice stays a register select.
__device__ __forceinline__ int seg_of(int j, int n_seg, int r0, int r1, int& jj) {
    const bool s1 = n_seg > 1 && j >= r0;
    const bool s2 = n_seg > 2 && j >= r0 + r1;
    jj = s2 ? j - r0 - r1 : (s1 ? j - r0 : j);
    return s2 ? 2 : (s1 ? 1 : 0);
}
template <class T> __device__ __forceinline__ T* pick3(int s, T* a, T* b, T* c) { return s == 2 ? c : (s == 1 ? b : a); }

// LDS layout of a launch (bytes), shared by the kernel and the host.
struct MLayout {
    int a_bytes, esc, sx, ssu, part, total;
};
__host__ __device__ inline MLayout mlayout(bool sx_sums, int nt, int U, int slots, int tr) {
    MLayout L;
    const int ntp4 = (nt + 3) & ~3;
    L.a_bytes = slots * 512 * nt + 256;                 // A entries (+ room for the unmasked reads past the end)
    L.esc = L.a_bytes;                                  // [U][ntp4] + 8 floats of slack
    L.sx = L.esc + (U * ntp4 + 8) * 4;                  // [nt][4 U]
    L.ssu = L.sx + (sx_sums ? nt * 4 * U * 4 : 0);      // [U][nt] sums of x^2
    L.part = L.ssu + U * nt * 4;                        // [2][16 waves][tr][nt][16]
    L.total = L.part + 2 * kWv * tr * nt * 16 * 4;
    return L;
}

// Stages the (unit, token) items [i0, i1) (item it = unit it / NT, token
// it % NT): 16-lane row `row` of the nrows taking part handles items
// i0 + row, i0 + row + nrows, ...: x (times the norm weight) in the A layout
// of LDS slot (unit - slot_base), its 2^-e, its sum of x^2 and (Q4_K) its
// per-sub-block sums of x g. Whatever the row, an item's values are formed
// by the same operations. B items per row are loaded before the first is
// converted. after_first() runs once the first batch's loads are issued
// (the weight ring then queues behind them, not before).
template <int NT, bool SX, int B, class F>
__device__ __forceinline__ void stage_items(const QmvParams& p, int i0, int i1, int row, int row_base, int nrows,
                                            int slot_base, uint8_t* abase, float* esc, float* sx, int sx_stride,
                                            float* ssu, int r16, F after_first) {
    constexpr int NTP = ntp<NT>();
    const bool norm = p.norm_w != nullptr;
    bool first = true;
    // the pass bound uses the wave's first row (row_base), so every lane of a
    // wave runs the same passes; a row's items past i1 load item i0 and store nothing
    if (i0 + row_base >= i1) after_first();
    for (int pb = i0 + row_base; pb < i1; pb += B * nrows) {
        const int ib = pb + (row - row_base);
        float v[B][8], g[B][8];
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const int it = ib + k * nrows;
            const int itc = it < i1 ? it : i0;
            const int u = itc / NT, t = itc % NT;
            // tokens past n_tok (a launch rounded up to NT) stage zeros: the
            // load reads token 0 (always valid) and the value is dropped
            const bool tin = t < p.n_tok;
            const float* src = p.x + (size_t)(tin ? t : 0) * p.ldx + 128 * u + 8 * r16;
            const float4 x0 = *(const float4*)src, x1 = *(const float4*)(src + 4);
            const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
            *(float4*)v[k] = tin ? x0 : z4;
            *(float4*)(v[k] + 4) = tin ? x1 : z4;
            const float* gp = (norm ? p.norm_w : p.x) + 128 * u + 8 * r16;
            *(float4*)g[k] = *(const float4*)gp;
            *(float4*)(g[k] + 4) = *(const float4*)(gp + 4);
        }
        if (first) {
            after_first();
            first = false;
        }
#pragma unroll
        for (int k = 0; k < B; ++k) {
            const int it = ib + k * nrows;
            const bool valid = it < i1;
            const int itc = valid ? it : i0;
            const int u = itc / NT, t = itc % NT;
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(v[k][e], v[k][e], ss);
            if (norm) {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[k][e] *= g[k][e];
            }
            float mx = 0.f;
#pragma unroll
            for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[k][e]));
            mx = row_max(mx);
            ss = row_sum(ss);
            int e2 = 0;
            if (mx > 0.f && mx <= 3.0e38f) {
                int ex;
                (void)frexpf(mx, &ex);  // mx < 2^ex
                e2 = 14 - ex;
            }
            float s8 = ((v[k][0] + v[k][1]) + (v[k][2] + v[k][3])) + ((v[k][4] + v[k][5]) + (v[k][6] + v[k][7]));
            if constexpr (SX) s8 = quad_sum(s8);
            if (!valid) continue;
            const float up = ldexpf(1.f, e2);
            h8v hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float w = v[k][e] * up;
                const _Float16 he = (_Float16)w;
                hi[perm8(e)] = he;
                lo[perm8(e)] = (_Float16)(w - (float)he);
            }
            uint8_t* ap = abase + (size_t)(u - slot_base) * 512 * NT;
            const int i = r16 >> 2, cc = r16 & 3;
            *(h8v*)(ap + a_off<NT>(i, cc, 0, t)) = hi;
            *(h8v*)(ap + a_off<NT>(i, cc, 1, t)) = lo;
            if (r16 == 0) {
                esc[u * NTP + t] = ldexpf(1.f, -e2);
                ssu[u * NT + t] = ss;
            }
            if (SX && (r16 & 3) == 0) sx[t * sx_stride + 4 * u + (r16 >> 2)] = s8;
        }
    }
}

// QT: ORC_Q4_K, ORC_Q6_K or kMixK; NT tokens; TR tiles per tile-group; KS
// waves per tile-group; UW units of weight loads in flight per wave; FULL:
// every unit staged once (else KS = 16 and windows of p.hs units).
template <int QT, int NT, int TR, int KS, int UW, bool FULL>
__global__ __launch_bounds__(kWG) void k_mmq(QmvParams p) {
    static_assert(FULL || KS == kWv, "windowed staging needs one tile-group per round");
    constexpr bool MIX = QT == kMixK;
    constexpr bool SX = QT == ORC_Q4_K || MIX;
    constexpr bool W = wide<NT>();
    constexpr int G = kWv / KS;  // tile-groups per round
    constexpr int SB = TR == 2 ? 1 : 2;  // staged items per lane row loaded at once
    extern __shared__ __attribute__((aligned(16))) uint8_t msm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane >> 4, n = lane & 15;
    const int kn = p.n_in, U = kn / 128;
    const int slot = wave / KS, kp = wave % KS;
    const int u0 = kp * U / KS, u1 = (kp + 1) * U / KS;  // this wave's unit range
    const int HS = FULL ? U : p.hs;                     // units held in LDS at once per wave (windowed)
    const MLayout L = mlayout(SX, NT, U, FULL ? U : kWv * HS, TR);
    uint8_t* abase = msm;
    float* esc = (float*)(msm + L.esc);
    float* sx = (float*)(msm + L.sx);
    float* ssu = (float*)(msm + L.ssu);
    float* part = (float*)(msm + L.part);
    const int sx_stride = 4 * U;
    // windowed: this wave's LDS slots start at wave * HS; a window starting at
    // unit wb sits at slots wave * HS + (u - wb)
    const MCtx mc{abase, sx, sx_stride, esc};

    const uint8_t *const sw0 = spin(p.w[0]), *const sw1 = spin(p.w[1]), *const sw2 = spin(p.w[2]);
    float *const sy0 = spin(p.y[0]), *const sy1 = spin(p.y[1]), *const sy2 = spin(p.y[2]);
    const float *const sb0 = spin(p.bias[0]), *const sb1 = spin(p.bias[1]), *const sb2 = spin(p.bias[2]);
    const int n_seg = p.n_seg, r0 = p.rows[0], r1 = p.rows[1];
    const uint32_t tys = (uint32_t)p.seg_type[0] | ((uint32_t)p.seg_type[1] << 8) | ((uint32_t)p.seg_type[2] << 16);
    auto seg_type = [=](int sgi) { return MIX ? (int)((tys >> (8 * sgi)) & 0xFFu) : QT; };
    const uint64_t rb_q4k = (uint64_t)(kn / 256) * 144, rb_q6k = (uint64_t)(kn / 256) * 210;
    auto wrow = [=](int jl) {  // weight row of logical row jl (row 0 past the end: loads stay in bounds)
        int jj;
        const int sgi = seg_of(jl < p.n_rows ? jl : 0, n_seg, r0, r1, jj);
        const uint64_t rb = MIX ? (seg_type(sgi) == ORC_Q4_K ? rb_q4k : rb_q6k) : p.row_bytes;
        return pick3(sgi, sw0, sw1, sw2) + (size_t)jj * rb;
    };
    auto orow = [=](int jl, float*& y, const float*& bias) {  // output of logical row jl; false past the end
        if (jl >= p.n_rows) return false;
        int jj;
        const int sgi = seg_of(jl, n_seg, r0, r1, jj);
        y = pick3(sgi, sy0, sy1, sy2) + jj;
        const float* bb = pick3(sgi, sb0, sb1, sb2);
        bias = bb ? bb + jj : nullptr;
        return true;
    };
    const bool swiglu = p.epi == ORC_EPI_SWIGLU;
    const int rows_out = swiglu ? r0 : p.n_rows;
    const int n_tg = swiglu ? (rows_out + 15) / 16 : (rows_out + 16 * TR - 1) / (16 * TR);
    auto tg_type = [=](int tg) {  // a tile-group's weight type (mixed launches: whole tiles per segment)
        int jj;
        return seg_type(seg_of(tg < n_tg ? tg * 16 * TR : 0, n_seg, r0, r1, jj));
    };
    auto tg_rows = [&](int tg, const uint8_t* (&rp)[TR]) {
        const int tgc = tg < n_tg ? tg : 0;
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) {
            const int jl = swiglu ? tr * r0 + (tgc * 16 + n < r0 ? tgc * 16 + n : r0 - 1) : (tgc * TR + tr) * 16 + n;
            rp[tr] = wrow(jl);
        }
    };

    // rounds: every wave of the workgroup runs the same number (barriers)
    const int tg_first = blockIdx.x * G, tg_stride = gridDim.x * G;
    const int rounds = tg_first < n_tg ? (n_tg - tg_first + tg_stride - 1) / tg_stride : 0;

    // Weight loads in batches of UW units: each batch is issued as one group
    // of loads and computed in the same loop step, so no load registers are
    // carried across iterations and each wait before a unit's arithmetic
    // counts exactly the loads issued after its own. Slots past the wave's
    // range (in its last batch) load a valid unit and consume it without
    // arithmetic. With every unit staged at once, round 0's first batch goes
    // out before the activations are staged.
    const int nu = u1 - u0;
    const int nb = (nu + UW - 1) / UW;
    const int u_ph = u0 < U ? u0 : U - 1;  // unit a padding slot loads
    MUnit buf[UW][TR];
    const uint8_t* rp[TR];  // rows of the current round's tile-group
    int tg = tg_first + slot;
    int tt = tg_type(tg);
    tg_rows(tg, rp);
    auto issue = [&](const uint8_t* const (&rows)[TR], int type, int b) {
#pragma unroll
        for (int k = 0; k < UW; ++k) {
            const int uo = b * UW + k;
#pragma unroll
            for (int tr = 0; tr < TR; ++tr) buf[k][tr].load(type, rows[tr], uo < nu ? u0 + uo : u_ph, c);
        }
    };

    // ── staging ──
    const int r16 = lane & 15, row_in_wave = lane >> 4;
    if constexpr (FULL) {
        // every (unit, token) item once, by all 64 rows of the workgroup; the
        // first weight batch goes out once the first batch of x loads has
        stage_items<NT, SX, SB>(p, 0, U * NT, wave * 4 + row_in_wave, wave * 4, kWv * 4, 0, abase, esc, sx, sx_stride,
                                ssu, r16, [&] { issue(rp, tt, 0); });
        __syncthreads();
    }

    auto inv_rms = [&](int tok) {
        if (!p.norm_w) return 1.f;
        float s = 0.f;
        for (int u = 0; u < U; ++u) s += ssu[u * NT + tok];
        return 1.f / sqrtf(s / (float)kn + p.eps);
    };

    // the wave's window of its range (windowed mode): units [wb, wb + HS) at
    // LDS slots wave * HS + (u - wb)
    auto wave_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    auto stage_window = [&](int wb) {
        const int we = min(u1, wb + HS);
        stage_items<NT, SX, SB>(p, wb * NT, we * NT, row_in_wave, 0, 4, wb - wave * HS, abase, esc, sx, sx_stride,
                                ssu, r16, [] {});
    };

    // one round: tile-group tg with rows rp. FIRST: round 0, whose first
    // batch (FULL mode) went out before the staging
    auto round_body = [&](auto first_tag, int rd) {
        constexpr bool FIRST = decltype(first_tag)::value;
        f4v acc[TR], acl[TR];
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) acc[tr] = acl[tr] = f4v{0.f, 0.f, 0.f, 0.f};
        int wb = u0;
        if constexpr (!FULL) {
            // the first window of this wave's own range (every round: the
            // previous round's last window may have replaced it)
            if (nu > 0) stage_window(wb);
            wave_sync();
        }
        auto consume = [&](int b) {
#pragma unroll
            for (int k = 0; k < UW; ++k) {
                const int uo = b * UW + k;
                if (uo < nu) {
                    const int u = u0 + uo;
                    int ua = u;
                    if constexpr (!FULL) {
                        if (u >= wb + HS) {  // the range's next window
                            wave_sync();
                            wb += HS;
                            stage_window(wb);
                            wave_sync();
                        }
                        ua = wave * HS + (u - wb);
                    }
                    h8v a[4], al[4];
                    float4 es;
                    a_load<NT>(u, ua, lane, mc, a, al, es);
                    if (MIX ? tt == ORC_Q4_K : QT == ORC_Q4_K)
                        core_q4k<NT, TR>(buf[k], u, lane, mc, a, al, es, acc, acl);
                    else
                        core_q6k<NT, TR>(buf[k], lane, a, al, es, acc, acl);
                } else {
                    // a padding slot: its loads are consumed here without arithmetic
#pragma unroll
                    for (int tr = 0; tr < TR; ++tr)
                        asm volatile("" ::"v"(buf[k][tr].a), "v"(buf[k][tr].b), "v"(buf[k][tr].c),
                                     "v"(buf[k][tr].d), "v"(buf[k][tr].e));
                }
            }
        };
        int b = 0;
        if constexpr (FIRST && FULL) {
            consume(0);
            b = 1;
        }
        for (; b < nb; ++b) {
            issue(rp, tt, b);
            consume(b);
        }
        // hi + lo: lanes 0..31 hold tokens 4 (c % 2) + e (stacked), all
        // lanes tokens 4 c + e (wide)
        if constexpr (W) {
#pragma unroll
            for (int tr = 0; tr < TR; ++tr)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[tr][e] += acl[tr][e];
        } else {
#pragma unroll
            for (int tr = 0; tr < TR; ++tr)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[tr][e] += __shfl_xor(acc[tr][e], 32, 64);
        }
        const int this_tg = tg;
        const int tok_lanes = W ? 4 : 2;  // lane groups holding tokens
        if constexpr (KS == 1) {
            // whole rows in one wave: the lane's outputs (token 4c + e, row n) directly
            if (this_tg < n_tg && c < tok_lanes) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int tok = 4 * c + e;
                    if (tok >= NT || tok >= p.n_tok) continue;
                    const float inv = inv_rms(tok);
                    if (swiglu) {
                        const int j = this_tg * 16 + n;
                        if (j < r0) {
                            const float gv = acc[0][e] * inv, uv = acc[TR - 1][e] * inv;
                            sy0[j + (size_t)tok * p.ldy] = (gv / (1.f + expf(-gv))) * uv;
                        }
                    } else {
#pragma unroll
                        for (int tr = 0; tr < TR; ++tr) {
                            float* y;
                            const float* bias;
                            if (orow((this_tg * TR + tr) * 16 + n, y, bias)) {
                                float v = acc[tr][e] * inv;
                                if (bias) v += *bias;
                                float* dst = y + (size_t)tok * p.ldy;
                                if (p.epi == ORC_EPI_ACCUM) *dst += v;
                                else *dst = v;
                            }
                        }
                    }
                }
            }
            return;
        }
        // partial sums of this wave's units: part[buf][wave][tr][token][row]
        float* pb = part + (size_t)(rd & 1) * kWv * TR * NT * 16;
        if (c < tok_lanes) {
#pragma unroll
            for (int tr = 0; tr < TR; ++tr)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int tok = 4 * c + e;
                    if (tok < NT) pb[((wave * TR + tr) * NT + tok) * 16 + n] = acc[tr][e];
                }
        }
        __syncthreads();
        // wave-ordered sums and the epilogue: one thread per (tile-group slot, tile, token, row)
        const int outs = G * TR * NT * 16;
        for (int o = tid; o < outs; o += kWG) {
            const int r = o & 15, tok = (o >> 4) % NT, tr = (o / (16 * NT)) % TR, sl = o / (16 * NT * TR);
            const int tgo = this_tg - slot + sl;  // the tile-group of slot sl this round
            if (tgo >= n_tg || tok >= p.n_tok) continue;
            if (swiglu && tr != 0) continue;  // thread of the gate tile writes the pair
            float s = 0.f, s2 = 0.f;
            for (int w = 0; w < KS; ++w) {
                s += pb[(((sl * KS + w) * TR + tr) * NT + tok) * 16 + r];
                if (swiglu) s2 += pb[(((sl * KS + w) * TR + (TR - 1)) * NT + tok) * 16 + r];
            }
            const float inv = inv_rms(tok);
            if (swiglu) {
                const int j = tgo * 16 + r;
                if (j < r0) {
                    const float gv = s * inv, uv = s2 * inv;
                    sy0[j + (size_t)tok * p.ldy] = (gv / (1.f + expf(-gv))) * uv;
                }
            } else {
                float* y;
                const float* bias;
                if (orow((tgo * TR + tr) * 16 + r, y, bias)) {
                    float v = s * inv;
                    if (bias) v += *bias;
                    float* dst = y + (size_t)tok * p.ldy;
                    if (p.epi == ORC_EPI_ACCUM) *dst += v;
                    else *dst = v;
                }
            }
        }
    };
    auto advance = [&]() {
        tg += tg_stride;
        tt = tg_type(tg);
        tg_rows(tg, rp);
    };
    if (rounds > 0) {
        round_body(std::integral_constant<bool, true>{}, 0);
        for (int rd = 1; rd < rounds; ++rd) {
            advance();
            round_body(std::integral_constant<bool, false>{}, rd);
        }
    }
}

}  // namespace orc

// ── host side ────────────────────────────────────────────────────────────────
namespace orc {

bool mmq_type(int type) { return type == ORC_Q4_K || type == ORC_Q6_K || type == kMixK; }

// Token counts with a kernel; a launch of n tokens runs the smallest one
// >= n, with the extra tokens' rows zero and their outputs dropped.
static const int kNTs[] = {1, 2, 3, 4, 5, 6, 7, 8, 9, 12, 16};
static int nt_inst(int n) {
    for (int v : kNTs)
        if (v >= n) return v;
    return 0;
}

// The launch shape of a matrix. TR, KS and the unit ranges depend on the
// shape only (so do the results); FULL / windowed staging, the batch size and
// the window size change no result. KS is the split that minimises rounds
// times units per wave (the longest a wave computes); whole rows per wave
// (KS = 1) when there are enough tile-groups.
struct MCfg {
    int tr, ks;
};
static MCfg mmq_cfg(int type, const QmvParams& p) {
    const bool swiglu = p.epi == ORC_EPI_SWIGLU;
    const int rows_out = swiglu ? p.rows[0] : p.n_rows;
    const int n_tg = (rows_out + 15) / 16;  // TR = 2 pairs gate and up tiles of the same rows
    const int U = p.n_in / 128;
    auto cost = [&](int ks) {
        const int per_round = (kWv / ks) * g_n_cu;
        return (long)((n_tg + per_round - 1) / per_round) * ((U + ks - 1) / ks);
    };
    int ks = cost(8) < cost(16) ? 8 : 16;
    if (!swiglu && type != kMixK && cost(1) < cost(ks)) ks = 1;
    return {swiglu ? 2 : 1, ks};
}

static size_t lds_full(int type, int nt, int U, int tr) {
    return (size_t)mlayout(type != ORC_Q6_K, nt, U, U, tr).total;
}
static size_t lds_win(int type, int nt, int U, int tr, int hs) {
    return (size_t)mlayout(type != ORC_Q6_K, nt, U, kWv * hs, tr).total;
}

int mmq_max_tokens(int type, const QmvParams& p) {
    const MCfg cfg = mmq_cfg(type, p);
    const int U = p.n_in / 128;
    for (int i = (int)(sizeof(kNTs) / sizeof(kNTs[0])) - 1; i >= 0; --i) {
        const int nt = kNTs[i];
        if (lds_full(type, nt, U, cfg.tr) <= g_lds_max) return nt;
        if (cfg.ks == kWv && type != kMixK && lds_win(type, nt, U, cfg.tr, 1) <= g_lds_max) return nt;
    }
    return 0;
}

template <int QT, int NT, int TR, int KS, int UW, bool FULL>
static int mmq_go(const QmvParams& p, hipStream_t s, const LaunchEvents& ev, size_t lds, int grid) {
    if (ev.start)
        hipExtLaunchKernelGGL((k_mmq<QT, NT, TR, KS, UW, FULL>), dim3(grid), dim3(kWG), lds, s, ev.start, ev.stop, 0,
                              p);
    else
        hipLaunchKernelGGL((k_mmq<QT, NT, TR, KS, UW, FULL>), dim3(grid), dim3(kWG), lds, s, p);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

template <int QT, int NT>
static int mmq_nt(QmvParams p, const MCfg& cfg, hipStream_t s, const LaunchEvents& ev) {
    const int U = p.n_in / 128;
    const bool swiglu = p.epi == ORC_EPI_SWIGLU;
    const int rows_out = swiglu ? p.rows[0] : p.n_rows;
    const int n_tg = swiglu ? (rows_out + 15) / 16 : (rows_out + 16 * cfg.tr - 1) / (16 * cfg.tr);
    const int G = kWv / cfg.ks;
    const int grid = std::max(1, std::min((n_tg + G - 1) / G, g_n_cu));
    const bool full = lds_full(QT, NT, U, cfg.tr) <= g_lds_max;
    p.hs = 0;
    if (!full) {  // windows of a wave's range (KS = 16): the fewest that fit
        const int per_wave = (U + kWv - 1) / kWv;
        for (int nwin = 1; nwin <= per_wave; ++nwin) {
            p.hs = (per_wave + nwin - 1) / nwin;
            if (lds_win(QT, NT, U, cfg.tr, p.hs) <= g_lds_max) break;
        }
        if (cfg.ks != kWv || QT == kMixK || lds_win(QT, NT, U, cfg.tr, p.hs) > g_lds_max)
            return set_error(ORC_E_UNSUPPORTED, "gemm: activations do not fit LDS");
    }
    const size_t lds = full ? lds_full(QT, NT, U, cfg.tr) : lds_win(QT, NT, U, cfg.tr, p.hs);
    // batch sizes: a wave's whole range where the registers allow
    if constexpr (QT == kMixK) {
        if (cfg.ks == 8) return mmq_go<QT, NT, 1, 8, 3, true>(p, s, ev, lds, grid);
        return mmq_go<QT, NT, 1, kWv, 2, true>(p, s, ev, lds, grid);
    } else {
        if (cfg.tr == 2) {
            if (cfg.ks == 8) return mmq_go<QT, NT, 2, 8, 2, true>(p, s, ev, lds, grid);
            return full ? mmq_go<QT, NT, 2, kWv, 2, true>(p, s, ev, lds, grid)
                        : mmq_go<QT, NT, 2, kWv, 2, false>(p, s, ev, lds, grid);
        }
        if (cfg.ks == 1) return mmq_go<QT, NT, 1, 1, 4, true>(p, s, ev, lds, grid);
        if (cfg.ks == 8) return mmq_go<QT, NT, 1, 8, 3, true>(p, s, ev, lds, grid);
        return full ? mmq_go<QT, NT, 1, kWv, 4, true>(p, s, ev, lds, grid)
                    : mmq_go<QT, NT, 1, kWv, 4, false>(p, s, ev, lds, grid);
    }
}

template <int QT>
static int mmq_type_launch(const QmvParams& p, const MCfg& cfg, hipStream_t s, const LaunchEvents& ev) {
    switch (nt_inst(p.n_tok)) {
        case 1: return mmq_nt<QT, 1>(p, cfg, s, ev);
        case 2: return mmq_nt<QT, 2>(p, cfg, s, ev);
        case 3: return mmq_nt<QT, 3>(p, cfg, s, ev);
        case 4: return mmq_nt<QT, 4>(p, cfg, s, ev);
        case 5: return mmq_nt<QT, 5>(p, cfg, s, ev);
        case 6: return mmq_nt<QT, 6>(p, cfg, s, ev);
        case 7: return mmq_nt<QT, 7>(p, cfg, s, ev);
        case 8: return mmq_nt<QT, 8>(p, cfg, s, ev);
        case 9: return mmq_nt<QT, 9>(p, cfg, s, ev);
        case 12: return mmq_nt<QT, 12>(p, cfg, s, ev);
        case 16: return mmq_nt<QT, 16>(p, cfg, s, ev);
        default: return set_error(ORC_E_UNSUPPORTED, "gemm: 1..16 tokens per matrix-core launch");
    }
}

int mmq_launch(int type, const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    if (p.n_in % 256) return set_error(ORC_E_INVALID, "gemm: K-quant rows hold a multiple of 256 values");
    const MCfg cfg = mmq_cfg(type, p);
    switch (type) {
        case ORC_Q4_K: return mmq_type_launch<ORC_Q4_K>(p, cfg, s, ev);
        case ORC_Q6_K: return mmq_type_launch<ORC_Q6_K>(p, cfg, s, ev);
        case kMixK: return mmq_type_launch<kMixK>(p, cfg, s, ev);
        default: return set_error(ORC_E_UNSUPPORTED, "gemm: not a matrix-core type");
    }
}

}  // namespace orc

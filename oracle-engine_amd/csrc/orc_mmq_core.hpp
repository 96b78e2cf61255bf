// Matrix-core GEMM kernel k_mmq and its split-tile dispatch, shared by
// orc_mmq.hip (launches staged in one window, the prefill kernel, the C ABI
// side) and orc_mmq_win.hip (launches whose wave ranges are restaged in
// windows): the two kernel sets compile in parallel.
#pragma once
#include "orc_gemm.hpp"

#include <algorithm>

namespace orc {

template <class T> __device__ __forceinline__ T* spin(T* p) {
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T*)(((uint64_t)hi << 32) | lo);
}

// ── matrix-core path (Q4_K, Q6_K) ────────────────────────────────────────────
// Activations are the MFMA's A operand, weights the B operand (16 weight rows
// of a tile), so D[a row][weight row] lands with one weight row per lane:
// lane l holds D[4 (l/16) + i][l % 16]. Each activation x' (x times the norm
// weight times a per-token power of two that keeps it inside the fp16 range)
// is split as hi = fp16(x'), lo = fp16(x' - hi); hi + lo carries ~22 bits and
// every product with a weight code is exact in fp32. Up to 8 tokens, A row t
// holds token t's hi halves and row 8 + t its lo halves:
// one MFMA takes both, and the two rows' sums are added once per tile
// (lanes l and l + 32), which matches an fp32 dot product to fp32 rounding.
// A unit is half a superblock (128 values) of one row, in four 32-value
// slices of one v_mfma_f32_16x16x32_f16 each; lane group c (lanes 16c..16c+15)
// holds values 8c..8c+7 of a slice, the same for both types:
//  * Q4_K: a slice is one sub-block; its 6-bit scale is folded into the code
//    (sc * q <= 945, exact in fp16), d scales the unit's chain and the
//    minimum term dmin * m * sum(x) is added per sub-block on the VALU.
//  * Q6_K: a slice spans two 16-value sub-blocks whose int8 scales do not
//    fit the code exactly (sc * (q - 32) up to 4096), so the scaled code is
//    split into hi = fp16(sc (q - 32)) and lo = sc (q - 32) - hi (exact,
//    |lo| <= 1): one MFMA per code half and slice, d scales the chain.
// The eight waves of a workgroup split a tile's units into fixed contiguous
// ranges and their partial sums are added in wave order, so a (token, row)
// result does not depend on the token count or the token block: the tokens
// of a launch are independent bit for bit.
typedef _Float16 h8v __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f2v __attribute__((ext_vector_type(2)));

constexpr int kMWG = 512, kMW = kMWG / 64;
// Tokens per launch: up to 8 as stacked hi / lo rows of one A tile (rows
// 0-7 the hi halves of tokens 0-7, rows 8-15 their lo halves); 9 to 16 as
// two A tiles (the hi halves of tokens 0-15, and their lo halves) against
// the same B: every (token, row) sum is formed by the same operations in
// the same order either way. Whole-tile (tall) launches stay at 8.
constexpr int kMmqMaxNT = 16, kMmqTallNT = 8;
template <int NT> constexpr bool mmq_wide() { return NT > 8; }

// code permutation of one 8-value run (bytes 0,2 / 1,3 / 4,6 / 5,7 land in
// consecutive halves when two dwords are unpacked into fp16 pairs)
__device__ __forceinline__ int perm8(int j) { return (j & 4) | ((j & 1) << 1) | ((j >> 1) & 1); }

// A entries: per unit, per (slice, lane group, half (hi, lo), token), 8 halves;
// kABytes per (slice, lane group, token)
constexpr int kASlices = 4, kABytes = 32;

// A entry of element kk (0..255) of superblock b: unit u, slice i, lane
// group c, position j of the element among the entry's 8 halves.
__device__ __forceinline__ void a_slot(int b, int kk, int& u, int& i, int& c, int& j) {
    u = 2 * b + (kk >> 7);
    i = (kk >> 5) & 3;
    c = (kk >> 3) & 3;
    j = perm8(kk & 7);
}

// Loads through the global address space (a generic pointer would make
// them flat loads, which LDS waits also have to drain).
typedef const __attribute__((address_space(1))) u32x4_u* g16p;
typedef const __attribute__((address_space(1))) u32x2_u* g8p;
typedef const __attribute__((address_space(1))) u16_u* g2p;
__device__ __forceinline__ u32x4 ldg16(const uint8_t* p) { return *(g16p)p; }
__device__ __forceinline__ u32x2 ldg8(const uint8_t* p) { return *(g8p)p; }
__device__ __forceinline__ uint32_t ldg2(const uint8_t* p) { return *(g2p)p; }
// outputs and biases through the global address space too (flat accesses
// would also count against the LDS wait counter)
typedef const __attribute__((address_space(1))) float* gfp;
typedef __attribute__((address_space(1))) float* gwp;

// Constants held in registers: a VOP3 operation such as v_and_or_b32 takes no
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

// Four 6-bit Q6_K codes (low nibbles at bit sh of the bytes of lw, the two
// high bits at bit 2i of the bytes of hw, i a compile-time slice index) as
// two words of fp16 pairs 1024 + q in the A entries' element order: bytes 0
// and 2 into r0, 1 and 3 into r1 (each code in the low byte of a half whose
// high byte is 0x64). One AND-OR and one shift-and build the clean codes,
// one byte permute per word places them.
template <int I>
__device__ __forceinline__ void q6k_magic(uint32_t lw, uint32_t hw, int sh, uint32_t& r0, uint32_t& r1) {
    uint32_t h;  // bits 4, 5 of each byte
    if constexpr (I < 2) h = (hw << (4 - 2 * I)) & 0x30303030u;
    else h = (hw >> (2 * I - 4)) & 0x30303030u;
    const uint32_t q = ((sh ? lw >> 4 : lw) & 0x0F0F0F0Fu) | h;
    const uint32_t mg = vreg(0x64646464u);
    r0 = __builtin_amdgcn_perm(mg, q, sreg(0x04020400u));  // [q0, 0x64, q2, 0x64]
    r1 = __builtin_amdgcn_perm(mg, q, sreg(0x04030401u));  // [q1, 0x64, q3, 0x64]
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

// Loaded bytes of one unit of one row for lane group c (either type).
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

__device__ __forceinline__ h2v as_h2(uint32_t v) { return __builtin_bit_cast(h2v, v); }
__device__ __forceinline__ uint32_t as_u32(h2v v) { return __builtin_bit_cast(uint32_t, v); }

// Where a unit's activations live in LDS.
struct MCtx {
    const uint8_t* abase;  // A entries: [unit slot][slice][lane group][token] hi | lo
    int a_stride_u;        // bytes per unit
    const float* sx;       // Q4_K: sums of x g over each 32-value sub-block, [token][sub-block]
    int sx_stride;
    const float* esc;      // 2^-e of each (unit, token), [unit][NTP]
};

template <int NT> constexpr int ntp() { return (NT + 3) & ~3; }

// Byte offset of A entry (slice i, lane group c, half hl, token t) in a unit.
template <int NT> __device__ __forceinline__ int a_off(int i, int c, int hl, int t) {
    return (((i * 4 + c) * 2 + hl) * NT + t) * 16;
}

// The lane's A entries of a unit (all four slices; lane row r = lane % 16)
// and the 2^-e of the tokens of its D rows, all LDS reads in flight. Up to
// 8 tokens: row r is the hi half of token r or the lo half of token r - 8,
// D rows are tokens 4 (c % 2) + i. 9 to 16 tokens: a holds the hi and al
// the lo half of token r, D rows are tokens 4 c + i.
// Rows of tokens past n_tok read whatever the neighbouring entries hold
// (always inside the workgroup's LDS: the esc, red and part arrays follow
// the A entries). An MFMA's D row depends only on the same A row, the hi
// and lo rows folded together belong to one token, and every epilogue
// drops rows of tokens >= n_tok, so those values reach no output; reading
// them unmasked saves zeroing 16 registers per unit.
template <int NT>
__device__ __forceinline__ void a_load(int u, int ua, int lane, const MCtx& m, h8v (&a)[4], h8v (&al)[4], float4& es) {
    constexpr bool W = mmq_wide<NT>();
    const int c = lane >> 4, r = lane & 15, t = W ? r : r & 7, tb = W ? 4 * c : 4 * (c & 1);
    u32x4 h[4], l[4];
    const uint8_t* ap = m.abase + (size_t)ua * m.a_stride_u + a_off<NT>(0, c, W ? 0 : r >> 3, t);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = *(const u32x4*)(ap + a_off<NT>(i, 0, 0, 0));
        if constexpr (W) l[i] = *(const u32x4*)(ap + a_off<NT>(i, 0, 1, 0));
        else l[i] = u32x4{0u, 0u, 0u, 0u};
    }
    es = *(const float4*)(m.esc + u * ntp<NT>() + tb);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[i] = __builtin_bit_cast(h8v, h[i]);
        al[i] = __builtin_bit_cast(h8v, l[i]);
    }
}

// Adds the lo rows' sums to the hi rows' (lanes l and l + 32): afterwards
// lanes 0..31 hold the tile's results for tokens 4 (l / 16) + i.
template <int TR> __device__ __forceinline__ void fold_lo(f4v (&acc)[TR]) {
#pragma unroll
    for (int tr = 0; tr < TR; ++tr)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[tr][e] += __shfl_xor(acc[tr][e], 32, 64);
}

// D entries e of a lane that can hold a token below n_tok: lane row c holds
// tokens 4 (c % 2) + e of stacked launches (4 c + e of wide ones), so below
// 4 tokens entries e >= n_tok belong to no token and are not scaled (they
// stay zero and reach no output).
template <int NT> constexpr int kDRows = (!mmq_wide<NT>() && NT < 4) ? NT : 4;

// Q4_K unit of TR tiles with the lane's A entries given: scale-folded codes
// (slices alternating between two chains), then acc += d 2^-e D, minus, on
// the hi rows only, the sum over the unit's sub-blocks of dmin m sum(x g).
template <int NT, int TR>
__device__ __forceinline__ void mmq_core_q4k(const MUnit (&M)[TR], int u, int lane, const MCtx& m, const h8v (&a)[4],
                                             const h8v (&al)[4], float4 es, f4v (&acc)[TR], f4v (&acl)[TR]) {
    constexpr bool W = mmq_wide<NT>();
    const int c = lane >> 4, h = u & 1, r = lane & 15;
    // A operand of the minimum term (one 16x16x4 fp32 MFMA per tile): lane
    // (c, r) holds token r's sum of x g over sub-block 4u + c; zero on the
    // lo rows of stacked launches and past the last token
    constexpr int NA = W ? NT : (NT < 8 ? NT : 8);
    const float sxa = r < NA ? m.sx[r * m.sx_stride + 4 * u + c] : 0.f;
    const float esv[4] = {es.x, es.y, es.z, es.w};
#pragma unroll
    for (int tr = 0; tr < TR; ++tr) {
        f4v D = f4v{0.f, 0.f, 0.f, 0.f}, Dl = D;  // even and odd slices in independent chains
        f4v E = D, El = D;                         // the same for the lo tile (9-16 tokens)
        const float dmin = h2f(M[tr].a.x >> 16);
        uint32_t sc4, mn4;
        q4k_unit_sm(h, M[tr].a.y, M[tr].b.x, M[tr].b.y, sc4, mn4);
        // B operand: minus dmin m of sub-block 4u + c of the lane's row
        const float bm = -(dmin * (float)((mn4 >> (8 * c)) & 0xFFu));
        // code words shifted by one byte, shared by a low-nibble slice and its high-nibble partner
        const uint32_t s8[4] = {M[tr].c.x >> 8, M[tr].c.y >> 8, M[tr].d.x >> 8, M[tr].d.y >> 8};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t sc = (sc4 >> (8 * i)) & 0xFFu;
            const u32x2 src = (i >> 1) ? M[tr].d : M[tr].c;
            // low nibbles as fp16 1024 + q: (1024 + q) sc - 1024 sc; high nibbles in
            // place as 1024 + 16 q: (1024 + 16 q) (sc / 16) - 64 sc; either way sc q
            // with one rounding (exact: sc q <= 945, sc / 16 and 64 sc exact in fp16)
            const bool hn = i & 1;
            const float scs = (float)sc;
            const _Float16 f = (_Float16)(hn ? scs * 0.0625f : scs), o = (_Float16)(hn ? scs * -64.f : scs * -1024.f);
            const h2v scv{f, f}, off{o, o};
            const uint32_t mk = hn ? sreg(0x00F000F0u) : sreg(0x000F000Fu), mg = vreg(0x64006400u);
            const uint32_t r[4] = {(src.x & mk) | mg, (s8[2 * (i >> 1)] & mk) | mg, (src.y & mk) | mg,
                                   (s8[2 * (i >> 1) + 1] & mk) | mg};
            u32x4 bq;
#pragma unroll
            for (int k = 0; k < 4; ++k) bq[k] = as_u32(__builtin_elementwise_fma(as_h2(r[k]), scv, off));
            const h8v b = __builtin_bit_cast(h8v, bq);
            if (i & 1) {
                Dl = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b, Dl, 0, 0, 0);
                if constexpr (W) El = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b, El, 0, 0, 0);
            } else {
                D = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[i], b, D, 0, 0, 0);
                if constexpr (W) E = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[i], b, E, 0, 0, 0);
            }
        }
        D += Dl;
        if constexpr (W) E += El;
        const float d = h2f(M[tr].a.x & 0xFFFFu);
        f4v t = acc[tr];
#pragma unroll
        for (int e = 0; e < kDRows<NT>; ++e) {
            t[e] = __builtin_fmaf(d * esv[e], D[e], acc[tr][e]);
            // the lo tile of 9-16 token launches takes no minimum term
            if constexpr (W) acl[tr][e] = __builtin_fmaf(d * esv[e], E[e], acl[tr][e]);
        }
        // acc = t - sum over the unit's four sub-blocks of dmin m sum(x g)
        acc[tr] = __builtin_amdgcn_mfma_f32_16x16x4f32(sxa, bm, t, 0, 0, 0);
    }
}

// Q4_K unit of TR tiles, A entries from the LDS.
template <int NT, int TR>
__device__ __forceinline__ void mmq_unit_q4k(const MUnit (&M)[TR], int u, int ua, int lane, const MCtx& m,
                                             f4v (&acc)[TR], f4v (&acl)[TR]) {
    h8v a[4], al[4];
    float4 es;
    a_load<NT>(u, ua, lane, m, a, al, es);
    mmq_core_q4k<NT, TR>(M, u, lane, m, a, al, es, acc, acl);
}

// Q6_K unit of TR tiles with the lane's A entries given: scale-folded hi /
// lo codes in two chains, acc += d 2^-e D.
template <int NT, int TR>
__device__ __forceinline__ void mmq_core_q6k(const MUnit (&M)[TR], int lane, const h8v (&a)[4], const h8v (&al)[4],
                                             float4 es, f4v (&acc)[TR], f4v (&acl)[TR]) {
    constexpr bool W = mmq_wide<NT>();
    const int c = lane >> 4;
    const float esv[4] = {es.x, es.y, es.z, es.w};
#pragma unroll
    for (int tr = 0; tr < TR; ++tr) {
        f4v D = f4v{0.f, 0.f, 0.f, 0.f}, Dl = D;  // hi and lo code halves in independent chains
        f4v E = D, El = D;                         // the same for the lo tile (9-16 tokens)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // 6-bit codes of the lane's 8 values of slice i (stored + 32)
            const u32x2 src = (i & 1) ? M[tr].b : M[tr].a;
            const int sh = 4 * (i >> 1);
            uint32_t r[4];
            switch (i) {  // the slice index as a constant of the helper
                case 0: q6k_magic<0>(src.x, M[tr].c.x, sh, r[0], r[1]), q6k_magic<0>(src.y, M[tr].c.y, sh, r[2], r[3]); break;
                case 1: q6k_magic<1>(src.x, M[tr].c.x, sh, r[0], r[1]), q6k_magic<1>(src.y, M[tr].c.y, sh, r[2], r[3]); break;
                case 2: q6k_magic<2>(src.x, M[tr].c.x, sh, r[0], r[1]), q6k_magic<2>(src.y, M[tr].c.y, sh, r[2], r[3]); break;
                default: q6k_magic<3>(src.x, M[tr].c.x, sh, r[0], r[1]), q6k_magic<3>(src.y, M[tr].c.y, sh, r[2], r[3]); break;
            }
            // scale of the lane's 16-value sub-block 2i + c/2
            const int si = 2 * i + (c >> 1);
            const uint32_t sw = si < 4 ? M[tr].d.x : M[tr].d.y;
            const _Float16 sf = (_Float16)(float)(int8_t)((sw >> (8 * (si & 3))) & 0xFFu);
            const h2v sc2{sf, sf}, off{(_Float16)-1056.f, (_Float16)-1056.f};  // 1024 + 32
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
        D += Dl;
        if constexpr (W) E += El;
        const float d = h2f(M[tr].e);
#pragma unroll
        for (int e = 0; e < kDRows<NT>; ++e) {
            acc[tr][e] = __builtin_fmaf(d * esv[e], D[e], acc[tr][e]);
            if constexpr (W) acl[tr][e] = __builtin_fmaf(d * esv[e], E[e], acl[tr][e]);
        }
    }
}

// Q6_K unit of TR tiles, A entries from the LDS.
template <int NT, int TR>
__device__ __forceinline__ void mmq_unit_q6k(const MUnit (&M)[TR], int u, int ua, int lane, const MCtx& m,
                                             f4v (&acc)[TR], f4v (&acl)[TR]) {
    h8v a[4], al[4];
    float4 es;
    a_load<NT>(u, ua, lane, m, a, al, es);
    mmq_core_q6k<NT, TR>(M, lane, a, al, es, acc, acl);
}

// DPP reductions inside one 16-lane row (fixed order): the quad sum, then the
// half-row and row mirrors
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

// Row -> segment by comparisons over values passed by value (scalar
// registers): no array or struct holds them, so a lane-dependent choice
// stays a register select instead of an indexed load.
__device__ __forceinline__ int seg_of(int j, int n_seg, int r0, int r1, int& jj) {
    const bool s1 = n_seg > 1 && j >= r0;
    const bool s2 = n_seg > 2 && j >= r0 + r1;
    jj = s2 ? j - r0 - r1 : (s1 ? j - r0 : j);
    return s2 ? 2 : (s1 ? 1 : 0);
}
template <class T> __device__ __forceinline__ T* pick3(int s, T* a, T* b, T* c) { return s == 2 ? c : (s == 1 ? b : a); }

// KS1 = false: the eight waves of a workgroup split one tile's units (small
// matrices, where tiles are few); true: each wave owns whole tiles and its
// ring of loads runs on across them without barriers (tall matrices).
// WPE: waves per SIMD the registers are sized for: 2 (one workgroup per CU),
// or 4 (two per CU, at most 128 registers) for the kernels that fit them
// without spills, whose launches then run up to two workgroups per CU.
template <int QT, int NT, int TR, int UW, int SW, bool KS1, bool MW, int WPE>
__global__ __launch_bounds__(kMWG) __attribute__((amdgpu_waves_per_eu(WPE))) void k_mmq(QmvParams p) {
    // token block blockIdx.y: tokens [NT y, NT (y + 1)) of the launch. Every
    // block holds exactly NT tokens (the kernel stages and writes NT rows).
    if (blockIdx.y) {
        const size_t t0 = (size_t)blockIdx.y * NT;
        p.x += t0 * p.ldx;
#pragma unroll
        for (int i = 0; i < 3; ++i)
            if (p.y[i]) p.y[i] += t0 * p.ldy;
    }
    constexpr bool MIX = QT == kMixK;  // each 16-row tile takes its segment's type
    constexpr bool SX = QT == ORC_Q4_K || MIX;
    extern __shared__ __attribute__((aligned(16))) uint8_t msm[];
    // wave index through readfirstlane: unit indices derived from it are
    // then known to be wave-uniform (scalar branches, no exec masking)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane >> 4, n = lane & 15;
    const int kn = p.n_in;
    const int U = kn / 128;                                      // units per row
    const int a_stride_u = kASlices * 4 * NT * kABytes;  // bytes per unit (all tokens)
    constexpr int NTP = ntp<NT>();
    // A entries: every unit (KS1), or per wave a window of HS units of its
    // range, restaged window by window when the range does not fit the LDS
    const int HS = KS1 ? U : p.hs;
    uint8_t* abase = msm;
    float* sx = (float*)(msm + (size_t)(KS1 ? U : kMW * HS) * a_stride_u);  // Q4_K: [NT][kn/32]
    const int sx_stride = kn / 32;
    float* esc = sx + (SX ? NT * sx_stride : 0);  // [U][NTP]
    float* red = esc + U * NTP;                                // [NT][kMW * 4] sums of x^2 per 16-lane row
    float* part = red + NT * kMW * 4;                          // [kMW][TR][NT][16]
    const MCtx mc{abase, a_stride_u, sx, sx_stride, esc};
    const uint8_t *const sw0 = spin(p.w[0]), *const sw1 = spin(p.w[1]), *const sw2 = spin(p.w[2]);
    float *const sy0 = spin(p.y[0]), *const sy1 = spin(p.y[1]), *const sy2 = spin(p.y[2]);
    const float *const sb0 = spin(p.bias[0]), *const sb1 = spin(p.bias[1]), *const sb2 = spin(p.bias[2]);
    const int n_seg = p.n_seg, r0 = p.rows[0], r1 = p.rows[1];
    // mixed launches: the segment types packed in one word (a choice between
    // separately loaded values would be folded into an indexed load of the
    // parameter block, which then lives on the stack); row bytes follow
    const uint32_t tys = (uint32_t)p.seg_type[0] | ((uint32_t)p.seg_type[1] << 8) | ((uint32_t)p.seg_type[2] << 16);
    auto seg_type = [=](int sgi) { return MIX ? (int)((tys >> (8 * sgi)) & 0xFFu) : QT; };
    const uint64_t rb_q4k = (uint64_t)(kn / 256) * 144, rb_q6k = (uint64_t)(kn / 256) * 210;
    // weight row of logical row jl (clamped to row 0 past the end: loads stay in bounds)
    auto wrow = [=](int jl) {
        int jj;
        const int sgi = seg_of(jl < p.n_rows ? jl : 0, n_seg, r0, r1, jj);
        const uint64_t rb = MIX ? (seg_type(sgi) == ORC_Q4_K ? rb_q4k : rb_q6k) : p.row_bytes;
        return pick3(sgi, sw0, sw1, sw2) + (size_t)jj * rb;
    };
    // weight type of a tile (its first row's segment; mixed launches keep
    // every segment a whole number of tiles)
    auto tile_type = [=](int tile) {
        int jj;
        return seg_type(seg_of(tile * 16 * TR < p.n_rows ? tile * 16 * TR : 0, n_seg, r0, r1, jj));
    };
    // output (and bias) of logical row jl; false past the end
    auto orow = [=](int jl, float*& y, const float*& bias) {
        if (jl >= p.n_rows) return false;
        int jj;
        const int sgi = seg_of(jl, n_seg, r0, r1, jj);
        y = pick3(sgi, sy0, sy1, sy2) + jj;
        const float* bb = pick3(sgi, sb0, sb1, sb2);
        bias = bb ? bb + jj : nullptr;
        return true;
    };

    const int u0 = wave * U / kMW, u1 = (wave + 1) * U / kMW;
    // windowed staging (MW: the host found a wave range longer than the LDS
    // window); kernels without it carry no restaging path in the unit loop,
    // which keeps their register count and load waits down
    const bool multi_win = MW && !KS1 && u0 + HS < u1;
    // LDS slot of unit u of the window that starts at unit wb
    auto aslot = [=](int u, int wb) { return KS1 ? u : wave * HS + (u - wb); };
    const bool swiglu = p.epi == ORC_EPI_SWIGLU;
    const int rows_out = swiglu ? p.rows[0] : p.n_rows;
    const int n_tiles = swiglu ? (rows_out + 15) / 16 : (rows_out + 16 * TR - 1) / (16 * TR);

    auto tile_rows = [&](int tile, const uint8_t* (&rp)[TR]) {
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) {
            const int jl = swiglu ? tr * r0 + (tile * 16 + n < r0 ? tile * 16 + n : r0) : (tile * TR + tr) * 16 + n;
            rp[tr] = wrow(jl);
        }
    };
    // a ring of UW units of the TR rows in flight: unit u sits in slot
    // (u - u0) % UW and its slot is refilled with unit u + UW once consumed
    MUnit buf[UW][TR];

    // the unit range a wave computes: its own eighth (split tiles) or all
    const int k0u = KS1 ? 0 : u0, k1u = KS1 ? U : u1;
    int tile = KS1 ? blockIdx.x * kMW + wave : blockIdx.x;
    const int tstride = KS1 ? gridDim.x * kMW : gridDim.x;
    const uint8_t* rp[TR];
    int tt = tile_type(tile < n_tiles ? tile : 0);  // type of the tile being computed
    // the first tile's first units go out once the wave's first staging
    // window is stored: issued before, the weight stream of the CU's waves
    // delays the x reads queued behind it (measured: 0.3-1.6 us per launch)
    auto start_ring = [&]() {
        if (tile < n_tiles) {
            tile_rows(tile, rp);
#pragma unroll
            for (int k = 0; k < UW; ++k)
                if (k0u + k < k1u) {
#pragma unroll
                    for (int tr = 0; tr < TR; ++tr) buf[k][tr].load(tt, rp[tr], k0u + k, c);
                }
        }
    };

    // ── stage this wave's K range as hi/lo fp16 in the A layout ──
    // Lane q of a pass holds 8 consecutive values (group q); a 16-lane row
    // holds one unit. Each (unit, token) gets its own power of two 2^e that
    // brings max |x g| below 2^14 (reduced inside the row with DPP), so the
    // halves stay in range; the sums of x g for the Q4_K minimum and of x^2
    // for the norm are taken unscaled.
    constexpr int GPL = SW / 4;  // groups per lane per pass of SW units
    const bool norm = p.norm_w != nullptr;
    float ssl[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) ssl[t] = 0.f;
    // stages units [s0, s1) of the wave's range; sum_sq adds their x^2 to ssl
    auto stage = [&](int s0, int s1, bool sum_sq) {
    for (int cs = s0; cs < s1; cs += SW) {
        const int ng = 16 * min(SW, s1 - cs);
        float v[NT][GPL][8], gw[GPL][8];
#pragma unroll
        for (int k = 0; k < GPL; ++k) {
            const int q = lane + 64 * k;
            const int qc = q < ng ? q : 0;  // lanes past the range read group 0 and are masked below
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float* src = p.x + (size_t)t * p.ldx + 128 * cs + 8 * qc;
                *(float4*)v[t][k] = *(const float4*)src;
                *(float4*)(v[t][k] + 4) = *(const float4*)(src + 4);
            }
            // norm weights (x itself stands in when there are none; unused then)
            const float* gp = (norm ? p.norm_w : p.x) + 128 * cs + 8 * qc;
            *(float4*)gw[k] = *(const float4*)gp;
            *(float4*)(gw[k] + 4) = *(const float4*)(gp + 4);
        }
        if (norm) {
#pragma unroll
            for (int k = 0; k < GPL; ++k) {
                const bool in = sum_sq && lane + 64 * k < ng;
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    // the chain over the lane's values, kept only for lanes inside the range
                    float sq = ssl[t];
#pragma unroll
                    for (int e = 0; e < 8; ++e) sq = __builtin_fmaf(v[t][k][e], v[t][k][e], sq);
                    ssl[t] = in ? sq : ssl[t];
#pragma unroll
                    for (int e = 0; e < 8; ++e) v[t][k][e] *= gw[k][e];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < GPL; ++k) {
            const int q = lane + 64 * k;
            const bool valid = q < ng;
            const int k0 = 128 * cs + 8 * q, b = k0 >> 8;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                float mx = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[t][k][e]));
                mx = row_max(valid ? mx : 0.f);
                int e2 = 0;
                if (mx > 0.f && mx <= 3.0e38f) {
                    int ex;
                    (void)frexpf(mx, &ex);  // mx < 2^ex
                    e2 = 14 - ex;
                }
                const float up = ldexpf(1.f, e2);
                float s8 = ((v[t][k][0] + v[t][k][1]) + (v[t][k][2] + v[t][k][3])) +
                           ((v[t][k][4] + v[t][k][5]) + (v[t][k][6] + v[t][k][7]));
                if constexpr (SX) s8 = quad_sum(s8);
                if (!valid) continue;
                if ((lane & 15) == 0) esc[(cs + (q >> 4)) * NTP + t] = ldexpf(1.f, -e2);
                float w[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) w[e] = v[t][k][e] * up;
                int u, i, cc, j;
                a_slot(b, k0 & 255, u, i, cc, j);
                // hi halves converted two at a time, lo from the same rounded halves
                h8v hi, lo;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const h2v hp = __builtin_convertvector((f2v){w[e], w[e + 1]}, h2v);
                    hi[perm8(e)] = hp.x;
                    hi[perm8(e + 1)] = hp.y;
                    lo[perm8(e)] = (_Float16)(w[e] - (float)hp.x);
                    lo[perm8(e + 1)] = (_Float16)(w[e + 1] - (float)hp.y);
                }
                uint8_t* ap = abase + (size_t)aslot(u, s0) * a_stride_u;
                *(h8v*)(ap + a_off<NT>(i, cc, 0, t)) = hi;
                *(h8v*)(ap + a_off<NT>(i, cc, 1, t)) = lo;
                if (SX && (lane & 3) == 0) sx[t * sx_stride + (k0 >> 5)] = s8;
            }
        }
    }
    };
    // the wave's LDS accesses before this point are ordered before those after
    auto wave_lds_sync = [] {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    };
    auto write_red = [&] {
        if (norm) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const float r = row_sum(ssl[t]);
                if ((lane & 15) == 0) red[t * kMW * 4 + wave * 4 + c] = r;
            }
        }
    };
    stage(u0, multi_win ? u0 + HS : u1, true);
    int wb = u0;  // first unit of the window of the wave's range held in the LDS
    start_ring();
    if (!multi_win) write_red();  // else once the first tile has staged every window
    if constexpr (KS1) {
        __syncthreads();  // every wave reads every unit
    } else {
        wave_lds_sync();  // the wave reads only what it wrote
    }
    auto inv_rms = [&](int tok) {
        if (!norm) return 1.f;
        float ss = 0.f;
        for (int j = 0; j < kMW * 4; ++j) ss += red[tok * kMW * 4 + j];
        return 1.f / sqrtf(ss / (float)kn + p.eps);
    };
    float inv_l[4] = {1.f, 1.f, 1.f, 1.f};  // whole-tile mode: 1/rms of the lane's tokens 4c + i
    if constexpr (KS1) {
#pragma unroll
        for (int i = 0; i < 4; ++i) inv_l[i] = inv_rms(min(4 * c + i, NT - 1));
    }

    bool first_tile = true;
    while (tile < n_tiles) {
        // the slot of unit uu is refilled after use with unit uu + UW, or,
        // past the end of the tile, with unit k of the wave's next tile
        const int next = tile + tstride;
        const uint8_t* rpn[TR];
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) rpn[tr] = rp[tr];
        if (next < n_tiles) tile_rows(next, rpn);
        const int ttn = next < n_tiles ? tile_type(next) : tt;
        f4v acc[TR], acl[TR];  // acl: the lo tile of 9-16 token launches
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) acc[tr] = acl[tr] = f4v{0.f, 0.f, 0.f, 0.f};
        for (int ub = k0u; ub < k1u; ub += UW) {
#pragma unroll
            for (int k = 0; k < UW; ++k)
                if (ub + k < k1u) {
                    if (multi_win) {  // windows are walked in order, from u0 again for every tile
                        const int nwb = ub + k == u0 ? u0 : (ub + k == wb + HS ? wb + HS : wb);
                        if (nwb != wb) {
                            wave_lds_sync();
                            stage(nwb, min(u1, nwb + HS), first_tile);
                            wave_lds_sync();
                            wb = nwb;
                        }
                    }
                    if (tt == ORC_Q4_K)
                        mmq_unit_q4k<NT, TR>(buf[k], ub + k, aslot(ub + k, wb), lane, mc, acc, acl);
                    else
                        mmq_unit_q6k<NT, TR>(buf[k], ub + k, aslot(ub + k, wb), lane, mc, acc, acl);
                    if (ub + k + UW < k1u) {
#pragma unroll
                        for (int tr = 0; tr < TR; ++tr) buf[k][tr].load(tt, rp[tr], ub + k + UW, c);
                    } else if (next < n_tiles && k0u + k < k1u) {
#pragma unroll
                        for (int tr = 0; tr < TR; ++tr) buf[k][tr].load(ttn, rpn[tr], k0u + k, c);
                    }
                }
        }
        if constexpr (mmq_wide<NT>()) {  // hi + lo, the sum fold_lo forms across lanes
#pragma unroll
            for (int tr = 0; tr < TR; ++tr)
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[tr][e] += acl[tr][e];
        } else {
            fold_lo<TR>(acc);
        }
        if (multi_win && first_tile) write_red();
        first_tile = false;
        const int this_tile = tile;
        tile = next;
        tt = ttn;
#pragma unroll
        for (int tr = 0; tr < TR; ++tr) rp[tr] = rpn[tr];
        if constexpr (KS1) {
            // whole rows in one wave: the lane's outputs (token 4c + i, row n) directly
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = 4 * c + i;
                if (tok >= NT) continue;
                const float inv = inv_l[i];
                if (swiglu) {
                    const int j = this_tile * 16 + n;
                    if (j < p.rows[0]) {
                        const float gv = acc[0][i] * inv, uv = acc[TR - 1][i] * inv;
                        *(gwp)(sy0 + j + (size_t)tok * p.ldy) = (gv / (1.f + expf(-gv))) * uv;
                    }
                } else {
#pragma unroll
                    for (int tr = 0; tr < TR; ++tr) {
                        float* y;
                        const float* bias;
                        if (orow((this_tile * TR + tr) * 16 + n, y, bias)) {
                            float v = acc[tr][i] * inv;
                            if (bias) v += *(gfp)bias;
                            float* dst = y + (size_t)tok * p.ldy;
                            if (p.epi == ORC_EPI_ACCUM) *(gwp)dst += v;
                            else *(gwp)dst = v;
                        }
                    }
                }
            }
            continue;
        }
        // partial sums of this wave's units for the lane's tokens 4c + i
#pragma unroll
        for (int tr = 0; tr < TR; ++tr)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int tok = 4 * c + i;
                if (tok < NT) part[((wave * TR + tr) * NT + tok) * 16 + n] = acc[tr][i];
            }
        __syncthreads();
        // wave-ordered sum and the epilogue: one thread per (tile row, token)
        if (swiglu) {
            if (tid < NT * 16) {
                const int tok = tid >> 4, r = tid & 15, j = this_tile * 16 + r;
                float gs = 0.f, us = 0.f;
                for (int w = 0; w < kMW; ++w) {
                    gs += part[((w * TR + 0) * NT + tok) * 16 + r];
                    us += part[((w * TR + (TR - 1)) * NT + tok) * 16 + r];
                }
                const float inv = inv_rms(tok);
                if (j < p.rows[0]) {
                    const float gv = gs * inv, uv = us * inv;
                    *(gwp)(sy0 + j + (size_t)tok * p.ldy) = (gv / (1.f + expf(-gv))) * uv;
                }
            }
        } else if (tid < TR * NT * 16) {
            const int tr = tid / (NT * 16), tok = (tid >> 4) % NT, r = tid & 15;
            float s = 0.f;
            for (int w = 0; w < kMW; ++w) s += part[((w * TR + tr) * NT + tok) * 16 + r];
            const float inv = inv_rms(tok);
            const int jl = (this_tile * TR + tr) * 16 + r;
            float* y;
            const float* bias;
            if (orow(jl, y, bias)) {
                float v = s * inv;
                if (bias) v += *(gfp)bias;
                float* dst = y + (size_t)tok * p.ldy;
                if (p.epi == ORC_EPI_ACCUM) *(gwp)dst += v;
                else *(gwp)dst = v;
            }
        }
        __syncthreads();
    }
}

// ── host side ────────────────────────────────────────────────────────────────
static size_t mmq_lds(int type, int nt, int kn, int tr, int hs) {
    const int U = kn / 128, ntp = (nt + 3) & ~3;
    size_t b = (size_t)(hs ? kMW * hs : U) * 512 * nt;          // hi + lo halves: 128 values x 4 B per unit and token
    if (type == ORC_Q4_K || type == kMixK) b += (size_t)nt * (kn / 32) * 4;  // per-sub-block sums
    b += (size_t)U * ntp * 4;                                    // per-(unit, token) scales
    b += (size_t)(nt * kMW * 4 + kMW * tr * nt * 16) * 4;        // x^2 row sums, partial sums
    return b;
}

// Whole-tile mode (each wave owns whole tiles, every unit of a row staged):
// chosen by the shape alone, at kMmqTallNT tokens, so a shape takes the same
// mode (and reduction order) at every token count.
static bool mmq_tall(int type, const QmvParams& p) {
    const bool two = type != kMixK && (p.epi == ORC_EPI_SWIGLU || (type == ORC_Q4_K && p.n_rows >= 32 * g_n_cu));
    const int rows_out = p.epi == ORC_EPI_SWIGLU ? p.rows[0] : p.n_rows;
    return type != kMixK && rows_out / (two ? 32 : 16) >= 2 * kMW * g_n_cu && p.epi != ORC_EPI_SWIGLU &&
           mmq_lds(type, kMmqTallNT, p.n_in, two ? 2 : 1, 0) <= g_lds_max;
}

// Units per staging window when a wave's range of per_wave units is staged
// in nwin windows. A window shorter than the range is a whole number of
// four-unit passes: lane row c then stages units c, c + 4, ... of the range
// in that order whatever the window, so the RMSNorm's per-lane sums of x^2
// (and the norm) do not depend on the window size, which the token count
// sets.
static int mmq_window(int per_wave, int nwin) {
    const int hs = (per_wave + nwin - 1) / nwin;
    return hs >= per_wave ? hs : (hs + 3) & ~3;
}

template <bool MW, int QT, int NT, int TR, int UW, int SW, bool KS1, int WPE = 2>
static int mmq_shape(const QmvParams& p0, hipStream_t s, const LaunchEvents& ev) {
    QmvParams p = p0;
    const bool swiglu = p.epi == ORC_EPI_SWIGLU;
    const int rows_out = swiglu ? p.rows[0] : p.n_rows;
    const int n_tiles = swiglu ? (rows_out + 15) / 16 : (rows_out + 16 * TR - 1) / (16 * TR);
    if (p.tok_block != NT || p.n_tok % NT) return set_error(ORC_E_INVALID, "gemm: token blocks must be whole");
    const dim3 grid(std::max(1, std::min(KS1 ? (n_tiles + kMW - 1) / kMW : n_tiles, (WPE / 2) * g_n_cu)),
                    p.n_tok / NT);  // the launch's token blocks
    // split-tile mode: the fewest staging windows per wave range that fit
    p.hs = 0;
    if (!KS1) {
        const int per_wave = (p.n_in / 128 + kMW - 1) / kMW;
        for (int nwin = 1; nwin <= per_wave; ++nwin) {
            p.hs = mmq_window(per_wave, nwin);
            if (mmq_lds(QT, NT, p.n_in, TR, p.hs) <= g_lds_max) break;
        }
    }
    const size_t lds = mmq_lds(QT, NT, p.n_in, TR, p.hs);
    if (lds > g_lds_max) return set_error(ORC_E_UNSUPPORTED, "gemm: activations do not fit LDS");
    // a wave range staged in more than one window: the kernel with the
    // restaging path, which the other kernels do not carry (orc_mmq_win.hip)
    if constexpr (!MW) {
        if (!KS1 && p.hs < (p.n_in / 128 + kMW - 1) / kMW) return mmq_launch_windowed(QT, p0, s, ev);
    }
    if (ev.start)
        hipExtLaunchKernelGGL((k_mmq<QT, NT, TR, UW, SW, KS1, MW, WPE>), grid, dim3(kMWG), lds, s, ev.start, ev.stop, 0,
                              p);
    else
        hipLaunchKernelGGL((k_mmq<QT, NT, TR, UW, SW, KS1, MW, WPE>), grid, dim3(kMWG), lds, s, p);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

// Two tiles per wave (one activation read for both) once there are enough
// rows to keep every CU busy; SwiGLU always pairs a gate tile with its up tile.
// UW: units of a wave's range in flight at once (a ring over longer ranges
// and across tiles); SW: units staged per pass. Tall matrices (at least two
// tiles per wave of the whole GPU) give each wave whole tiles; the split
// depends on the shape only, never on the token count.
template <bool MW, int QT, int NT>
static int mmq_nt(const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    const int per_wave = (p.n_in / 128 + kMW - 1) / kMW;
    const bool two = QT != kMixK && (p.epi == ORC_EPI_SWIGLU || (QT == ORC_Q4_K && p.n_rows >= 32 * g_n_cu));
    // whole-tile mode by the shape alone (never for mixed launches: their
    // segments are split-tile sized)
    const bool tall = mmq_tall(QT, p);
    // (ring depth and staging width change no result; two-tile and wide-batch
    // shapes keep them small enough that nothing spills)
    if constexpr (QT != kMixK) {
        if constexpr (!mmq_wide<NT>()) {
            if (tall)
                return two ? mmq_shape<MW, QT, NT, 2, 4, 4, true>(p, s, ev) : mmq_shape<MW, QT, NT, 1, 6, 4, true>(p, s, ev);
        } else {  // the lo tile's registers: a shorter ring
            if (tall)
                return two ? mmq_shape<MW, QT, NT, 2, 2, 4, true>(p, s, ev) : mmq_shape<MW, QT, NT, 1, 6, 4, true>(p, s, ev);
        }
        if constexpr (mmq_wide<NT>()) {  // the lo tile's registers leave room for a ring of two
            if (two) return mmq_shape<MW, QT, NT, 2, 2, 4, false>(p, s, ev);
        } else {
            if (two) return mmq_shape<MW, QT, NT, 2, 3, 4, false>(p, s, ev);
        }
    }
    if constexpr (mmq_wide<NT>()) {
        return mmq_shape<MW, QT, NT, 1, 3, 4, false>(p, s, ev);
    } else {
        // a mixed Q|K|V of three units per wave (n_in 3072: 320 tiles at the
        // 3B shape) fits two workgroups per CU with a ring of two, so every
        // tile runs at once (measured at 5 tokens: 13.8 -> 12.4 us per launch)
        if constexpr (QT == kMixK && !MW) {
            if (per_wave <= 3 && 2 * mmq_lds(QT, NT, p.n_in, 1, 0) <= 160 * 1024)
                return mmq_shape<MW, QT, NT, 1, 2, 4, false, 4>(p, s, ev);
        }
        if (per_wave <= 3) return mmq_shape<MW, QT, NT, 1, 3, 4, false>(p, s, ev);
        if constexpr (NT > 4) return mmq_shape<MW, QT, NT, 1, 4, 4, false>(p, s, ev);
        else {
            if (per_wave <= 4) return mmq_shape<MW, QT, NT, 1, 4, 4, false>(p, s, ev);
            return mmq_shape<MW, QT, NT, 1, 4, 8, false>(p, s, ev);
        }
    }
}

template <bool MW, int QT>
static int mmq_type_launch(const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    switch (p.tok_block) {
        case 1: return mmq_nt<MW, QT, 1>(p, s, ev);
        case 2: return mmq_nt<MW, QT, 2>(p, s, ev);
        case 3: return mmq_nt<MW, QT, 3>(p, s, ev);
        case 4: return mmq_nt<MW, QT, 4>(p, s, ev);
        case 5: return mmq_nt<MW, QT, 5>(p, s, ev);
        case 6: return mmq_nt<MW, QT, 6>(p, s, ev);
        case 7: return mmq_nt<MW, QT, 7>(p, s, ev);
        case 8: return mmq_nt<MW, QT, 8>(p, s, ev);
        case 9: return mmq_nt<MW, QT, 9>(p, s, ev);
        case 10: return mmq_nt<MW, QT, 10>(p, s, ev);
        case 11: return mmq_nt<MW, QT, 11>(p, s, ev);
        case 12: return mmq_nt<MW, QT, 12>(p, s, ev);
        case 13: return mmq_nt<MW, QT, 13>(p, s, ev);
        case 14: return mmq_nt<MW, QT, 14>(p, s, ev);
        case 15: return mmq_nt<MW, QT, 15>(p, s, ev);
        case 16: return mmq_nt<MW, QT, 16>(p, s, ev);
        default: return set_error(ORC_E_UNSUPPORTED, "n_tok chunk must be 1..16");
    }
}

// The split-tile dispatch of one kernel set: MW = false holds the kernels of
// wave ranges staged in one window, MW = true those with the restaging path.
template <bool MW> int mmq_launch_t(int type, const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    switch (type) {
        case ORC_Q4_K: return mmq_type_launch<MW, ORC_Q4_K>(p, s, ev);
        case ORC_Q6_K: return mmq_type_launch<MW, ORC_Q6_K>(p, s, ev);
        case kMixK: return mmq_type_launch<MW, kMixK>(p, s, ev);
        default: return set_error(ORC_E_UNSUPPORTED, "gemm: not a matrix-core type");
    }
}

}  // namespace orc

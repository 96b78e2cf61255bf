// Quantized GEMM on the matrix cores for Q4_K and Q6_K blocks (gfx950): the
// (k+1)-token verify and the prefill of a Q4_K_M / Q6_K target, 2..16 tokens
// per token block and any number of blocks per launch (second grid
// dimension). One-token calls (decode) run the vector path in orc_gemm.hip.
//
// Replaces gemm_q (core/gguf_parser.cpp:919-997) for the K-quant types, with
// the RMSNorm prologue and the bias / residual / SwiGLU epilogues of
// Model::forward_prefill (core/model.cpp:565-643) fused in.
#include "orc_mmq_core.hpp"

#include <algorithm>
#include <type_traits>

namespace orc {

// ── prefill: 64 tokens per workgroup ────────────────────────────────────────
// Calls of at least kPfMinTok tokens (the batched prefill of
// Model::forward_prefill, core/model.cpp:510-674; verify passes are far
// smaller) on Q4_K or Q6_K weights. One workgroup of eight waves per (block of
// 128 rows, or of 128 SwiGLU gate / up row pairs, block of 64 tokens) walks
// every unit of its rows once: each wave decodes its row tile's slice (the
// same unit arithmetic as k_mmq: Q4_K scale folded into the codes, Q6_K
// codes split into exact hi / lo halves) and feeds it to the hi and the lo
// A tiles of four 16-token tiles (Q6_K: hi x hi, lo x hi and hi x lo; the
// lo x lo term is below 2^-22 of each product and dropped), so a weight
// byte is streamed once per 64 tokens instead of once per 16-token block. The activations of the next
// unit (64 tokens x 128 values) are loaded while this unit's MFMAs run, then
// split into hi / lo fp16 with a power of two per (unit, token) that keeps
// them in range (as k_mmq stages them) into the other of two LDS buffers;
// the Q4_K minimum term is the same 16x16x4 fp32 MFMA per unit and tile.
// A (token, row) sum runs over the units in order, one chain per unit
// scaled by d 2^-e: within fp32 rounding of k_mmq's, not equal to it bit for
// bit (calls below kPfMinTok tokens, which every verify pass is, keep k_mmq;
// the reference's own prefill and decode round differently as well).
constexpr int kPfTT = 4, kPfBM = 16 * kPfTT, kPfW = 8, kPfWG = 64 * kPfW;
// Internal epilogue of the second of a two-pass SwiGLU (Q8_0 prefill: one
// row tile per wave keeps the kernel inside its registers): the first pass
// stored g = gate rows, this one the up rows u: y = silu(y) * u, the fused
// epilogue's arithmetic.
constexpr int kEpiSwigluUp = 16;
constexpr int kPfABuf = 4 * 4 * 2 * kPfBM * 16;  // A bytes per unit: [slice][lane group][hi, lo][token] x 8 halves
constexpr size_t kPfLds = 2 * kPfABuf + (2 * kPfBM + 2 * kPfBM * 4 + kPfBM) * sizeof(float);

// B operand of slice i of a Q4_K unit: sc q in fp16 (exact; see mmq_core_q4k)
__device__ __forceinline__ h8v q4k_slice_b(const MUnit& M, int i, uint32_t sc4) {
    const uint32_t sc = (sc4 >> (8 * i)) & 0xFFu;
    const u32x2 src = (i >> 1) ? M.d : M.c;
    const int sh = 4 * (i & 1);
    const _Float16 f = (_Float16)(float)sc;
    const h2v scv{f, f}, off{(_Float16)(-1024.f * (float)sc), (_Float16)(-1024.f * (float)sc)};
    const uint32_t m4 = sreg(0x000F000Fu), mg = vreg(0x64006400u);
    const uint32_t r[4] = {((src.x >> sh) & m4) | mg, ((src.x >> (sh + 8)) & m4) | mg, ((src.y >> sh) & m4) | mg,
                           ((src.y >> (sh + 8)) & m4) | mg};
    u32x4 bq;
#pragma unroll
    for (int k = 0; k < 4; ++k) bq[k] = as_u32(__builtin_elementwise_fma(as_h2(r[k]), scv, off));
    return __builtin_bit_cast(h8v, bq);
}

// B operands of slice i of a Q6_K unit for lane group c: hi and exact lo
// halves of sc (q - 32) (see mmq_core_q6k)
__device__ __forceinline__ void q6k_slice_b(const MUnit& M, int i, int c, h8v& bhi, h8v& blo) {
    const u32x2 src = (i & 1) ? M.b : M.a;
    const int sh = 4 * (i >> 1);
    uint32_t r[4];
    switch (i) {  // the slice index as a constant of the helper
        case 0: q6k_magic<0>(src.x, M.c.x, sh, r[0], r[1]), q6k_magic<0>(src.y, M.c.y, sh, r[2], r[3]); break;
        case 1: q6k_magic<1>(src.x, M.c.x, sh, r[0], r[1]), q6k_magic<1>(src.y, M.c.y, sh, r[2], r[3]); break;
        case 2: q6k_magic<2>(src.x, M.c.x, sh, r[0], r[1]), q6k_magic<2>(src.y, M.c.y, sh, r[2], r[3]); break;
        default: q6k_magic<3>(src.x, M.c.x, sh, r[0], r[1]), q6k_magic<3>(src.y, M.c.y, sh, r[2], r[3]); break;
    }
    const int si = 2 * i + (c >> 1);
    const uint32_t sw = si < 4 ? M.d.x : M.d.y;
    const _Float16 sf = (_Float16)(float)(int8_t)((sw >> (8 * (si & 3))) & 0xFFu);
    const h2v sc2{sf, sf}, off{(_Float16)-1056.f, (_Float16)-1056.f};
    u32x4 bh, bl;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const h2v v = as_h2(r[k]) + off;
        const h2v hi = v * sc2;
        bh[k] = as_u32(hi);
        bl[k] = as_u32(__builtin_elementwise_fma(v, sc2, -hi));
    }
    bhi = __builtin_bit_cast(h8v, bh);
    blo = __builtin_bit_cast(h8v, bl);
}

// Q8_0 unit of 128 values (four 32-value blocks, core/gguf_parser.cpp:
// 1073-1082) for lane group c: codes 8c .. 8c + 7 of each block and the
// blocks' four fp16 scales, from the GGUF blocks or the regrouped
// ORC_Q8_0_X8 groups (the unit is half of a group: scales 4 (u & 1) ..,
// then their code runs).
struct Q8Unit {
    u32x2 q[4];
    u32x2 s;
    __device__ __forceinline__ void load(int type, const uint8_t* row, int u, int cg) {
        if (type == ORC_Q8_0_X8) {
            const uint8_t* grp = row + (size_t)(u >> 1) * 272;
            const int b0 = 4 * (u & 1);
            s = ldg8(grp + 2 * b0);
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = ldg8(grp + 16 + 32 * (b0 + i) + 8 * cg);
        } else {
            const uint8_t* blk = row + (size_t)(4 * u) * 34;
            s = u32x2{ldg2(blk) | (ldg2(blk + 34) << 16), ldg2(blk + 68) | (ldg2(blk + 102) << 16)};
#pragma unroll
            for (int i = 0; i < 4; ++i) q[i] = ldg8(blk + 34 * i + 2 + 8 * cg);
        }
    }
};

// B operand of block i of a Q8_0 unit: its 8 int8 codes, exact in fp16, in
// the A entries' element order (perm8): code bytes move up by 128 and into
// the low byte of fp16 1024 + b, then 1152 comes off
__device__ __forceinline__ h8v q8_slice_b(const Q8Unit& M, int i) {
    const uint32_t a = M.q[i].x ^ 0x80808080u, b = M.q[i].y ^ 0x80808080u;
    const uint32_t m = sreg(0x00FF00FFu), mg = vreg(0x64006400u);
    const uint32_t r[4] = {(a & m) | mg, ((a >> 8) & m) | mg, (b & m) | mg, ((b >> 8) & m) | mg};
    const h2v off{(_Float16)-1152.f, (_Float16)-1152.f};
    u32x4 bq;
#pragma unroll
    for (int k = 0; k < 4; ++k) bq[k] = as_u32(as_h2(r[k]) + off);
    return __builtin_bit_cast(h8v, bq);
}

// RT row tiles per wave: 1, or 2 for SwiGLU (a gate tile and its up tile)
template <int QT, int RT>
__global__ __launch_bounds__(kPfWG) void k_mmq_pf(QmvParams p) {
    static_assert(QT == ORC_Q4_K || QT == ORC_Q6_K || QT == ORC_Q8_0 || QT == ORC_Q8_0_X8, "one type per launch");
    constexpr bool Q8 = QT == ORC_Q8_0 || QT == ORC_Q8_0_X8;
    using UnitT = std::conditional_t<Q8, Q8Unit, MUnit>;
    extern __shared__ __attribute__((aligned(16))) uint8_t msm[];
    float* esc = (float*)(msm + 2 * kPfABuf);  // [2][token] 2^-e of the unit
    float* sxs = esc + 2 * kPfBM;               // [2][token][sub-block] sums of x g (Q4_K)
    float* irms = sxs + 2 * kPfBM * 4;          // [token] 1 / rms
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane >> 4, n = lane & 15;
    const int U = p.n_in / 128;
    const int t0 = blockIdx.y * kPfBM, nt = min(kPfBM, p.n_tok - t0);
    const bool swiglu = p.epi == ORC_EPI_SWIGLU, norm = p.norm_w != nullptr;
    const uint8_t *const sw0 = spin(p.w[0]), *const sw1 = spin(p.w[1]), *const sw2 = spin(p.w[2]);
    float *const sy0 = spin(p.y[0]), *const sy1 = spin(p.y[1]), *const sy2 = spin(p.y[2]);
    const float *const sb0 = spin(p.bias[0]), *const sb1 = spin(p.bias[1]), *const sb2 = spin(p.bias[2]);
    const int n_seg = p.n_seg, r0 = p.rows[0], r1 = p.rows[1];
    // the wave's weight rows (clamped to row 0 past the end: loads stay in bounds)
    const int jo = (blockIdx.x * kPfW + wave) * 16 + n;  // SwiGLU output row
    const uint8_t* rp[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) {
        int jl = swiglu ? rt * r0 + (jo < r0 ? jo : r0) : ((blockIdx.x * kPfW + wave) * RT + rt) * 16 + n;
        if (jl >= p.n_rows) jl = 0;
        int jj;
        const int sgi = seg_of(jl, n_seg, r0, r1, jj);
        rp[rt] = pick3(sgi, sw0, sw1, sw2) + (size_t)jj * p.row_bytes;
    }

    // staging: thread (token st, 16 values kk0..kk0+15 of slice si) per unit
    const int st = tid >> 3, si = (tid >> 1) & 3, hf = tid & 1, kk0 = 32 * si + 16 * hf;
    const bool st_in = st < nt;
    const float* xrow = p.x + (size_t)(t0 + (st_in ? st : 0)) * p.ldx + kk0;
    float4 xv[4], gv[4];
    float ssq = 0.f;
    auto st_load = [&](int u) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            xv[j] = st_in ? *(const float4*)(xrow + 128 * u + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
            gv[j] = norm ? *(const float4*)(p.norm_w + 128 * u + kk0 + 4 * j) : make_float4(1.f, 1.f, 1.f, 1.f);
        }
    };
    auto st_store = [&](int u, int b) {
        float v[16];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float xs[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w}, gs[4] = {gv[j].x, gv[j].y, gv[j].z, gv[j].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                ssq = __builtin_fmaf(xs[e], xs[e], ssq);
                v[4 * j + e] = xs[e] * gs[e];
            }
        }
        float mx = 0.f, s16 = 0.f;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            mx = fmaxf(mx, fabsf(v[e]));
            s16 += v[e];
        }
        mx = fmaxf(mx, dpp<0xB1>(mx));   // over the token's eight lanes
        mx = fmaxf(mx, dpp<0x4E>(mx));
        mx = fmaxf(mx, dpp<0x141>(mx));
        int e2 = 0;
        if (mx > 0.f && mx <= 3.0e38f) {
            int ex;
            (void)frexpf(mx, &ex);  // mx < 2^ex
            e2 = 14 - ex;
        }
        const float up = ldexpf(1.f, e2);
        const float s32 = s16 + dpp<0xB1>(s16);  // the slice's 32 values (two lanes)
        if ((tid & 7) == 0) esc[b * kPfBM + st] = ldexpf(1.f, -e2);
        if (hf == 0) sxs[(b * kPfBM + st) * 4 + si] = s32;
        uint8_t* ab = msm + b * kPfABuf;
#pragma unroll
        for (int g8 = 0; g8 < 2; ++g8) {
            h8v hi, lo;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float w = v[8 * g8 + e] * up;
                const _Float16 he = (_Float16)w;
                hi[perm8(e)] = he;
                lo[perm8(e)] = (_Float16)(w - (float)he);
            }
            const int cc = 2 * hf + g8;
            *(h8v*)(ab + (((si * 4 + cc) * 2 + 0) * kPfBM + st) * 16) = hi;
            *(h8v*)(ab + (((si * 4 + cc) * 2 + 1) * kPfBM + st) * 16) = lo;
        }
    };

    UnitT cur[RT], nxt[RT];
#pragma unroll
    for (int rt = 0; rt < RT; ++rt) cur[rt].load(QT, rp[rt], 0, c);
    st_load(0);
    st_store(0, 0);
    __syncthreads();
    f4v acc[kPfTT][RT];
#pragma unroll
    for (int tt = 0; tt < kPfTT; ++tt)
#pragma unroll
        for (int rt = 0; rt < RT; ++rt) acc[tt][rt] = f4v{0.f, 0.f, 0.f, 0.f};

    for (int u = 0; u < U; ++u) {
        const int b = u & 1;
        if (u + 1 < U) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) nxt[rt].load(QT, rp[rt], u + 1, c);
            st_load(u + 1);
        }
        const uint8_t* ab = msm + b * kPfABuf;
        f4v D[kPfTT][RT];
#pragma unroll
        for (int tt = 0; tt < kPfTT; ++tt)
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) D[tt][rt] = f4v{0.f, 0.f, 0.f, 0.f};
        if constexpr (Q8) {
            // a block per slice, each with its own scale: its two products
            // (hi and lo activations) are scaled into acc before the next;
            // one token tile at a time keeps few operands live
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h8v bq[RT];
                float dq[RT];
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    bq[rt] = q8_slice_b(cur[rt], i);
                    const uint32_t sw = (i >> 1) ? cur[rt].s.y : cur[rt].s.x;
                    dq[rt] = h2f((sw >> (16 * (i & 1))) & 0xFFFFu);
                }
#pragma unroll
                for (int tt = 0; tt < kPfTT; ++tt) {
                    const uint8_t* ap = ab + ((i * 4 + c) * 2 * kPfBM + tt * 16 + n) * 16;
                    const h8v ah = *(const h8v*)ap, al = *(const h8v*)(ap + kPfBM * 16);
                    const float4 es = *(const float4*)&esc[b * kPfBM + tt * 16 + 4 * c];
                    const float esv[4] = {es.x, es.y, es.z, es.w};
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt) {
                        f4v z = f4v{0.f, 0.f, 0.f, 0.f};
                        z = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bq[rt], z, 0, 0, 0);
                        z = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bq[rt], z, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[tt][rt][e] = __builtin_fmaf(dq[rt] * esv[e], z[e], acc[tt][rt][e]);
                    }
                }
            }
        } else {
        uint32_t sc4[RT], mn4[RT];
        if constexpr (QT == ORC_Q4_K) {
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) q4k_unit_sm(u & 1, cur[rt].a.y, cur[rt].b.x, cur[rt].b.y, sc4[rt], mn4[rt]);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            h8v bh[RT], bl[RT];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                if constexpr (QT == ORC_Q4_K) bh[rt] = q4k_slice_b(cur[rt], i, sc4[rt]);
                else q6k_slice_b(cur[rt], i, c, bh[rt], bl[rt]);
            }
            h8v ah[kPfTT], al[kPfTT];
#pragma unroll
            for (int tt = 0; tt < kPfTT; ++tt) {
                const uint8_t* ap = ab + ((i * 4 + c) * 2 * kPfBM + tt * 16 + n) * 16;
                ah[tt] = *(const h8v*)ap;
                al[tt] = *(const h8v*)(ap + kPfBM * 16);
            }
            // each product over every (token tile, row tile) accumulator in
            // turn, so consecutive MFMAs never wait on each other; Q6_K drops
            // the lo activations x lo codes term (below 2^-22 of each product)
#pragma unroll
            for (int tt = 0; tt < kPfTT; ++tt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    D[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[tt], bh[rt], D[tt][rt], 0, 0, 0);
#pragma unroll
            for (int tt = 0; tt < kPfTT; ++tt)
#pragma unroll
                for (int rt = 0; rt < RT; ++rt)
                    D[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al[tt], bh[rt], D[tt][rt], 0, 0, 0);
            if constexpr (QT == ORC_Q6_K) {
#pragma unroll
                for (int tt = 0; tt < kPfTT; ++tt)
#pragma unroll
                    for (int rt = 0; rt < RT; ++rt)
                        D[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[tt], bl[rt], D[tt][rt], 0, 0, 0);
            }
        }
        // acc += d 2^-e D (Q4_K: minus the unit's minimum terms, one MFMA)
#pragma unroll
        for (int tt = 0; tt < kPfTT; ++tt) {
            const float4 es = *(const float4*)&esc[b * kPfBM + tt * 16 + 4 * c];
            const float esv[4] = {es.x, es.y, es.z, es.w};
            float sxa = 0.f;
            if constexpr (QT == ORC_Q4_K) sxa = sxs[(b * kPfBM + tt * 16 + n) * 4 + c];
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) {
                if constexpr (QT == ORC_Q4_K) {
                    const float d = h2f(cur[rt].a.x & 0xFFFFu), dmin = h2f(cur[rt].a.x >> 16);
                    const float bm = -(dmin * (float)((mn4[rt] >> (8 * c)) & 0xFFu));
                    f4v t;
#pragma unroll
                    for (int e = 0; e < 4; ++e) t[e] = __builtin_fmaf(d * esv[e], D[tt][rt][e], acc[tt][rt][e]);
                    acc[tt][rt] = __builtin_amdgcn_mfma_f32_16x16x4f32(sxa, bm, t, 0, 0, 0);
                } else {
                    const float d = h2f(cur[rt].e);
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[tt][rt][e] = __builtin_fmaf(d * esv[e], D[tt][rt][e], acc[tt][rt][e]);
                }
            }
        }
        }
        if (u + 1 < U) {
            st_store(u + 1, b ^ 1);  // the other buffer: its readers passed the last barrier
#pragma unroll
            for (int rt = 0; rt < RT; ++rt) cur[rt] = nxt[rt];
        }
        __syncthreads();
    }

    // 1 / rms of each token: its eight staging lanes' sums of x^2 (fixed order)
    if (norm) {
        float ss = ssq + dpp<0xB1>(ssq);
        ss += dpp<0x4E>(ss);
        ss += dpp<0x141>(ss);
        if ((tid & 7) == 0) irms[st] = 1.f / sqrtf(ss / (float)p.n_in + p.eps);
        __syncthreads();
    }
    // epilogue: lane (c, n) holds tokens tt 16 + 4c + e of row tile rows n
#pragma unroll
    for (int tt = 0; tt < kPfTT; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int tl = tt * 16 + 4 * c + e;
            if (tl >= nt) continue;
            const float inv = norm ? irms[tl] : 1.f;
            const size_t to = (size_t)(t0 + tl) * p.ldy;
            if (swiglu) {
                if (jo < r0) {
                    const float g = acc[tt][0][e] * inv, v = acc[tt][RT - 1][e] * inv;
                    sy0[jo + to] = (g / (1.f + expf(-g))) * v;
                }
            } else {
#pragma unroll
                for (int rt = 0; rt < RT; ++rt) {
                    const int jl = ((blockIdx.x * kPfW + wave) * RT + rt) * 16 + n;
                    if (jl >= p.n_rows) continue;
                    int jj;
                    const int sgi = seg_of(jl, n_seg, r0, r1, jj);
                    float* y = pick3(sgi, sy0, sy1, sy2) + jj + to;
                    const float* bb = pick3(sgi, sb0, sb1, sb2);
                    float v = acc[tt][rt][e] * inv;
                    if (bb) v += bb[jj];
                    if (p.epi == ORC_EPI_ACCUM) {
                        *y += v;
                    } else if (p.epi == kEpiSwigluUp) {
                        const float g = *y;
                        *y = (g / (1.f + expf(-g))) * v;
                    } else {
                        *y = v;
                    }
                }
            }
        }
}

bool mmq_type(int type) { return type == ORC_Q4_K || type == ORC_Q6_K || type == kMixK; }

// tokens per launch: up to kMmqMaxNT as long as the activations fit: the
// smallest staging window (one four-unit pass per wave) in split-tile mode,
// every unit of the row in whole-tile mode, with the launch's tiles per wave
// (two for SwiGLU pairs and tall Q4_K matrices)
int mmq_max_tokens(int type, const QmvParams& p) {
    const int per_wave = (p.n_in / 128 + kMW - 1) / kMW;
    const int hs = mmq_tall(type, p) ? 0 : std::min(per_wave, 4);
    const bool two = type != kMixK && (p.epi == ORC_EPI_SWIGLU || (type == ORC_Q4_K && p.n_rows >= 32 * g_n_cu));
    const int tr = two ? 2 : 1;
    int nt = kMmqMaxNT;
    while (nt > 1 && mmq_lds(type, nt, p.n_in, tr, hs) > g_lds_max) --nt;
    return mmq_lds(type, nt, p.n_in, tr, hs) <= g_lds_max ? nt : 0;
}

bool mmq_prefill(int type, const QmvParams& p) {
    return (type == ORC_Q4_K || type == ORC_Q6_K || type == ORC_Q8_0 || type == ORC_Q8_0_X8) &&
           p.n_tok >= kPfMinTok && p.n_in % (type == ORC_Q8_0_X8 ? 256 : 128) == 0 &&
           (p.epi != ORC_EPI_SWIGLU || p.n_seg == 2) && kPfLds <= g_lds_max;
}

template <int QT, int RT> static int mmq_pf_shape(const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    const bool swiglu = p.epi == ORC_EPI_SWIGLU;
    const int rows_blk = swiglu ? kPfW * 16 : kPfW * RT * 16;
    const dim3 grid(((swiglu ? p.rows[0] : p.n_rows) + rows_blk - 1) / rows_blk, (p.n_tok + kPfBM - 1) / kPfBM);
    if (ev.start)
        hipExtLaunchKernelGGL((k_mmq_pf<QT, RT>), grid, dim3(kPfWG), kPfLds, s, ev.start, ev.stop, 0, p);
    else
        hipLaunchKernelGGL((k_mmq_pf<QT, RT>), grid, dim3(kPfWG), kPfLds, s, p);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

int mmq_prefill_launch(int type, const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    if (!mmq_prefill(type, p)) return set_error(ORC_E_INVALID, "gemm: not a prefill launch");
    const bool swiglu = p.epi == ORC_EPI_SWIGLU;
    if (type == ORC_Q4_K) return swiglu ? mmq_pf_shape<ORC_Q4_K, 2>(p, s, ev) : mmq_pf_shape<ORC_Q4_K, 1>(p, s, ev);
    if (type == ORC_Q6_K) return swiglu ? mmq_pf_shape<ORC_Q6_K, 2>(p, s, ev) : mmq_pf_shape<ORC_Q6_K, 1>(p, s, ev);
    // Q8_0: one row tile per wave; SwiGLU in two passes over the output
    // rows (gate stored, then the up rows' epilogue applies silu(g) * u)
    auto q8 = [&](const QmvParams& q) {
        return type == ORC_Q8_0 ? mmq_pf_shape<ORC_Q8_0, 1>(q, s, ev) : mmq_pf_shape<ORC_Q8_0_X8, 1>(q, s, ev);
    };
    if (!swiglu) return q8(p);
    QmvParams g = p;
    g.epi = ORC_EPI_STORE;
    g.n_seg = 1;
    g.n_rows = p.rows[0];
    g.bias[0] = g.bias[1] = nullptr;
    g.w[1] = nullptr;
    g.y[1] = nullptr;
    g.rows[1] = 0;
    if (int rc = q8(g)) return rc;
    QmvParams u = g;
    u.w[0] = p.w[1];
    u.epi = kEpiSwigluUp;
    return q8(u);
}

int mmq_launch(int type, const QmvParams& p, hipStream_t s, const LaunchEvents& ev) {
    return mmq_launch_t<false>(type, p, s, ev);
}

}  // namespace orc

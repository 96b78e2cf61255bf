// Transformer elementwise ops, GQA attention over the device KV cache, argmax
// and greedy acceptance (gfx950).
//
// Replaces ops::rmsnorm / ops::rope / ops::softmax / ops::argmax
// (core/ops.cpp:149-195, 386-497), the KV store and per-head attention loops
// of Model::forward (core/model.cpp:401-435) and Model::forward_prefill
// (core/model.cpp:595-626), and the acceptance step of the batched spec loop
// (benchmark/bench_engine.cpp:337-355).
#include "orc_internal.hpp"
#include <hip/hip_ext.h>

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <unordered_map>
#include <cfloat>

namespace orc {

// ── RMSNorm: one workgroup per row, the same reduction as the GEMM prologue ───
// Rows of a multiple of 4 floats are read as float4s; any other n (which the
// reference's scalar tail also takes, core/ops.cpp:149-195) one float per
// thread and step.
__global__ __launch_bounds__(256) void k_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
    __shared__ float red[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const bool v4 = (n & 3) == 0;
    const float* xr = x + (size_t)blockIdx.x * n;
    float* orow = out + (size_t)blockIdx.x * n;
    float ss = 0.f;
    if (v4) {
        for (int i = tid; i < n / 4; i += 256) {
            float4 v = ((const float4*)xr)[i];
            ss = __builtin_fmaf(v.x, v.x, ss);
            ss = __builtin_fmaf(v.y, v.y, ss);
            ss = __builtin_fmaf(v.z, v.z, ss);
            ss = __builtin_fmaf(v.w, v.w, ss);
        }
    } else {
        for (int i = tid; i < n; i += 256) ss = __builtin_fmaf(xr[i], xr[i], ss);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) red[wave] = ss;
    __syncthreads();
    const float s = 1.f / sqrtf(((red[0] + red[1]) + (red[2] + red[3])) / (float)n + eps);
    if (v4) {
        float4* o4 = (float4*)orow;
        const float4* w4 = (const float4*)w;
        for (int i = tid; i < n / 4; i += 256) {
            float4 v = ((const float4*)xr)[i], g = w4[i];
            o4[i] = make_float4((v.x * s) * g.x, (v.y * s) * g.y, (v.z * s) * g.z, (v.w * s) * g.w);
        }
    } else {
        for (int i = tid; i < n; i += 256) orow[i] = (xr[i] * s) * w[i];
    }
}

// ── Per-head RMSNorm of q and k (QK-norm) in place on QKV rows ───────────────
// One wave per (head, token): rows [q heads | k heads] of each token's QKV row
// [q (n_heads*hd) | k (n_kv*hd) | v], the q heads scaled by qw, the k heads by
// kw (head_dim weights each, shared by the heads). Sum of squares as one FMA
// chain per lane, then a fixed xor-butterfly; out = (x * s) * w, the order of
// ops::rmsnorm's store.
__global__ __launch_bounds__(256) void k_qk_norm(float* qkv, int ldqkv, int n_heads, int n_kv, int hd, const float* qw,
                                                 const float* kw, float eps) {
    const int lane = threadIdx.x & 63, h = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (h >= n_heads + n_kv) return;  // wave-uniform: the last workgroup's spare waves
    float* row = qkv + (size_t)blockIdx.y * ldqkv + (size_t)h * hd;
    const float* w = h < n_heads ? qw : kw;
    float v[2];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = lane + 64 * j;
        v[j] = i < hd ? row[i] : 0.f;
        ss = __builtin_fmaf(v[j], v[j], ss);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    const float s = 1.f / sqrtf(ss / (float)hd + eps);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int i = lane + 64 * j;
        if (i < hd) row[i] = (v[j] * s) * w[i];
    }
}

// ── RoPE on q,k + KV store. One workgroup per token. ─────────────────────────
// rope table: [pos][half] of (cos, sin); KV cache per layer: [n_kv][ctx][hd].
// The first position is *d_pos + pos_off (d_pos may be null): with a device
// position a captured graph stays valid while decoding advances.
__device__ __forceinline__ int start_position(const int* d_pos, int pos_off) { return (d_pos ? *d_pos : 0) + pos_off; }

__global__ __launch_bounds__(256) void k_rope_kv(float* qkv, int ldqkv, int n_heads, int n_kv, int hd,
                                                 const int* d_pos, int pos_off, const float2* rope, float* kc,
                                                 float* vc, int ctx) {
    const int t = blockIdx.x, pos = start_position(d_pos, pos_off) + t, half = hd / 2;
    if (pos < 0 || pos >= ctx) return;  // outside the cache: nothing to rotate or store
    float* row = qkv + (size_t)t * ldqkv;
    const float2* cs = rope + (size_t)pos * half;
    const int nrot = (n_heads + n_kv) * half;
    for (int i = threadIdx.x; i < nrot; i += blockDim.x) {
        const int h = i / half, k = i - h * half;
        float* v = row + h * hd;  // q heads then k heads are contiguous
        const float2 c = cs[k];
        const float a = v[k], b = v[k + half];
        v[k] = a * c.x - b * c.y;
        v[k + half] = a * c.y + b * c.x;
    }
    __syncthreads();
    const float* kr = row + n_heads * hd;
    const float* vr = kr + n_kv * hd;
    for (int i = threadIdx.x; i < n_kv * hd; i += blockDim.x) {
        const int g = i / hd, k = i - g * hd;
        const size_t o = ((size_t)g * ctx + pos) * hd + k;
        kc[o] = kr[i];
        vc[o] = vr[i];
    }
}

// ── GQA attention, split over KV chunks ──────────────────────────────────────
// Grid (chunk, kv head). A workgroup stages its KV chunk in LDS once and
// serves every query row of the group: n_gqa heads x n_tok tokens, processed
// in batches of RB rows. Per row it writes the chunk-local max m, sum l and
// unnormalized output O; k_attn_combine merges chunks (online softmax).
constexpr int kCH = 32, kRB = 16;

template <int HD>
__global__ __launch_bounds__(256) void k_attn_partial(const float* q, int ldq, int n_tok, int n_heads, int n_kv,
                                                      const int* d_pos, int pos_off, const float* kc, const float* vc,
                                                      int ctx, float* work) {
    __shared__ float Ks[kCH][HD + 4];
    __shared__ float Vs[kCH][HD];
    __shared__ float Qs[kRB][HD];
    __shared__ float Ps[kRB][kCH];
    const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int gqa = n_heads / n_kv;
    const int p0 = c * kCH;
    const int start_pos = start_position(d_pos, pos_off);
    const int pmax = min(start_pos + n_tok, ctx) - 1;
    if (p0 > pmax) return;  // chunk past the last position (grids sized for the whole context)
    const int np = min(kCH, pmax + 1 - p0);
    const float scale = 1.f / sqrtf((float)HD);
    const float* kg = kc + ((size_t)g * ctx + p0) * HD;
    const float* vg = vc + ((size_t)g * ctx + p0) * HD;
    for (int i = tid; i < kCH * HD / 4; i += 256) {
        const int p = i / (HD / 4), k = 4 * (i - p * (HD / 4));
        float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
        if (p < np) {
            kv = *(const float4*)(kg + (size_t)p * HD + k);
            vv = *(const float4*)(vg + (size_t)p * HD + k);
        }
        *(float4*)&Ks[p][k] = kv;
        *(float4*)&Vs[p][k] = vv;
    }
    const int nqr = gqa * n_tok;
    for (int rb = 0; rb < nqr; rb += kRB) {
        __syncthreads();
        for (int i = tid; i < kRB * HD; i += 256) {
            const int r = i / HD, k = i - r * HD, qr = rb + r;
            float v = 0.f;
            if (qr < nqr) {
                const int t = qr / gqa, h = g * gqa + (qr - t * gqa);
                v = q[(size_t)t * ldq + h * HD + k];
            }
            Qs[r][k] = v;
        }
        __syncthreads();
        for (int i = tid; i < kRB * kCH; i += 256) {
            const int r = i / kCH, p = i - r * kCH, qr = rb + r;
            float s = -INFINITY;
            if (qr < nqr && p < np && p0 + p <= start_pos + qr / gqa) {
                float d = 0.f;
#pragma unroll 8
                for (int k = 0; k < HD; k += 4) {
                    const float4 a = *(const float4*)&Qs[r][k], b = *(const float4*)&Ks[p][k];
                    d = __builtin_fmaf(a.x, b.x, d);
                    d = __builtin_fmaf(a.y, b.y, d);
                    d = __builtin_fmaf(a.z, b.z, d);
                    d = __builtin_fmaf(a.w, b.w, d);
                }
                s = d * scale;
            }
            Ps[r][p] = s;
        }
        __syncthreads();
        // row softmax pieces: 32 lanes per row, 8 rows per pass over 256 threads
        {
            const int r = tid >> 5, p = tid & 31;
            for (int rr = r; rr < kRB; rr += 8) {
                float s = Ps[rr][p];
                float m = s;
#pragma unroll
                for (int o = 16; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 32));
                const float e = (m == -INFINITY) ? 0.f : expf(s - m);
                float l = e;
#pragma unroll
                for (int o = 16; o >= 1; o >>= 1) l += __shfl_xor(l, o, 32);
                Ps[rr][p] = e;
                const int qr = rb + rr;
                if (p == 0 && qr < nqr) {
                    const int t = qr / gqa, h = g * gqa + (qr - t * gqa);
                    float* w = work + (((size_t)c * n_heads + h) * n_tok + t) * (HD + 2);
                    w[HD] = m;
                    w[HD + 1] = l;
                }
            }
        }
        __syncthreads();
        for (int i = tid; i < kRB * HD; i += 256) {
            const int r = i / HD, k = i - r * HD, qr = rb + r;
            if (qr >= nqr) continue;
            float o = 0.f;
            for (int p = 0; p < np; ++p) o = __builtin_fmaf(Ps[r][p], Vs[p][k], o);
            const int t = qr / gqa, h = g * gqa + (qr - t * gqa);
            work[(((size_t)c * n_heads + h) * n_tok + t) * (HD + 2) + k] = o;
        }
    }
}

template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(int n_tok, int n_heads, const int* d_pos, int pos_off, int ctx,
                                                     const float* work, float* out, int ldo) {
    const int h = blockIdx.x, t = blockIdx.y, k = threadIdx.x;
    const int last = min(start_position(d_pos, pos_off) + t, ctx - 1);
    const int nch = last / kCH + 1;  // chunks that hold positions <= start_pos + t
    float M = -INFINITY;
    for (int c = 0; c < nch; ++c) {
        const float* w = work + (((size_t)c * n_heads + h) * n_tok + t) * (HD + 2);
        if (w[HD + 1] > 0.f) M = fmaxf(M, w[HD]);
    }
    float L = 0.f, O = 0.f;
    for (int c = 0; c < nch; ++c) {
        const float* w = work + (((size_t)c * n_heads + h) * n_tok + t) * (HD + 2);
        const float l = w[HD + 1];
        if (!(l > 0.f)) continue;
        const float f = expf(w[HD] - M);
        L = __builtin_fmaf(l, f, L);
        O = __builtin_fmaf(w[k], f, O);
    }
    out[(size_t)t * ldo + h * HD + k] = O / L;
}

// ── fused RoPE + KV store + causal GQA attention, split over KV chunks ──────
// Grid (chunk c, kv head g, token t). Token t sits at position pt = start + t
// and attends to positions 0..pt (core/model.cpp:410-435, 604-626), cut into
// chunks of CP positions, CP a function of pt alone (so a token's result does
// not depend on how many tokens share the launch: a (k+1)-token verify pass
// equals k+1 decode steps bit for bit). A workgroup:
//  * rotates the gqa query heads of kv head g (ops::rope rotate-half pairs,
//    core/ops.cpp:440-485) into LDS;
//  * walks its chunk in sub-blocks of kSB positions: four lanes per position
//    form the scores from K rows (the cache, or for the batch's own positions
//    the QKV rows rotated in the lane, so no workgroup reads a cache row
//    another one is writing), an online softmax per head, then P.V with the
//    sub-block's V rows, which were loaded before the scores;
//  * the workgroup of the last chunk stores K (rotated) and V of position pt;
//  * writes its chunk's (O, m, l) per head to the workspace; k_attn_merge
//    (the next launch, so no fence is needed) merges the chunks in chunk
//    order: O = sum_c O_c e^(m_c - M) / sum_c l_c e^(m_c - M). A token whose
//    positions fit one chunk gets its output written directly.
constexpr int kSW = 256, kSB = 64, kNCMax = 256, kRMax = 8, kMaxTokAttn = 16;

__host__ __device__ inline int chunk_positions(int P) {
    const int per = (P + kNCMax - 1) / kNCMax;
    return (per + kSB - 1) / kSB * kSB;
}
__host__ __device__ inline int n_chunks(int P) { return (P + chunk_positions(P) - 1) / chunk_positions(P); }
// up to kMtMax positions the chunks are kSB long (k_attn_mt); above, wider (k_attn_split)
constexpr int kMtMax = kSB * kNCMax;

// Tokens attending to at most kWGMax positions take k_attn_wg (one launch,
// one workgroup per query head, at most three passes of its waves); longer
// ones the split over workgroups plus the merge, which keeps more CUs
// streaming K and V.
constexpr int kWGMax = 512;

struct LaunchEv {
    hipEvent_t a = nullptr, b = nullptr;
};
// waves of a k_attn_wg workgroup (head_dim 128: twelve, the most whose registers need no spill)
template <int HD> constexpr int wg_waves() { return HD == 128 ? 12 : 16; }

// rotate-half of the pair (a = x[i], b = x[i + hd/2]) by (cos, sin) = cs, with
// one fixed rounding sequence wherever a row is rotated
__device__ __forceinline__ float rot_lo(float a, float b, float2 cs) { return __builtin_fmaf(a, cs.x, -(b * cs.y)); }
__device__ __forceinline__ float rot_hi(float a, float b, float2 cs) { return __builtin_fmaf(b, cs.x, a * cs.y); }

// Rotates the nh query heads h0 .. h0 + nh - 1 of token t (at position pt)
// into Qs[r][d] with NTH threads; every load of a thread's entries is issued
// before the first is used.
template <int HD, int RM, int NTH>
__device__ __forceinline__ void rope_q_lds(float (&Qs)[RM][HD], const float* qkv, int ldqkv, int t, int h0, int nh,
                                           int pt, const float2* rope, int tid) {
    constexpr int half = HD / 2, QI = (RM * HD + NTH - 1) / NTH;
    const int R = nh;
    const float* qt = qkv + (size_t)t * ldqkv + (size_t)h0 * HD;
    const float2* cr = rope + (size_t)pt * half;
    float a[QI], b[QI];
    float2 cs[QI];
#pragma unroll
    for (int j = 0; j < QI; ++j) {
        const int i = tid + j * NTH;
        if (i < R * HD) {
            const int r = i / HD, d = i - r * HD, dl = d < half ? d : d - half;
            a[j] = qt[r * HD + dl];
            b[j] = qt[r * HD + dl + half];
            cs[j] = cr[dl];
        }
    }
#pragma unroll
    for (int j = 0; j < QI; ++j) {
        const int i = tid + j * NTH;
        if (i < R * HD) {
            const int r = i / HD, d = i - r * HD;
            Qs[r][d] = d < half ? rot_lo(a[j], b[j], cs[j]) : rot_hi(a[j], b[j], cs[j]);
        }
    }
}

// rope_q_lds in two steps: load issues every load of the thread's entries,
// store rotates them into Qs (same arithmetic), so other loads can be issued
// in between.
template <int HD, int RM, int NTH> struct QRot {
    static constexpr int half = HD / 2, QI = (RM * HD + NTH - 1) / NTH;
    float a[QI], b[QI];
    float2 cs[QI];
    int R = 0;
    __device__ __forceinline__ void load(const float* qkv, int ldqkv, int t, int h0, int nh, int pt,
                                         const float2* rope, int tid) {
        R = nh;
        const float* qt = qkv + (size_t)t * ldqkv + (size_t)h0 * HD;
        const float2* cr = rope + (size_t)pt * half;
#pragma unroll
        for (int j = 0; j < QI; ++j) {
            const int i = tid + j * NTH;
            if (i < R * HD) {
                const int r = i / HD, d = i - r * HD, dl = d < half ? d : d - half;
                a[j] = qt[r * HD + dl];
                b[j] = qt[r * HD + dl + half];
                cs[j] = cr[dl];
            }
        }
    }
    __device__ __forceinline__ void store(float (&Qs)[RM][HD], int tid) const {
#pragma unroll
        for (int j = 0; j < QI; ++j) {
            const int i = tid + j * NTH;
            if (i < R * HD) {
                const int r = i / HD, d = i - r * HD;
                Qs[r][d] = d < half ? rot_lo(a[j], b[j], cs[j]) : rot_hi(a[j], b[j], cs[j]);
            }
        }
    }
};

// floats per partial row: O[HD], m, l, padded to whole 128-byte lines
template <int HD> constexpr int part_stride() { return HD + 32; }

template <int HD, int RS>
__global__ __launch_bounds__(kSW) void k_attn_split(const float* qkv, int ldqkv, int n_heads, int n_kv,
                                                    const int* d_pos, int pos_off, const float2* rope, float* kc,
                                                    float* vc, int ctx, float* out, int ldo, float* work) {
    constexpr int half = HD / 2;
    constexpr int FL = HD / 16;     // float4 of a K row per lane (four lanes per position)
    constexpr int NC = HD / 4;      // float4 columns in the P.V phase
    constexpr int NPS = kSW / NC;   // position subsets in the P.V phase
    constexpr int VPL = kSB / NPS;  // V rows per lane per sub-block
    constexpr int PS = part_stride<HD>();
    static_assert(kSB * 4 == kSW, "four lanes per position");
    __shared__ __align__(16) float Qs[RS][HD];
    __shared__ float S[RS][kSB];
    __shared__ float st_m[RS], st_l[RS], st_a[RS];
    constexpr int kRB = RS < 4 ? RS : 4;  // heads per pass of the final reduction
    __shared__ __align__(16) float red[kRB][NPS][HD];
    // workgroup = (chunk c, heads rw0 .. rw0 + RH - 1 of kv head g, token t)
    const int R = n_heads / n_kv, nbh = (R + RS - 1) / RS;
    const int c = blockIdx.x, g = blockIdx.y / nbh, t = blockIdx.z, tid = threadIdx.x;
    const int rw0 = (blockIdx.y - g * nbh) * RS, RH = min(RS, R - rw0);
    const int start = start_position(d_pos, pos_off);
    const int pt = start + t;
    if (pt < 0 || pt >= ctx) return;  // outside the cache (graph replays past the end): nothing to do
    const int P = pt + 1, CP = chunk_positions(P), nch = n_chunks(P);
    if (P <= kMtMax || c >= nch) return;  // shorter contexts: k_attn_wg, k_attn_mt; grids cover the most chunks any position needs
    const int p0 = c * CP, p1 = min(P, p0 + CP);
    const float scale = 1.f / sqrtf((float)HD);
    const size_t kvh = (size_t)(n_heads + g) * HD, vvh = (size_t)(n_heads + n_kv + g) * HD;
    const float* kg = kc + (size_t)g * ctx * HD;
    const float* vg = vc + (size_t)g * ctx * HD;
    const int sp = tid >> 2, sl = tid & 3;    // score phase: position in the sub-block, lane of four
    const int col = tid % NC, ps = tid / NC;  // P.V phase: float4 column, position subset

    // K row of position p as float4s sl + 4 j (the pair partner of float4 j <
    // FL/2 is float4 j + FL/2 of the same lane); zero past the chunk
    auto load_k = [&](float4 (&k)[FL], int p, bool valid) {
        if (!valid) {
#pragma unroll
            for (int j = 0; j < FL; ++j) k[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        } else if (p < start) {
            const float* src = kg + (size_t)p * HD;
#pragma unroll
            for (int j = 0; j < FL; ++j) k[j] = *(const float4*)(src + 4 * (sl + 4 * j));
        } else {
            const float* src = qkv + (size_t)(p - start) * ldqkv + kvh;
            const float2* cs = rope + (size_t)p * half;
#pragma unroll
            for (int j = 0; j < FL; ++j) k[j] = *(const float4*)(src + 4 * (sl + 4 * j));
#pragma unroll
            for (int j = 0; j < FL / 2; ++j) {
                const int f = sl + 4 * j;
                const float4 c01 = *(const float4*)(cs + 4 * f), c23 = *(const float4*)(cs + 4 * f + 2);
                const float4 a = k[j], b = k[j + FL / 2];
                const float2 e0{c01.x, c01.y}, e1{c01.z, c01.w}, e2{c23.x, c23.y}, e3{c23.z, c23.w};
                k[j] = make_float4(rot_lo(a.x, b.x, e0), rot_lo(a.y, b.y, e1), rot_lo(a.z, b.z, e2), rot_lo(a.w, b.w, e3));
                k[j + FL / 2] =
                    make_float4(rot_hi(a.x, b.x, e0), rot_hi(a.y, b.y, e1), rot_hi(a.z, b.z, e2), rot_hi(a.w, b.w, e3));
            }
        }
    };

    // the first sub-block's V rows and this lane's share of its K row go out
    // first; the later sub-blocks' are loaded at the end of the one before
    float4 v[VPL], k[FL];
    auto load_v = [&](int b0, int nb) {
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int pp = ps + NPS * j, p = b0 + pp;
            if (pp >= nb) v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
            else if (p < start) v[j] = *(const float4*)(vg + (size_t)p * HD + 4 * col);
            else v[j] = *(const float4*)(qkv + (size_t)(p - start) * ldqkv + vvh + 4 * col);
        }
    };
    load_v(p0, min(kSB, p1 - p0));
    load_k(k, p0 + sp, sp < min(kSB, p1 - p0));

    // this token's K (rotated) and V at pt go to the cache, from the last chunk
    if (c == nch - 1 && rw0 == 0 && tid < HD) {
        const float* kr = qkv + (size_t)t * ldqkv + kvh;
        const float2* cs = rope + (size_t)pt * half;
        const int d = tid;
        const float v = d < half ? rot_lo(kr[d], kr[d + half], cs[d]) : rot_hi(kr[d - half], kr[d], cs[d - half]);
        const size_t o = ((size_t)g * ctx + pt) * HD + d;
        kc[o] = v;
        vc[o] = qkv[(size_t)t * ldqkv + vvh + d];
    }
    rope_q_lds<HD, RS, kSW>(Qs, qkv, ldqkv, t, g * R + rw0, RH, pt, rope, tid);
    if (tid < RS) {
        st_m[tid] = -INFINITY;
        st_l[tid] = 0.f;
    }
    float4 acc[RS];
#pragma unroll
    for (int r = 0; r < RS; ++r) acc[r] = make_float4(0.f, 0.f, 0.f, 0.f);

    for (int b0 = p0; b0 < p1; b0 += kSB) {
        const int nb = min(kSB, p1 - b0);
        __syncthreads();  // Qs written (first sub-block); S and st_a consumed (later ones)
        // scores: each lane's partial dot over its FL float4s, summed over the four lanes
        float dr[RS];
#pragma unroll
        for (int r = 0; r < RS; ++r) {
            float s = 0.f;
            if (r < RH) {
#pragma unroll
                for (int j = 0; j < FL; ++j) {
                    const float4 q = *(const float4*)&Qs[r][4 * (sl + 4 * j)];
                    s = __builtin_fmaf(q.x, k[j].x, s);
                    s = __builtin_fmaf(q.y, k[j].y, s);
                    s = __builtin_fmaf(q.z, k[j].z, s);
                    s = __builtin_fmaf(q.w, k[j].w, s);
                }
                s = quad_sum(s);
            }
            dr[r] = s;
        }
        if (sl == 0) {
#pragma unroll
            for (int r = 0; r < RS; ++r)
                if (r < RH) S[r][sp] = sp < nb ? dr[r] * scale : -INFINITY;
        }
        // the next sub-block's K rows, in flight during the softmax and P.V
        const int b1 = b0 + kSB;
        if (b1 < p1) load_k(k, b1 + sp, sp < min(kSB, p1 - b1));
        __syncthreads();
        // online softmax over the sub-block: wave w owns heads w, w + 4
        {
            const int w = tid >> 6, ln = tid & 63;
            for (int r = w; r < RH; r += kSW / 64) {
                const float s = S[r][ln];
                float m = s;
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
                const float m_old = st_m[r];
                const float m_new = fmaxf(m_old, m);
                const float e = ln < nb ? expf(s - m_new) : 0.f;
                S[r][ln] = e;
                float l = e;
#pragma unroll
                for (int o = 32; o >= 1; o >>= 1) l += __shfl_xor(l, o, 64);
                if (ln == 0) {
                    const float a = m_old == -INFINITY ? 0.f : expf(m_old - m_new);
                    st_a[r] = a;
                    st_l[r] = st_l[r] * a + l;
                    st_m[r] = m_new;
                }
            }
        }
        __syncthreads();
        // O_r = a_r O_r + sum_p e_r[p] V[p]
#pragma unroll
        for (int r = 0; r < RS; ++r) {
            if (r < RH) {
                const float a = st_a[r];
                acc[r].x *= a;
                acc[r].y *= a;
                acc[r].z *= a;
                acc[r].w *= a;
            }
        }
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const int pp = ps + NPS * j;
            if (pp < nb) {
#pragma unroll
                for (int r = 0; r < RS; ++r) {
                    if (r < RH) {
                        const float e = S[r][pp];
                        acc[r].x = __builtin_fmaf(e, v[j].x, acc[r].x);
                        acc[r].y = __builtin_fmaf(e, v[j].y, acc[r].y);
                        acc[r].z = __builtin_fmaf(e, v[j].z, acc[r].z);
                        acc[r].w = __builtin_fmaf(e, v[j].w, acc[r].w);
                    }
                }
            }
        }
        if (b1 < p1) load_v(b1, min(kSB, p1 - b1));
    }

    // sum the position subsets in a fixed order: the output (one chunk) or
    // this chunk's partial row
    const bool single = nch == 1;
    float* part = work + ((size_t)t * n_kv + g) * kNCMax * R * PS;
    // heads in batches of kRB through the LDS; each sum runs over k = 0..NPS-1
#pragma unroll
    for (int r0 = 0; r0 < RS; r0 += kRB) {
        if (r0 >= RH) break;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kRB; ++j)
            if (r0 + j < RH) *(float4*)&red[j][ps][4 * col] = acc[r0 + j];
        __syncthreads();
        for (int i = tid; i < kRB * HD; i += kSW) {
            const int j = i / HD, dd = i - j * HD, r = r0 + j;
            if (r >= RH) break;
            float o = 0.f;
#pragma unroll
            for (int k = 0; k < NPS; ++k) o += red[j][k][dd];
            if (single) {
                out[(size_t)t * ldo + (g * R + rw0 + r) * HD + dd] = o / st_l[r];
            } else {
                float* pr = part + ((size_t)c * R + rw0 + r) * PS;
                pr[dd] = o;
                if (dd == 0) {
                    pr[HD] = st_m[r];
                    pr[HD + 1] = st_l[r];
                }
            }
        }
    }
}

// ── positions kWGMax < P <= kMtMax: every token of a launch in one pass ────
// One workgroup per (chunk of kSB positions, kv head g) forms the partial
// (O, m, l) of every (token, query head) row that reads the chunk, so each
// cached K / V byte is read once per launch however many tokens verify. The
// rows (token-major, NR = tokens x gqa heads, padded to whole 16-row tiles)
// are a small dense contraction, done on the matrix cores in fp32
// (v_mfma_f32_16x16x4_f32: fp32 operands and sums):
//  * scores S = Q K^T: wave w holds the K rows of positions 16w..16w+15 of
//    the chunk as the B operand (lane group kg = lane / 16 holds dims
//    [kg HD/8, (kg+1) HD/8) and the same range + HD/2, so the rotate-half
//    pairs of the batch's own positions rotate in the lane); step m of the
//    HD/4-step chain sums dim(m, kg) over the four lane groups; A = the
//    rotated query rows from LDS;
//  * softmax of each row over the chunk on the VALU (four lanes per row),
//    e written back over the scores;
//  * O = E V: wave w owns output dims [w HD/4, (w+1) HD/4); step m of the
//    16-step chain sums positions kg*16 + m; B = the V rows from the cache
//    (or the QKV rows of the batch's own positions), A = e from LDS.
// The order of every sum is fixed by the position and the chunk alone, and a
// row's result depends on its own query alone (masked positions enter as
// exact zeros), so an n-token call equals n one-token calls bit for bit.
// Tokens past kMtMax positions take k_attn_split (wider chunks); each token's
// path depends on its own position only.
constexpr int kQPad = 4, kSPad = 4;  // LDS row padding (floats) against bank conflicts
typedef float mt_f4 __attribute__((ext_vector_type(4)));
// dynamic LDS floats of k_attn_mt for nr rows: rotated queries, scores / e
template <int HD> constexpr size_t mt_lds_floats(int nr) {
    return (size_t)((nr + 15) / 16 * 16) * (HD + kQPad + kSB + kSPad);
}

template <int HD>
__global__ __launch_bounds__(kSW) void k_attn_mt(const float* qkv, int ldqkv, int n_tok, int n_heads, int n_kv,
                                                 const int* d_pos, int pos_off, const float2* rope, float* kc,
                                                 float* vc, int ctx, float* work) {
    constexpr int half = HD / 2, E8 = HD / 8, KPL = HD / 4;  // dims per lane-group block; K values per lane
    constexpr int CT = HD / 64;                              // 16-dim output tiles per wave
    constexpr int QS = HD + kQPad, SS = kSB + kSPad, PS = part_stride<HD>();
    static_assert(kSW == 256 && kSB == 64, "four waves, 16 positions each");
    extern __shared__ __align__(16) float lds[];
    const int R = n_heads / n_kv;
    const int c = blockIdx.x, g = blockIdx.y, tid = threadIdx.x;
    const int w = tid >> 6, ln = tid & 63, li = ln & 15, kg = ln >> 4;
    const int start = start_position(d_pos, pos_off);
    const int p0 = c * kSB;
    // tokens reading this chunk on this path: kWGMax < P_t <= kMtMax,
    // p0 < P_t, P_t = start + t + 1 <= ctx; they are consecutive
    const int t_hi = min(n_tok - 1, min(ctx, kMtMax) - 1 - start);
    const int t_lo = max(0, max(kWGMax, p0) - start);
    if (t_hi < t_lo) return;
    const int NR = (t_hi - t_lo + 1) * R, NRP = (NR + 15) & ~15;
    float* Qs = lds;                   // [NRP][QS]
    float* S = lds + (size_t)NRP * QS;  // [NRP][SS]
    const float scale = 1.f / sqrtf((float)HD);
    const size_t kvh = (size_t)(n_heads + g) * HD, vvh = (size_t)(n_heads + n_kv + g) * HD;
    const float* kg_c = kc + (size_t)g * ctx * HD;
    const float* vg_c = vc + (size_t)g * ctx * HD;
    const int p_end = start + t_hi + 1;  // positions [p0, p_end) hold data the rows read

    // B operand of the scores: K of position p0 + 16w + li, dims [kg E8, +E8) and + half
    float kb[KPL];
    {
        const int p = p0 + 16 * w + li;
        if (p >= p_end) {
#pragma unroll
            for (int i = 0; i < KPL; ++i) kb[i] = 0.f;
        } else if (p < start) {
            const float* src = kg_c + (size_t)p * HD + kg * E8;
#pragma unroll
            for (int i = 0; i < E8; i += 4) {
                const float4 lo = *(const float4*)(src + i), hi = *(const float4*)(src + half + i);
                kb[i] = lo.x, kb[i + 1] = lo.y, kb[i + 2] = lo.z, kb[i + 3] = lo.w;
                kb[E8 + i] = hi.x, kb[E8 + i + 1] = hi.y, kb[E8 + i + 2] = hi.z, kb[E8 + i + 3] = hi.w;
            }
        } else {
            const float* src = qkv + (size_t)(p - start) * ldqkv + kvh + kg * E8;
            const float2* cs = rope + (size_t)p * half + kg * E8;
#pragma unroll
            for (int i = 0; i < E8; i += 4) {
                const float4 lo = *(const float4*)(src + i), hi = *(const float4*)(src + half + i);
                const float4 c01 = *(const float4*)(cs + i), c23 = *(const float4*)(cs + i + 2);
                const float2 e0{c01.x, c01.y}, e1{c01.z, c01.w}, e2{c23.x, c23.y}, e3{c23.z, c23.w};
                kb[i] = rot_lo(lo.x, hi.x, e0), kb[i + 1] = rot_lo(lo.y, hi.y, e1);
                kb[i + 2] = rot_lo(lo.z, hi.z, e2), kb[i + 3] = rot_lo(lo.w, hi.w, e3);
                kb[E8 + i] = rot_hi(lo.x, hi.x, e0), kb[E8 + i + 1] = rot_hi(lo.y, hi.y, e1);
                kb[E8 + i + 2] = rot_hi(lo.z, hi.z, e2), kb[E8 + i + 3] = rot_hi(lo.w, hi.w, e3);
            }
        }
    }
    // B operand of P.V: V[p0 + 16 kg + m][w HD/4 + 16 ct + li]
    float vb[CT][16];
#pragma unroll
    for (int m = 0; m < 16; ++m) {
        const int p = p0 + 16 * kg + m;
        const float* src = p >= p_end ? nullptr
                           : p < start ? vg_c + (size_t)p * HD
                                       : qkv + (size_t)(p - start) * ldqkv + vvh;
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) vb[ct][m] = src ? src[w * (HD / 4) + 16 * ct + li] : 0.f;
    }

    // K (rotated) and V of the tokens whose own position lies in this chunk go to the cache
    {
        const int tw = min(t_hi, p0 + kSB - 1 - start) - t_lo + 1;
        for (int i = tid; i < tw * HD; i += kSW) {
            const int t = t_lo + i / HD, d = i % HD, pt = start + t;
            const float* kr = qkv + (size_t)t * ldqkv + kvh;
            const float2* cs = rope + (size_t)pt * half;
            const float kv = d < half ? rot_lo(kr[d], kr[d + half], cs[d]) : rot_hi(kr[d - half], kr[d], cs[d - half]);
            const size_t o = ((size_t)g * ctx + pt) * HD + d;
            kc[o] = kv;
            vc[o] = qkv[(size_t)t * ldqkv + vvh + d];
        }
    }

    // rotated queries of every row (rope_q_lds's arithmetic): an item is four
    // dims of the first half and their rotate-half partners for one token;
    // its rope pairs are loaded once and applied to the token's R query heads
    // (every head's loads in flight first). Padded rows are zero.
    {
        constexpr int QD = half / 4;  // items per token
        const int ntk = t_hi - t_lo + 1;
        for (int i = tid; i < ntk * QD; i += kSW) {
            const int ti = i / QD, d = 4 * (i - ti * QD), t = t_lo + ti;
            const float* qt = qkv + (size_t)t * ldqkv + (size_t)g * R * HD + d;
            const float2* cs = rope + (size_t)(start + t) * half + d;
            const float4 c01 = *(const float4*)cs, c23 = *(const float4*)(cs + 2);
            float4 lo[kRMax], hi[kRMax];
#pragma unroll
            for (int h = 0; h < kRMax; ++h)
                if (h < R) {
                    lo[h] = *(const float4*)(qt + (size_t)h * HD);
                    hi[h] = *(const float4*)(qt + (size_t)h * HD + half);
                }
            const float2 e0{c01.x, c01.y}, e1{c01.z, c01.w}, e2{c23.x, c23.y}, e3{c23.z, c23.w};
#pragma unroll
            for (int h = 0; h < kRMax; ++h)
                if (h < R) {
                    float* qr = Qs + (size_t)(ti * R + h) * QS;
                    *(float4*)&qr[d] = make_float4(rot_lo(lo[h].x, hi[h].x, e0), rot_lo(lo[h].y, hi[h].y, e1),
                                                   rot_lo(lo[h].z, hi[h].z, e2), rot_lo(lo[h].w, hi[h].w, e3));
                    *(float4*)&qr[half + d] = make_float4(rot_hi(lo[h].x, hi[h].x, e0), rot_hi(lo[h].y, hi[h].y, e1),
                                                          rot_hi(lo[h].z, hi[h].z, e2), rot_hi(lo[h].w, hi[h].w, e3));
                }
        }
        for (int i = NR * (HD / 4) + tid; i < NRP * (HD / 4); i += kSW) {
            const int row = i / (HD / 4), d = 4 * (i - row * (HD / 4));
            *(float4*)&Qs[(size_t)row * QS + d] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    __syncthreads();

    // scores of 16-row tiles against this wave's 16 positions
    for (int rt = 0; rt < NRP / 16; ++rt) {
        const float* q = Qs + (size_t)(rt * 16 + li) * QS + kg * E8;
        float qa[KPL];
#pragma unroll
        for (int i = 0; i < E8; i += 4) {
            const float4 lo = *(const float4*)(q + i), hi = *(const float4*)(q + half + i);
            qa[i] = lo.x, qa[i + 1] = lo.y, qa[i + 2] = lo.z, qa[i + 3] = lo.w;
            qa[E8 + i] = hi.x, qa[E8 + i + 1] = hi.y, qa[E8 + i + 2] = hi.z, qa[E8 + i + 3] = hi.w;
        }
        mt_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < KPL; ++m) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[m], kb[m], acc, 0, 0, 0);
        const int pos = 16 * w + li;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = rt * 16 + 4 * kg + r;
            if (row < NR) {
                const int nb = min(kSB, start + t_lo + row / R + 1 - p0);
                S[(size_t)row * SS + pos] = pos < nb ? acc[r] * scale : -INFINITY;
            }
        }
    }
    __syncthreads();

    // softmax of each row over the chunk: four lanes per row, sixteen
    // positions per lane (max and sum in position order, then over the four
    // lanes by DPP in a fixed order); (m, l) go to the row's partial; padded
    // rows get e = 0
    for (int row0 = 0; row0 < NRP; row0 += kSW / 4) {
        const int row = row0 + (tid >> 2), q4 = tid & 3;
        if (row < NRP) {  // whole quads: the DPP exchanges stay inside active quads
            float* sr = S + (size_t)row * SS + 16 * q4;
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; i += 4) {
                const float4 v4 = *(const float4*)(sr + i);
                x[i] = v4.x, x[i + 1] = v4.y, x[i + 2] = v4.z, x[i + 3] = v4.w;
            }
            const int ti = row / R, t = t_lo + ti;
            const int nb = row < NR ? min(kSB, start + t + 1 - p0) : 0;
            float mx = x[0];
#pragma unroll
            for (int i = 1; i < 16; ++i) mx = fmaxf(mx, x[i]);
            mx = fmaxf(mx, dpp<0xB1>(mx));
            mx = fmaxf(mx, dpp<0x4E>(mx));
            float l = 0.f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                x[i] = 16 * q4 + i < nb ? expf(x[i] - mx) : 0.f;
                l += x[i];
            }
            l = quad_sum(l);
#pragma unroll
            for (int i = 0; i < 16; i += 4) *(float4*)(sr + i) = make_float4(x[i], x[i + 1], x[i + 2], x[i + 3]);
            if (q4 == 0 && row < NR) {
                float* pr = work + (((size_t)t * n_kv + g) * kNCMax * R + (size_t)c * R + (row - ti * R)) * PS;
                pr[HD] = mx;
                pr[HD + 1] = l;
            }
        }
    }
    __syncthreads();

    // O = E V per 16-row tile and this wave's output dims, into the partial rows
    for (int rt = 0; rt < NRP / 16; ++rt) {
        const float* e = S + (size_t)(rt * 16 + li) * SS + 16 * kg;
        float ea[16];
#pragma unroll
        for (int m = 0; m < 16; m += 4) {
            const float4 x = *(const float4*)(e + m);
            ea[m] = x.x, ea[m + 1] = x.y, ea[m + 2] = x.z, ea[m + 3] = x.w;
        }
        mt_f4 acc[CT];
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) {
            acc[ct] = mt_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < 16; ++m) acc[ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(ea[m], vb[ct][m], acc[ct], 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = rt * 16 + 4 * kg + r;
            if (row < NR) {
                const int ti = row / R, t = t_lo + ti;
                float* pr = work + (((size_t)t * n_kv + g) * kNCMax * R + (size_t)c * R + (row - ti * R)) * PS;
#pragma unroll
                for (int ct = 0; ct < CT; ++ct) pr[w * (HD / 4) + 16 * ct + li] = acc[ct][r];
            }
        }
    }
}

// ── prefill attention: 16-token query blocks, no partials ───────────────────
// orc_attn_prefill (prompt passes, host positions): one workgroup per (block
// of kPaTok tokens, kv head g) carries the block's kPaTok x gqa rows
// (token-major) through every kSB-position key chunk up to the block's last
// position with an online softmax (running max and sum per row in LDS), so
// there are no partial rows and no merge launch, and a chunk's K / V rows are
// read once per query block. Per chunk, as in k_attn_mt: scores on fp32
// MFMA chains (wave w: positions 16w..16w+15 of the chunk), the causal mask
// (key p <= the row's own position), the softmax update four lanes per row
// (rows whose chunk is all masked keep their state: factor 1, e = 0), then
// O = a O + E V on the matrix cores (wave w: output dims [w HD/4, (w+1)
// HD/4)). The next chunk's K rows are loaded after the scores and its V rows
// after P.V; the batch's own positions come from the QKV rows, rotated when
// used. Different rounding from the decode path (one online softmax over all
// chunks instead of per-chunk partials), as the reference's prefill and
// decode differ: within fp32 rounding of the exact attention.
constexpr int kPaTok = 16;
template <int HD> constexpr size_t pa_lds_bytes(int R) {
    const size_t nrp = (size_t)kPaTok * R;
    return (nrp * (HD + kQPad) + 2 * nrp * (kSB + kSPad) + 4 * nrp) * sizeof(float);
}

template <int HD>
__global__ __launch_bounds__(kSW) void k_attn_pf(const float* qkv, int ldqkv, int n_tok, int n_heads, int n_kv,
                                                 int start, const float2* rope, float* kc, float* vc, int ctx,
                                                 float* out, int ldo) {
    constexpr int half = HD / 2, E8 = HD / 8, KPL = HD / 4, CT = HD / 64;
    constexpr int QS = HD + kQPad, SS = kSB + kSPad;
    static_assert(kSW == 256 && kSB == 64, "four waves, 16 positions each");
    extern __shared__ __align__(16) float lds[];
    const int R = n_heads / n_kv;
    const int t0 = blockIdx.x * kPaTok, g = blockIdx.y, tid = threadIdx.x;
    const int w = tid >> 6, ln = tid & 63, li = ln & 15, kg = ln >> 4;
    const int nt = min(kPaTok, n_tok - t0), NR = nt * R, NRP = kPaTok * R;
    float* Qs = lds;                          // [NRP][QS] rotated queries
    float* S = Qs + (size_t)NRP * QS;         // [2][NRP][SS] scores, then e (chunk parity)
    float* m_run = S + 2 * (size_t)NRP * SS;  // [NRP] running max
    float* l_run = m_run + NRP;               // [NRP] running sum
    float* a_row = l_run + NRP;               // [2][NRP] rescale factor of the chunk
    const float scale = 1.f / sqrtf((float)HD);
    const size_t kvh = (size_t)(n_heads + g) * HD, vvh = (size_t)(n_heads + n_kv + g) * HD;
    const float* kg_c = kc + (size_t)g * ctx * HD;
    const float* vg_c = vc + (size_t)g * ctx * HD;
    const int p_end = start + t0 + nt;  // keys [0, p_end) hold data the rows read
    const int nch = (p_end + kSB - 1) / kSB;

    // K rows of chunk c (B operand of the scores; lane: position 16w + li,
    // dims [kg E8, +E8) and + half), raw; rows of the batch's own positions
    // also carry their rope pairs and are rotated when used
    float kb[KPL];
    float2 kcs[E8];
    bool krot = false;
    auto load_k = [&](int c) {
        const int p = c * kSB + 16 * w + li;
        krot = false;
        if (p >= p_end) {
#pragma unroll
            for (int i = 0; i < KPL; ++i) kb[i] = 0.f;
            return;
        }
        const float* src = p < start ? kg_c + (size_t)p * HD + kg * E8 : qkv + (size_t)(p - start) * ldqkv + kvh + kg * E8;
#pragma unroll
        for (int i = 0; i < E8; i += 4) {
            const float4 lo = *(const float4*)(src + i), hi = *(const float4*)(src + half + i);
            kb[i] = lo.x, kb[i + 1] = lo.y, kb[i + 2] = lo.z, kb[i + 3] = lo.w;
            kb[E8 + i] = hi.x, kb[E8 + i + 1] = hi.y, kb[E8 + i + 2] = hi.z, kb[E8 + i + 3] = hi.w;
        }
        if (p >= start) {
            krot = true;
            const float2* cs = rope + (size_t)p * half + kg * E8;
#pragma unroll
            for (int i = 0; i < E8; ++i) kcs[i] = cs[i];
        }
    };
    // V rows of chunk c (B operand of P.V: V[p0 + 16 kg + m][w HD/4 + 16 ct + li])
    float vb[CT][16];
    auto load_v = [&](int c) {
#pragma unroll
        for (int m = 0; m < 16; ++m) {
            const int p = c * kSB + 16 * kg + m;
            const float* src = p >= p_end ? nullptr
                               : p < start ? vg_c + (size_t)p * HD
                                           : qkv + (size_t)(p - start) * ldqkv + vvh;
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) vb[ct][m] = src ? src[w * (HD / 4) + 16 * ct + li] : 0.f;
        }
    };
    load_k(0);
    load_v(0);

    // K (rotated) and V of the block's tokens go to the cache
    for (int i = tid; i < nt * HD; i += kSW) {
        const int t = t0 + i / HD, d = i % HD, pt = start + t;
        const float* kr = qkv + (size_t)t * ldqkv + kvh;
        const float2* cs = rope + (size_t)pt * half;
        const float kv = d < half ? rot_lo(kr[d], kr[d + half], cs[d]) : rot_hi(kr[d - half], kr[d], cs[d - half]);
        const size_t o = ((size_t)g * ctx + pt) * HD + d;
        kc[o] = kv;
        vc[o] = qkv[(size_t)t * ldqkv + vvh + d];
    }
    // rotated queries of the block's rows (rope_q_lds's arithmetic; padded rows zero), running state
    {
        constexpr int QD = half / 4;
        for (int i0 = 0; i0 < NRP * QD; i0 += 4 * kSW) {
            float4 lo[4], hi[4], c01[4], c23[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = i0 + tid + j * kSW, row = i / QD, d = 4 * (i - row * QD);
                if (row < NR) {
                    const int ti = row / R, t = t0 + ti;
                    const float* qt = qkv + (size_t)t * ldqkv + (size_t)(g * R + row - ti * R) * HD + d;
                    const float2* cs = rope + (size_t)(start + t) * half + d;
                    lo[j] = *(const float4*)qt;
                    hi[j] = *(const float4*)(qt + half);
                    c01[j] = *(const float4*)cs;
                    c23[j] = *(const float4*)(cs + 2);
                }
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int i = i0 + tid + j * kSW, row = i / QD, d = 4 * (i - row * QD);
                if (row < NRP) {
                    float4 ql = make_float4(0.f, 0.f, 0.f, 0.f), qh = ql;
                    if (row < NR) {
                        const float2 e0{c01[j].x, c01[j].y}, e1{c01[j].z, c01[j].w};
                        const float2 e2{c23[j].x, c23[j].y}, e3{c23[j].z, c23[j].w};
                        ql = make_float4(rot_lo(lo[j].x, hi[j].x, e0), rot_lo(lo[j].y, hi[j].y, e1),
                                         rot_lo(lo[j].z, hi[j].z, e2), rot_lo(lo[j].w, hi[j].w, e3));
                        qh = make_float4(rot_hi(lo[j].x, hi[j].x, e0), rot_hi(lo[j].y, hi[j].y, e1),
                                         rot_hi(lo[j].z, hi[j].z, e2), rot_hi(lo[j].w, hi[j].w, e3));
                    }
                    *(float4*)&Qs[(size_t)row * QS + d] = ql;
                    *(float4*)&Qs[(size_t)row * QS + half + d] = qh;
                }
            }
        }
        for (int row = tid; row < NRP; row += kSW) {
            m_run[row] = -INFINITY;
            l_run[row] = 0.f;
        }
    }
    mt_f4 o[kRMax][CT];  // O of row tile rt (rows 16 rt + 4 kg + r), this wave's columns
#pragma unroll
    for (int rt = 0; rt < kRMax; ++rt)
#pragma unroll
        for (int ct = 0; ct < CT; ++ct) o[rt][ct] = mt_f4{0.f, 0.f, 0.f, 0.f};
    __syncthreads();

    for (int c = 0; c < nch; ++c) {
        const int b = c & 1, p0 = c * kSB;
        float* Sb = S + (size_t)b * NRP * SS;
        if (krot) {  // the batch's own positions: rotate-half with the position's rope pairs
#pragma unroll
            for (int i = 0; i < E8; ++i) {
                const float a = kb[i], h = kb[E8 + i];
                kb[i] = rot_lo(a, h, kcs[i]);
                kb[E8 + i] = rot_hi(a, h, kcs[i]);
            }
        }
        // scores of every row tile against this wave's 16 positions, causal mask
#pragma unroll
        for (int rt = 0; rt < kRMax; ++rt) {
            if (rt >= R) break;
            const float* q = Qs + (size_t)(rt * 16 + li) * QS + kg * E8;
            float qa[KPL];
#pragma unroll
            for (int i = 0; i < E8; i += 4) {
                const float4 lo = *(const float4*)(q + i), hi = *(const float4*)(q + half + i);
                qa[i] = lo.x, qa[i + 1] = lo.y, qa[i + 2] = lo.z, qa[i + 3] = lo.w;
                qa[E8 + i] = hi.x, qa[E8 + i + 1] = hi.y, qa[E8 + i + 2] = hi.z, qa[E8 + i + 3] = hi.w;
            }
            mt_f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int m = 0; m < KPL; ++m) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[m], kb[m], acc, 0, 0, 0);
            const int pos = 16 * w + li;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = rt * 16 + 4 * kg + r;
                const bool ok = row < NR && p0 + pos <= start + t0 + row / R;
                Sb[(size_t)row * SS + pos] = ok ? acc[r] * scale : -INFINITY;
            }
        }
        if (c + 1 < nch) load_k(c + 1);
        __syncthreads();
        // online softmax update, four lanes per row (sixteen positions each)
        for (int row0 = 0; row0 < NRP; row0 += kSW / 4) {
            const int row = row0 + (tid >> 2), q4 = tid & 3;
            if (row < NRP) {  // whole quads
                float* sr = Sb + (size_t)row * SS + 16 * q4;
                float x[16];
#pragma unroll
                for (int i = 0; i < 16; i += 4) {
                    const float4 v4 = *(const float4*)(sr + i);
                    x[i] = v4.x, x[i + 1] = v4.y, x[i + 2] = v4.z, x[i + 3] = v4.w;
                }
                float mx = x[0];
#pragma unroll
                for (int i = 1; i < 16; ++i) mx = fmaxf(mx, x[i]);
                mx = fmaxf(mx, dpp<0xB1>(mx));
                mx = fmaxf(mx, dpp<0x4E>(mx));
                const float m_old = m_run[row], m_new = fmaxf(m_old, mx);
                const bool live = m_new != -INFINITY;  // padded rows stay all -inf
                const float a = live && m_old != -INFINITY ? expf(m_old - m_new) : 0.f;
                float l = 0.f;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    x[i] = live && x[i] != -INFINITY ? expf(x[i] - m_new) : 0.f;
                    l += x[i];
                }
                l = quad_sum(l);
#pragma unroll
                for (int i = 0; i < 16; i += 4) *(float4*)(sr + i) = make_float4(x[i], x[i + 1], x[i + 2], x[i + 3]);
                if (q4 == 0) {
                    l_run[row] = __builtin_fmaf(l_run[row], a, l);
                    m_run[row] = m_new;
                    a_row[b * NRP + row] = a;
                }
            }
        }
        __syncthreads();
        // O = a O + E V
#pragma unroll
        for (int rt = 0; rt < kRMax; ++rt) {
            if (rt >= R) break;
            const float* e = Sb + (size_t)(rt * 16 + li) * SS + 16 * kg;
            float ea[16];
#pragma unroll
            for (int m = 0; m < 16; m += 4) {
                const float4 x = *(const float4*)(e + m);
                ea[m] = x.x, ea[m + 1] = x.y, ea[m + 2] = x.z, ea[m + 3] = x.w;
            }
            const float4 av = *(const float4*)&a_row[b * NRP + rt * 16 + 4 * kg];
            const float ar[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
            for (int ct = 0; ct < CT; ++ct) {
#pragma unroll
                for (int r = 0; r < 4; ++r) o[rt][ct][r] *= ar[r];
#pragma unroll
                for (int m = 0; m < 16; ++m)
                    o[rt][ct] = __builtin_amdgcn_mfma_f32_16x16x4f32(ea[m], vb[ct][m], o[rt][ct], 0, 0, 0);
            }
        }
        if (c + 1 < nch) load_v(c + 1);
    }
    __syncthreads();
    // O / l into the output rows
#pragma unroll
    for (int rt = 0; rt < kRMax; ++rt) {
        if (rt >= R) break;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = rt * 16 + 4 * kg + r;
            if (row >= NR) continue;
            const int ti = row / R, t = t0 + ti, h = g * R + row - ti * R;
            const float L = l_run[row];
#pragma unroll
            for (int ct = 0; ct < CT; ++ct)
                out[(size_t)t * ldo + (size_t)h * HD + w * (HD / 4) + 16 * ct + li] = o[rt][ct][r] / L;
        }
    }
}

// Merge of the chunk partials of k_attn_mt / k_attn_split: one workgroup of
// kMG threads per (query head, token). Every thread loads one chunk's (m, l)
// and forms e^(m_c - M) in parallel (M = the maximum, which no order
// changes). The sums O = sum_c O_c e^(m_c - M) and L = sum_c l_c e^(m_c - M)
// then run in chunk order: up to kSerialMerge chunks in one lane per output
// dimension (L in one more lane); above, the kMG / HD lanes of a dimension
// each take a contiguous range of the chunks (at most eight at C5's 8 K
// positions: one batch of loads) and their sums are added in range order.
// Either way the order depends on the token's position alone. Tokens with a
// single chunk were written directly and are skipped.
constexpr int kSerialMerge = 8, kMG = 1024;  // serial up to one batch of loads; threads of a merge workgroup
template <int HD>
__global__ __launch_bounds__(kMG) void k_attn_merge(int n_heads, int n_kv, const int* d_pos, int pos_off, int ctx,
                                                    const float* work, float* out, int ldo) {
    constexpr int PS = part_stride<HD>(), S = kMG / HD;
    static_assert(kNCMax <= kMG, "one chunk per thread");
    static_assert(S >= 2, "a lane outside the output dimensions sums L in serial merges");
    __shared__ float sf[kNCMax], sl[kNCMax];  // e^(m_c - M), l_c
    __shared__ float smax[kMG / 64], sLq[S];
    __shared__ __align__(16) float so[S][HD];
    const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int R = n_heads / n_kv, g = h / R, r = h - g * R;
    const int pt = start_position(d_pos, pos_off) + t;
    if (pt < 0 || pt >= ctx) return;
    const int P = pt + 1, nch = n_chunks(P);
    if (P <= kWGMax || nch == 1) return;
    const size_t cs = (size_t)R * PS;  // floats from one chunk's row of this head to the next chunk's
    const float* part = work + ((size_t)t * n_kv + g) * kNCMax * cs + (size_t)r * PS;
    float mc = -INFINITY;
    if (tid < nch) {
        mc = part[tid * cs + HD];
        sl[tid] = part[tid * cs + HD + 1];
    }
    float M = mc;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    if (lane == 0) smax[w] = M;
    __syncthreads();
    M = smax[0];
#pragma unroll
    for (int i = 1; i < kMG / 64; ++i) M = fmaxf(M, smax[i]);
    if (tid < nch) sf[tid] = expf(mc - M);
    __syncthreads();
    const bool serial = nch <= kSerialMerge;
    const int d = tid % HD, q = tid / HD;
    int c0 = 0, c1 = nch;  // this lane's chunk range
    if (!serial) {
        c0 = q * nch / S;
        c1 = (q + 1) * nch / S;
    } else if (q) {
        c1 = 0;
    }
    float O = 0.f;
    {
        int c = c0;
        for (; c + 8 <= c1; c += 8) {  // eight loads in flight, then the eight FMAs in chunk order
            float v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = part[(c + j) * cs + d];
#pragma unroll
            for (int j = 0; j < 8; ++j) O = __builtin_fmaf(v[j], sf[c + j], O);
        }
        for (; c < c1; ++c) O = __builtin_fmaf(part[c * cs + d], sf[c], O);
    }
    if (serial ? tid == HD : d == 0) {  // L over all chunks, or over this lane group's range
        const int l0 = serial ? 0 : c0, l1 = serial ? nch : c1;
        float L = 0.f;
        for (int c = l0; c < l1; ++c) L = __builtin_fmaf(sl[c], sf[c], L);
        sLq[serial ? 0 : q] = L;
    }
    if (!serial) so[q][d] = O;
    __syncthreads();
    if (tid < HD) {
        float L = sLq[0];
        if (!serial) {
            O = so[0][d];
#pragma unroll
            for (int i = 1; i < S; ++i) {
                O += so[i][d];
                L += sLq[i];
            }
        }
        out[(size_t)t * ldo + h * HD + d] = O / L;
    }
}

// ── short contexts: all positions of a (query heads, token) in one workgroup ─
// Tokens attending to at most kWGMax positions: one workgroup of kWW waves per
// (RM query heads of kv head g, token t); the launch uses RM = 1, so the
// per-pass chains carry one head and the grid holds n_heads x n_tok
// workgroups (each head's arithmetic is the same whatever RM is). Wave w takes positions [w CPW, (w + 1) CPW) with
// CPW = ceil(P / waves), a function of the position alone (so an n-token call
// still equals n one-token calls bit for bit), in passes of 16: four lanes
// per position form the scores (K rows from the cache, or for the batch's
// own positions the QKV rows rotated in the lane), the wave keeps its own
// online softmax (max and sum by lane exchanges over the 16 positions), and
// each lane accumulates P.V for HD/64 dims from the pass's V rows, which were
// loaded before the scores. The waves' (O, m, l) are merged through LDS in
// wave order: one launch, no workspace, no fence.
template <int HD, int RM>
__global__ __launch_bounds__(wg_waves<HD>() * 64) void k_attn_wg(const float* qkv, int ldqkv, int n_heads, int n_kv, const int* d_pos,
                                                 int pos_off, const float2* rope, float* kc, float* vc, int ctx,
                                                 float* out, int ldo) {
    constexpr int half = HD / 2, FL = HD / 16, DPL = HD / 64;
    constexpr int kWW = wg_waves<HD>(), kWT = kWW * 64;
    __shared__ __align__(16) float Qs[RM][HD];
    __shared__ __align__(16) float Es[kWW][RM][16];  // a pass's exp(s - m) per wave, head, position
    __shared__ __align__(16) float Ow[kWW][RM][HD];
    __shared__ float mw[kWW][RM], lw[kWW][RM];
    // workgroup = (kv head g, heads r0 .. r0 + RH - 1 of its group, token t)
    const int R = n_heads / n_kv;
    // kv head g = blockIdx.x % n_kv: consecutive workgroup ids go to the 8
    // XCDs in turn, so with 8 kv heads (and a grid width a multiple of 8)
    // every workgroup reading kv head g's K / V runs on one XCD and shares
    // its L2 instead of fetching the rows into several
    const int g = blockIdx.x % n_kv, r0 = (blockIdx.x / n_kv) * RM, RH = min(RM, R - r0);
    const int t = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int start = start_position(d_pos, pos_off);
    const int pt = start + t;
    if (pt < 0 || pt >= ctx) return;  // outside the cache (graph replays past the end): nothing to do
    const int P = pt + 1;
    if (P > kWGMax) return;  // split over workgroups instead
    const float scale = 1.f / sqrtf((float)HD);
    const size_t kvh = (size_t)(n_heads + g) * HD, vvh = (size_t)(n_heads + n_kv + g) * HD;
    const float* kg = kc + (size_t)g * ctx * HD;
    const float* vg = vc + (size_t)g * ctx * HD;
    const int sp = lane >> 2, sl = lane & 3;

    // this token's K (rotated) and V at pt go to the cache, from the group's
    // first workgroup
    if (r0 == 0 && tid < HD) {
        const float* kr = qkv + (size_t)t * ldqkv + kvh;
        const float2* cs = rope + (size_t)pt * half;
        const int d = tid;
        const float v = d < half ? rot_lo(kr[d], kr[d + half], cs[d]) : rot_hi(kr[d - half], kr[d], cs[d - half]);
        const size_t o = ((size_t)g * ctx + pt) * HD + d;
        kc[o] = v;
        vc[o] = qkv[(size_t)t * ldqkv + vvh + d];
    }
    // the query heads' loads go out first (rotated into the LDS below)
    QRot<HD, RM, kWT> qrot;
    qrot.load(qkv, ldqkv, t, g * R + r0, RH, pt, rope, tid);
    const int CPW = (P + kWW - 1) / kWW;
    const int p0 = w * CPW, p1 = min(P, p0 + CPW);

    // K row of position p as this lane's FL float4s (float4 sl + 4 j; its
    // pair partner is float4 j + FL/2 of the same lane); zero when invalid
    auto load_k = [&](float4 (&k)[FL], int p, bool valid) {
        if (!valid) {
#pragma unroll
            for (int j = 0; j < FL; ++j) k[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        } else if (p < start) {
            const float* src = kg + (size_t)p * HD;
#pragma unroll
            for (int j = 0; j < FL; ++j) k[j] = *(const float4*)(src + 4 * (sl + 4 * j));
        } else {
            const float* src = qkv + (size_t)(p - start) * ldqkv + kvh;
            const float2* cs = rope + (size_t)p * half;
#pragma unroll
            for (int j = 0; j < FL; ++j) k[j] = *(const float4*)(src + 4 * (sl + 4 * j));
#pragma unroll
            for (int j = 0; j < FL / 2; ++j) {
                const int f = sl + 4 * j;
                const float4 c01 = *(const float4*)(cs + 4 * f), c23 = *(const float4*)(cs + 4 * f + 2);
                const float4 a = k[j], b = k[j + FL / 2];
                const float2 e0{c01.x, c01.y}, e1{c01.z, c01.w}, e2{c23.x, c23.y}, e3{c23.z, c23.w};
                k[j] = make_float4(rot_lo(a.x, b.x, e0), rot_lo(a.y, b.y, e1), rot_lo(a.z, b.z, e2), rot_lo(a.w, b.w, e3));
                k[j + FL / 2] =
                    make_float4(rot_hi(a.x, b.x, e0), rot_hi(a.y, b.y, e1), rot_hi(a.z, b.z, e2), rot_hi(a.w, b.w, e3));
            }
        }
    };

    float m[RM], l[RM], O[RM][DPL];
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
#pragma unroll
        for (int k = 0; k < DPL; ++k) O[r][k] = 0.f;
    }
    // V of a pass's positions (this lane's DPL dims) and its K rows; head_dim
    // 64 (at most two passes: 16 waves, 512 positions) holds both passes'
    // rows, so the second pass's loads are in flight with the first
    constexpr bool PF = HD == 64;
    static_assert(!PF || kWGMax <= 2 * 16 * kWW, "head_dim 64: at most two passes per wave");
    float vv[16][DPL], vv2[PF ? 16 : 1][DPL];
    float4 k[FL], k2[PF ? FL : 1];
    auto load_pass = [&](auto& vb, auto& kb, int b0, int nb) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int p = b0 + j;
            const float* src = p < start ? vg + (size_t)p * HD : qkv + (size_t)(p - start) * ldqkv + vvh;
#pragma unroll
            for (int kk = 0; kk < DPL; ++kk) vb[j][kk] = 0.f;
            if (j < nb) {
                if constexpr (DPL == 2) {
                    const float2 v2 = *(const float2*)(src + 2 * lane);
                    vb[j][0] = v2.x;
                    vb[j][1] = v2.y;
                } else {
                    vb[j][0] = src[lane];
                }
            }
        }
        load_k(kb, b0 + sp, sp < nb);
    };
    // the first pass's loads are in flight while the query heads are rotated
    if (p0 < p1) load_pass(vv, k, p0, min(16, p1 - p0));
    if constexpr (PF) {
        if (p0 + 16 < p1) load_pass(vv2, k2, p0 + 16, min(16, p1 - p0 - 16));
    }
    qrot.store(Qs, tid);
    __syncthreads();  // Qs written
    for (int b0 = p0; b0 < p1; b0 += 16) {
        const int nb = min(16, p1 - b0);
        if (b0 != p0) {
            if constexpr (PF) {  // the second pass (the last one at head_dim 64): its rows are loaded
#pragma unroll
                for (int j = 0; j < 16; ++j)
#pragma unroll
                    for (int kk = 0; kk < DPL; ++kk) vv[j][kk] = vv2[j][kk];
#pragma unroll
                for (int j = 0; j < FL; ++j) k[j] = k2[j];
            } else {
                load_pass(vv, k, b0, nb);
            }
        }
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            if (r >= RH) break;
            float sc = 0.f;
#pragma unroll
            for (int j = 0; j < FL; ++j) {
                const float4 q = *(const float4*)&Qs[r][4 * (sl + 4 * j)];
                sc = __builtin_fmaf(q.x, k[j].x, sc);
                sc = __builtin_fmaf(q.y, k[j].y, sc);
                sc = __builtin_fmaf(q.z, k[j].z, sc);
                sc = __builtin_fmaf(q.w, k[j].w, sc);
            }
            sc = sp < nb ? quad_sum(sc) * scale : -INFINITY;
            // max and sum over the pass's 16 positions (lanes 4 apart)
            float mx = sc;
#pragma unroll
            for (int o = 4; o <= 32; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
            const float m_new = fmaxf(m[r], mx);
            const float a = m[r] == -INFINITY ? 0.f : expf(m[r] - m_new);
            const float e = sp < nb ? expf(sc - m_new) : 0.f;
            float es = e;
#pragma unroll
            for (int o = 4; o <= 32; o <<= 1) es += __shfl_xor(es, o, 64);
            l[r] = l[r] * a + es;
            m[r] = m_new;
#pragma unroll
            for (int kk = 0; kk < DPL; ++kk) O[r][kk] *= a;
            if (sl == 0) Es[w][r][sp] = e;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int r = 0; r < RM; ++r) {
            if (r >= RH) break;
            float ev[16];
#pragma unroll
            for (int j4 = 0; j4 < 4; ++j4) *(float4*)&ev[4 * j4] = *(const float4*)&Es[w][r][4 * j4];
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (j < nb) {
#pragma unroll
                    for (int kk = 0; kk < DPL; ++kk) O[r][kk] = __builtin_fmaf(ev[j], vv[j][kk], O[r][kk]);
                }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // the wave's partial results, then the merge in wave order
#pragma unroll
    for (int r = 0; r < RM; ++r) {
        if (r >= RH) break;
#pragma unroll
        for (int kk = 0; kk < DPL; ++kk) Ow[w][r][DPL * lane + kk] = O[r][kk];
        if (lane == 0) {
            mw[w][r] = m[r];
            lw[w][r] = l[r];
        }
    }
    __syncthreads();
    for (int i = tid; i < RH * HD; i += kWT) {
        const int r = i / HD, d = i - r * HD;
        float M = -INFINITY;
        for (int v = 0; v < kWW; ++v) M = fmaxf(M, mw[v][r]);
        float L = 0.f, o = 0.f;
        for (int v = 0; v < kWW; ++v) {
            if (mw[v][r] == -INFINITY) continue;  // a wave without positions
            const float f = expf(mw[v][r] - M);
            L = __builtin_fmaf(lw[v][r], f, L);
            o = __builtin_fmaf(Ow[v][r][d], f, o);
        }
        out[(size_t)t * ldo + (g * R + r0 + r) * HD + d] = o / L;
    }
}

// ── argmax (first index of the maximum) ──────────────────────────────────────
constexpr int kArgBlock = 1024;  // elements per stage-1 workgroup slice x 4

struct VI { float v; int i; };
__device__ __forceinline__ VI vi_max(VI a, VI b) {
    // larger value wins; equal values -> lower index (the reference scans
    // left to right with a strict '>')
    if (b.v > a.v || (b.v == a.v && b.i < a.i)) return b;
    return a;
}
__device__ __forceinline__ VI wave_vi_max(VI a) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        VI b{__shfl_xor(a.v, o, 64), __shfl_xor(a.i, o, 64)};
        a = vi_max(a, b);
    }
    return a;
}

__global__ __launch_bounds__(256) void k_argmax1(const float* x, int n, int ld, int n_slices, VI* part) {
    __shared__ VI red[4];
    const int row = blockIdx.y, s = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (size_t)row * ld;
    const int per = (n + n_slices - 1) / n_slices;
    const int b = s * per, e = min(n, b + per);
    VI best{-INFINITY, 0x7FFFFFFF};
    for (int i = b + tid; i < e; i += 256) best = vi_max(best, VI{xr[i], i});
    best = wave_vi_max(best);
    if ((tid & 63) == 0) red[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) part[(size_t)row * n_slices + s] = vi_max(vi_max(red[0], red[1]), vi_max(red[2], red[3]));
}

__global__ __launch_bounds__(64) void k_argmax2(const VI* part, int n_slices, int32_t* out) {
    const int row = blockIdx.x;
    VI best{-INFINITY, 0x7FFFFFFF};
    for (int i = threadIdx.x; i < n_slices; i += 64) best = vi_max(best, part[(size_t)row * n_slices + i]);
    best = wave_vi_max(best);
    if (threadIdx.x == 0) out[row] = best.i == 0x7FFFFFFF ? 0 : best.i;
}

__global__ void k_accept_greedy(const int32_t* tgt, const int32_t* dft, int n_draft, int32_t* out, int32_t* pos,
                                int32_t* next) {
    if (threadIdx.x != 0) return;
    int a = 0;
    while (a < n_draft && tgt[a] == dft[a]) ++a;
    out[0] = a;
    out[1] = tgt[a];
    if (pos) {  // device-resident round state: emitted ids, next position, next input
        for (int i = 0; i <= a; ++i) out[2 + i] = tgt[i];
        *pos += a + 1;
        *next = tgt[a];
    }
}

// One captured greedy step ends here: the argmax of the step (tok[1]) is
// appended to the history and becomes the next input; position and count
// advance on the device.
__global__ void k_decode_advance(int32_t* tok, int32_t* hist, int32_t* pos, int32_t* count) {
    if (threadIdx.x != 0) return;
    const int32_t t = tok[1];
    hist[*count] = t;
    *count += 1;
    *pos += 1;
    tok[0] = t;
}

}  // namespace orc

using namespace orc;

extern "C" int orc_rmsnorm(float* d_out, const float* d_x, const float* d_w, int n, int n_rows, float eps,
                           orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n <= 0 || n_rows < 0 || !d_out || !d_x || !d_w) return set_error(ORC_E_INVALID, "rmsnorm: bad args");
    if (n % 4 == 0 && (((uintptr_t)d_out | (uintptr_t)d_x | (uintptr_t)d_w) & 15))
        return set_error(ORC_E_INVALID, "rmsnorm: pointers must be 16-byte aligned when n is a multiple of 4");
    if (!n_rows) return ORC_OK;
    hipLaunchKernelGGL(k_rmsnorm, dim3(n_rows), dim3(256), 0, resolve_stream(s), d_out, d_x, d_w, n, eps);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_qk_norm(float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim, const float* d_qw,
                           const float* d_kw, float eps, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n_tok < 0 || n_heads <= 0 || n_kv <= 0 || head_dim <= 0 || head_dim > 128 ||
        ldqkv < (n_heads + 2 * n_kv) * head_dim || !d_qkv || !d_qw || !d_kw)
        return set_error(ORC_E_INVALID, "qk_norm: bad args (1 <= head_dim <= 128, ldqkv covers q | k | v)");
    if (!n_tok) return ORC_OK;
    if (n_tok > 65535) return set_error(ORC_E_INVALID, "qk_norm: at most 65535 tokens per call");
    hipLaunchKernelGGL(k_qk_norm, dim3((n_heads + n_kv + 3) / 4, n_tok), dim3(256), 0, resolve_stream(s), d_qkv, ldqkv,
                       n_heads, n_kv, head_dim, d_qw, d_kw, eps);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_rope_kv_store_at(float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim,
                                    const int32_t* d_pos, int pos_off, const float* d_rope, float* d_kc, float* d_vc,
                                    int ctx, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n_tok < 0 || n_heads <= 0 || n_kv <= 0 || head_dim <= 0 || head_dim % 2 ||
        (!d_pos && (pos_off < 0 || pos_off + n_tok > ctx)) || ldqkv < (n_heads + 2 * n_kv) * head_dim || !d_qkv ||
        !d_rope || !d_kc || !d_vc)
        return set_error(ORC_E_INVALID, "rope_kv_store: bad args (positions must fit the context)");
    if (!n_tok) return ORC_OK;
    hipLaunchKernelGGL(k_rope_kv, dim3(n_tok), dim3(256), 0, resolve_stream(s), d_qkv, ldqkv, n_heads, n_kv, head_dim,
                       d_pos, pos_off, (const float2*)d_rope, d_kc, d_vc, ctx);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_rope_kv_store(float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim,
                                 int start_pos, const float* d_rope, float* d_kc, float* d_vc, int ctx,
                                 orc_stream_t s) {
    return orc_rope_kv_store_at(d_qkv, ldqkv, n_tok, n_heads, n_kv, head_dim, nullptr, start_pos, d_rope, d_kc, d_vc,
                                ctx, s);
}

extern "C" size_t orc_attn_workspace(int n_tok, int n_heads, int head_dim, int max_pos) {
    const size_t nch = (size_t)(max_pos + kCH - 1) / kCH;
    return nch * (size_t)n_heads * (size_t)n_tok * (size_t)(head_dim + 2) * sizeof(float);
}

extern "C" int orc_attn_gqa_at(const float* d_q, int ldq, int n_tok, int n_heads, int n_kv, int head_dim,
                               const int32_t* d_pos, int pos_off, const float* d_kc, const float* d_vc, int ctx,
                               float* d_out, int ldo, void* d_work, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n_tok <= 0 || n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || (!d_pos && (pos_off < 0 || pos_off + n_tok > ctx)) ||
        !d_q || !d_kc || !d_vc || !d_out || !d_work || ldq % 4 || ((uintptr_t)d_q & 15))
        return set_error(ORC_E_INVALID, "attn_gqa: bad args");
    if (head_dim != 64 && head_dim != 128) return set_error(ORC_E_UNSUPPORTED, "attn_gqa: head_dim must be 64 or 128");
    // a device position sizes the grid for the whole context (chunks past the
    // last position exit at once); a host position sizes it exactly
    const int nch = d_pos ? (ctx + kCH - 1) / kCH : (pos_off + n_tok + kCH - 1) / kCH;
    hipStream_t st = resolve_stream(s);
    if (head_dim == 64) {
        hipLaunchKernelGGL(k_attn_partial<64>, dim3(nch, n_kv), dim3(256), 0, st, d_q, ldq, n_tok, n_heads, n_kv,
                           d_pos, pos_off, d_kc, d_vc, ctx, (float*)d_work);
        ORC_LAUNCH_CHECK();
        hipLaunchKernelGGL(k_attn_combine<64>, dim3(n_heads, n_tok), dim3(64), 0, st, n_tok, n_heads, d_pos, pos_off,
                           ctx, (const float*)d_work, d_out, ldo);
    } else {
        hipLaunchKernelGGL(k_attn_partial<128>, dim3(nch, n_kv), dim3(256), 0, st, d_q, ldq, n_tok, n_heads, n_kv,
                           d_pos, pos_off, d_kc, d_vc, ctx, (float*)d_work);
        ORC_LAUNCH_CHECK();
        hipLaunchKernelGGL(k_attn_combine<128>, dim3(n_heads, n_tok), dim3(128), 0, st, n_tok, n_heads, d_pos, pos_off,
                           ctx, (const float*)d_work, d_out, ldo);
    }
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_attn_gqa(const float* d_q, int ldq, int n_tok, int n_heads, int n_kv, int head_dim, int start_pos,
                            const float* d_kc, const float* d_vc, int ctx, float* d_out, int ldo, void* d_work,
                            orc_stream_t s) {
    return orc_attn_gqa_at(d_q, ldq, n_tok, n_heads, n_kv, head_dim, nullptr, start_pos, d_kc, d_vc, ctx, d_out, ldo,
                           d_work, s);
}

static int argmax_slices(int n) { return std::max(1, std::min(256, (n + kArgBlock - 1) / kArgBlock)); }

// ── allocation-free argmax (orc_argmax_noalloc) ─────────────────────────────
// The per-slice partial maxima of up to kNoAllocRows rows live in a
// file-scope device array, one copy per GPU (32 KiB, held until the process
// ends). Host code never passes the array's name to a kernel: its address on
// each device is looked up once, with that device current, by
// argmax_noalloc_device_init (called from orc_init) and kept per device.
constexpr int kNoAllocRows = 16;
constexpr int kNoAllocSlices = 256;  // the most slices argmax_slices() makes
static __device__ __align__(256) VI scratch[kNoAllocRows * kNoAllocSlices];
static std::mutex g_scratch_mu;
static std::unordered_map<int, VI*> g_scratch_ptr;  // device -> its copy of `scratch`

int orc::argmax_noalloc_device_init(int device) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr.count(device)) return ORC_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return set_error(ORC_E_HIP, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[device] = (VI*)p;
    return ORC_OK;
}

extern "C" size_t orc_argmax_workspace(int n_rows, int n) { return (size_t)n_rows * argmax_slices(n) * sizeof(VI); }

extern "C" int orc_argmax(const float* d_x, int n_rows, int n, int ld, int32_t* d_out, void* d_work, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n <= 0 || n_rows <= 0 || ld < n || !d_x || !d_out || !d_work) return set_error(ORC_E_INVALID, "argmax: bad args");
    const int ns = argmax_slices(n);
    hipStream_t st = resolve_stream(s);
    hipLaunchKernelGGL(k_argmax1, dim3(ns, n_rows), dim3(256), 0, st, d_x, n, ld, ns, (VI*)d_work);
    ORC_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_argmax2, dim3(n_rows), dim3(64), 0, st, (const VI*)d_work, ns, d_out);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

// orc_argmax with its partials in this device's `scratch` instead of a
// caller workspace: the same two kernels, so the same results. k_argmax1
// writes every partial k_argmax2 reads, so nothing needs clearing between
// calls. No allocation, no memset.
extern "C" int orc_argmax_noalloc(const float* d_x, int n_rows, int n, int ld, int32_t* d_out, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n <= 0 || n_rows <= 0 || ld < n || !d_x || !d_out) return set_error(ORC_E_INVALID, "argmax_noalloc: bad args");
    if (n_rows > kNoAllocRows)
        return set_error(ORC_E_INVALID, "argmax_noalloc: at most " + std::to_string(kNoAllocRows) + " rows per call");
    const int ns = argmax_slices(n);
    if ((size_t)n_rows * ns > (size_t)kNoAllocRows * kNoAllocSlices)
        return set_error(ORC_E_INVALID, "argmax_noalloc: partials exceed the scratch");
    int dev = -1;
    ORC_HIP_CHECK(hipGetDevice(&dev));
    VI* w = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        auto it = g_scratch_ptr.find(dev);
        if (it != g_scratch_ptr.end()) w = it->second;
    }
    if (!w) return set_error(ORC_E_NOINIT, "argmax_noalloc: orc_init was not called for the current device");
    hipStream_t st = resolve_stream(s);
    hipLaunchKernelGGL(k_argmax1, dim3(ns, n_rows), dim3(256), 0, st, d_x, n, ld, ns, w);
    ORC_LAUNCH_CHECK();
    hipLaunchKernelGGL(k_argmax2, dim3(n_rows), dim3(64), 0, st, (const VI*)w, ns, d_out);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_spec_accept_greedy(const int32_t* d_tgt, const int32_t* d_dft, int n_draft, int32_t* d_out,
                                      orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n_draft < 0 || !d_tgt || !d_out || (n_draft && !d_dft)) return set_error(ORC_E_INVALID, "accept: bad args");
    hipLaunchKernelGGL(k_accept_greedy, dim3(1), dim3(64), 0, resolve_stream(s), d_tgt, d_dft, n_draft, d_out,
                       (int32_t*)nullptr, (int32_t*)nullptr);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_spec_accept_greedy_at(const int32_t* d_tgt, const int32_t* d_dft, int n_draft, int32_t* d_out,
                                         int32_t* d_pos, int32_t* d_next, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n_draft < 0 || !d_tgt || !d_out || (n_draft && !d_dft) || !d_pos || !d_next)
        return set_error(ORC_E_INVALID, "accept: bad args");
    hipLaunchKernelGGL(k_accept_greedy, dim3(1), dim3(64), 0, resolve_stream(s), d_tgt, d_dft, n_draft, d_out, d_pos,
                       d_next);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_decode_advance(int32_t* d_tok, int32_t* d_hist, int32_t* d_pos, int32_t* d_count, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_tok || !d_hist || !d_pos || !d_count) return set_error(ORC_E_INVALID, "decode_advance: null pointer");
    hipLaunchKernelGGL(k_decode_advance, dim3(1), dim3(64), 0, resolve_stream(s), d_tok, d_hist, d_pos, d_count);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}


// A timed launch takes its dispatch's start / stop events (hipExtLaunchKernelGGL);
// every other launch, and so every launch recorded into a graph, is a plain one.
template <typename K, typename... A>
static void attn_launch(bool timed, const LaunchEv& ev, K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st,
                        A... args) {
    if (timed) hipExtLaunchKernelGGL(kernel, grid, block, lds, st, ev.a, ev.b, 0, args...);
    else hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
}

extern "C" int orc_attn_prefill(const float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim,
                                int pos_off, const float* d_rope, float* d_kc, float* d_vc, int ctx, float* d_out,
                                int ldo, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n_tok <= 0 || n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || pos_off < 0 || pos_off + n_tok > ctx ||
        ldqkv < (n_heads + 2 * n_kv) * head_dim || ldqkv % 4 || ldo % 4 || !d_qkv || !d_rope || !d_kc || !d_vc ||
        !d_out || ((uintptr_t)d_qkv & 15) || ((uintptr_t)d_kc & 15) || ((uintptr_t)d_vc & 15) ||
        ((uintptr_t)d_rope & 15) || ((uintptr_t)d_out & 15))
        return set_error(ORC_E_INVALID, "attn_prefill: bad args");
    if (n_heads / n_kv > kRMax) return set_error(ORC_E_UNSUPPORTED, "attn_prefill: more than 8 query heads per kv head");
    if (head_dim != 64 && head_dim != 128) return set_error(ORC_E_UNSUPPORTED, "attn_prefill: head_dim must be 64 or 128");
    const int R = n_heads / n_kv;
    hipStream_t st = resolve_stream(s);
    const dim3 grid((n_tok + kPaTok - 1) / kPaTok, n_kv);
    double bytes = 0;  // K / V rows of every query block's positions, once per block; QKV rows in, rows out
    for (int t0 = 0; t0 < n_tok; t0 += kPaTok)
        bytes += 8.0 * n_kv * head_dim * (pos_off + std::min(n_tok, t0 + kPaTok));
    bytes += 4.0 * n_tok * ((double)(n_heads + 2 * n_kv) * head_dim + (double)n_heads * head_dim);
    LaunchEv ev;
    const bool tm = prof_arm(st, kProfAttnPf, n_tok, bytes, &ev.a, &ev.b);
    if (head_dim == 64) {
        const size_t lds = pa_lds_bytes<64>(R);
        if (lds > 160 * 1024) return set_error(ORC_E_UNSUPPORTED, "attn_prefill: LDS");
        attn_launch(tm, ev, (k_attn_pf<64>), grid, dim3(kSW), lds, st, d_qkv, ldqkv, n_tok, n_heads, n_kv, pos_off,
                    (const float2*)d_rope, d_kc, d_vc, ctx, d_out, ldo);
    } else {
        const size_t lds = pa_lds_bytes<128>(R);
        if (lds > 160 * 1024) return set_error(ORC_E_UNSUPPORTED, "attn_prefill: LDS");
        attn_launch(tm, ev, (k_attn_pf<128>), grid, dim3(kSW), lds, st, d_qkv, ldqkv, n_tok, n_heads, n_kv, pos_off,
                    (const float2*)d_rope, d_kc, d_vc, ctx, d_out, ldo);
    }
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" size_t orc_attn_fused_workspace(int n_heads, int n_kv, int head_dim) {
    if (n_heads <= 0 || n_kv <= 0 || head_dim <= 0) return 0;
    return (size_t)kMaxTokAttn * n_heads * kNCMax * (head_dim + 32) * sizeof(float);
}

extern "C" int orc_attn_wg_limit(void) { return kWGMax; }

extern "C" int orc_attn_fused_at(const float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim,
                                 const int32_t* d_pos, int pos_off, const float* d_rope, float* d_kc, float* d_vc,
                                 int ctx, int pos_floor, int pos_limit, float* d_out, int ldo, void* d_work,
                                 orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n_tok <= 0 || n_heads <= 0 || n_kv <= 0 || n_heads % n_kv || (!d_pos && (pos_off < 0 || pos_off + n_tok > ctx)) ||
        ldqkv < (n_heads + 2 * n_kv) * head_dim || ldqkv % 4 || ldo % 4 || !d_qkv || !d_rope || !d_kc || !d_vc ||
        !d_out || !d_work || ((uintptr_t)d_qkv & 15) || ((uintptr_t)d_kc & 15) || ((uintptr_t)d_vc & 15) ||
        ((uintptr_t)d_rope & 15) || ((uintptr_t)d_work & 15))
        return set_error(ORC_E_INVALID, "attn_fused: bad args");
    if (n_heads / n_kv > kRMax) return set_error(ORC_E_UNSUPPORTED, "attn_fused: more than 8 query heads per kv head");
    if (n_tok > kMaxTokAttn) return set_error(ORC_E_UNSUPPORTED, "attn_fused: at most 16 tokens per launch");
    if (head_dim != 64 && head_dim != 128) return set_error(ORC_E_UNSUPPORTED, "attn_fused: head_dim must be 64 or 128");
    if (pos_limit < 1 || pos_limit > ctx) return set_error(ORC_E_INVALID, "attn_fused: pos_limit must be in [1, ctx]");
    if (pos_floor < 0 || pos_floor >= pos_limit)
        return set_error(ORC_E_INVALID, "attn_fused: pos_floor must be in [0, pos_limit)");
    hipStream_t st = resolve_stream(s);
    // which paths the tokens take: by their own positions (host position) or
    // for any position in [pos_floor, pos_limit) (device position):
    // P <= kWGMax k_attn_wg, P <= kMtMax k_attn_mt, above k_attn_split; the
    // chunk grids cover the most chunks such a position needs
    bool short_ctx = false;
    int nch_mt = 0, nch_sp = 0;
    if (!d_pos) {
        for (int t = 0; t < n_tok; ++t) {
            const int P = pos_off + t + 1;
            if (P <= kWGMax) short_ctx = true;
            else if (P <= kMtMax) nch_mt = std::max(nch_mt, n_chunks(P));
            else nch_sp = std::max(nch_sp, n_chunks(P));
        }
    } else {
        short_ctx = pos_floor + 1 <= kWGMax;
        // below kMtMax, n_chunks grows with P: the band's last position needs the most
        if (pos_limit > kWGMax && pos_floor + 1 <= kMtMax) nch_mt = n_chunks(std::min(pos_limit, kMtMax));
        for (int P = std::max(kMtMax, pos_floor) + 1; P <= pos_limit && nch_sp < kNCMax; ++P)
            nch_sp = std::max(nch_sp, n_chunks(P));
    }
    const int R = n_heads / n_kv;
    float* w = (float*)d_work;
    // live timing (host positions only): algorithmic bytes of a launch = the
    // K and V rows of the positions its tokens read, once (the verify tokens
    // share them), + the QKV rows in + the attention rows out
    double kv_bytes[3] = {0, 0, 0};  // [k_attn_wg, k_attn_mt, k_attn_split]
    if (!d_pos) {
        const double io = 4.0 * n_tok * ((double)(n_heads + 2 * n_kv) * head_dim + (double)n_heads * head_dim);
        const int pmax = pos_off + n_tok;
        kv_bytes[0] = 8.0 * n_kv * head_dim * std::min(pmax, kWGMax) + io;
        kv_bytes[1] = 8.0 * n_kv * head_dim * std::min(pmax, kMtMax) + io;
        kv_bytes[2] = 8.0 * n_kv * head_dim * pmax + io;
    }
    auto armed = [&](int fam, double bytes, LaunchEv& ev) {
        return !d_pos && prof_arm(st, fam, n_tok, bytes, &ev.a, &ev.b);
    };
    auto launch = [&](auto hd_tag) {
        constexpr int HD = decltype(hd_tag)::value;
        LaunchEv ev;
        if (short_ctx) {
            // one workgroup per (query head, token)
            const dim3 blk(wg_waves<HD>() * 64), grid(n_heads, n_tok);
            const bool tm = armed(kProfAttnWG, kv_bytes[0], ev);
            attn_launch(tm, ev, (k_attn_wg<HD, 1>), grid, blk, 0, st, d_qkv, ldqkv, n_heads, n_kv, d_pos, pos_off,
                        (const float2*)d_rope, d_kc, d_vc, ctx, d_out, ldo);
            ORC_LAUNCH_CHECK();
        }
        if (nch_mt > 0) {
            // one workgroup per (chunk, kv head) for all tokens and query heads
            const bool tm = armed(kProfAttnMt, kv_bytes[1], ev);
            attn_launch(tm, ev, (k_attn_mt<HD>), dim3(nch_mt, n_kv), dim3(kSW),
                        mt_lds_floats<HD>(n_tok * R) * sizeof(float), st, d_qkv, ldqkv, n_tok, n_heads, n_kv, d_pos,
                        pos_off, (const float2*)d_rope, d_kc, d_vc, ctx, w);
            ORC_LAUNCH_CHECK();
        }
        if (nch_sp > 0) {
            // all query heads of a kv head in one workgroup (one workgroup
            // per query head measured slower: 12.1 vs 9.2 us for a
            // 0.5B-draft decode step at 8.4 K positions)
            const bool tm = armed(kProfAttnSplit, kv_bytes[2], ev);
            attn_launch(tm, ev, (k_attn_split<HD, kRMax>), dim3(nch_sp, n_kv * ((R + kRMax - 1) / kRMax), n_tok),
                        dim3(kSW), 0, st, d_qkv, ldqkv, n_heads, n_kv, d_pos, pos_off, (const float2*)d_rope, d_kc,
                        d_vc, ctx, d_out, ldo, w);
            ORC_LAUNCH_CHECK();
        }
        if (nch_mt > 0 || nch_sp > 0) {
            const bool tm = armed(kProfAttnMerge, 0.0, ev);
            attn_launch(tm, ev, (k_attn_merge<HD>), dim3(n_heads, n_tok), dim3(kMG), 0, st, n_heads, n_kv, d_pos,
                        pos_off, ctx, (const float*)w, d_out, ldo);
            ORC_LAUNCH_CHECK();
        }
        return ORC_OK;
    };
    return head_dim == 64 ? launch(std::integral_constant<int, 64>{}) : launch(std::integral_constant<int, 128>{});
}

// Device sampler, Engine-style stochastic acceptance and speculative
// sampling (gfx950).
//
// Replaces Sampler::sample / record (core/sampler.cpp:15-105) and the
// stochastic verify loop of Engine::generate (core/engine.cpp:150-240) with
// kernels, so only the emitted ids cross to the host. The same transform,
// written out as distributions, feeds the min(1, p/q) acceptance chain with
// residual resampling (no reference counterpart).
//
// One 1024-thread workgroup samples one row of logits, in place as the
// reference does (the row ends up holding the probabilities); the transform
// and the acceptance chain also run split over many workgroups (below):
//  * repeat penalty over the device-resident history, one entry at a time
//    (repeated ids compound), then temperature (skipped for T <= 0 or 1);
//  * T <= 0: first index of the maximum;
//  * otherwise softmax: block max, block sum of expf(l - max), p = e * (1/sum);
//  * top-k by an exact radix select on the bits of p (eight 4-bit digits;
//    p >= 0, so the bit patterns order like the values), then the candidates
//    (p >= the k-th value) are sorted by (p desc, index asc) with a bitonic
//    sort in LDS;
//    at most 16384 candidates (top_k = 0, "all tokens" in the reference, is
//    exact for vocabularies up to that size; the entry points refuse a
//    larger vocabulary with ORC_E_UNSUPPORTED for a state initialised with
//    top_k = 0, since the nucleus could then need more candidates);
//  * top-p cut at cumulative >= top_p, r = u * total with
//    u = generate_canonical<float, 24>(mt19937) as libstdc++ forms it, then
//    r -= p_i until r <= 0 (fallback: the first candidate);
//  * the token is recorded; the history keeps the reference's trim rule
//    (more than 2 * repeat_last entries: drop the oldest repeat_last).
// mt19937 runs in one lane from a state kept in device memory.
#include "orc_internal.hpp"

#include <cstring>
#include <mutex>
#include <unordered_set>

namespace orc {

constexpr int kST = 1024;          // threads of a sampling workgroup
constexpr int kSampHist = 4096;    // history capacity (repeat_last <= kSampHist - 1)
constexpr int kCandMax = 16384;    // candidates sorted in LDS (largest top_k; top_k = 0 means this many)

// The transform of a row split over workgroups (k_tx_*): each workgroup owns
// a slice of kTxSlice logits, passes on at most kTxCand candidates, and the
// state holds the per-slice partial results between the launches.
constexpr int kTxSlice = 4 * kST;  // logits per workgroup, four per thread
constexpr int kTxMaxG = 48;        // slices per row (vocabularies up to 196608)
constexpr int kTxRows = 17;        // rows per call (a verify pass of 16 proposals + the bonus row)
constexpr int kTxCand = 192;       // candidates one slice passes on
constexpr int kTxStop = 128;       // a slice's threshold search stops at this many candidates (or top_k)
constexpr int kTxK = 128;          // largest top_k of the split path

struct TxWork {
    float mx[kTxRows][kTxMaxG];   // slice maxima of the scaled logits
    float sum[kTxRows][kTxMaxG];  // slice sums of exp(l - max)
    int nc[kTxRows][kTxMaxG];     // candidates per slice
    int ovf[kTxRows];             // a slice had more than kTxCand candidates
    int cut[kTxRows];             // kept set of each row (list mode)
    float total[kTxRows];         // its mass
    uint2 kept[kTxRows][kTxK];    // (index, bits of p), sorted by (p desc, index asc)
    // the acceptance chain split over workgroups (k_chain_*)
    int ch_mode, ch_row, ch_emitted, ch_accepted, ch_max;  // mode 0: no draw, 1: residual, 2: bonus
    float ch_u;
    double ch_sum[kTxMaxG];  // slice sums of the draw's weights
    int ch_last[kTxMaxG];    // last positive weight of each slice (-1: none)
    uint2 cand[kTxRows][kTxMaxG][kTxCand];  // (bits of exp(l - max), index)
};

struct DevSampler {
    uint32_t mt[624];
    int mti;
    float temp, top_p, pen;
    int top_k, last;
    int nh;
    int32_t hist[kSampHist];
    TxWork tx;  // scratch of the split transform (calls on one state must not overlap)
};

__device__ uint32_t mt_next(DevSampler* s) {
    if (s->mti >= 624) {
        for (int i = 0; i < 624; i++) {
            const uint32_t y = (s->mt[i] & 0x80000000u) | (s->mt[(i + 1) % 624] & 0x7FFFFFFFu);
            s->mt[i] = s->mt[(i + 397) % 624] ^ (y >> 1) ^ ((y & 1u) ? 0x9908B0DFu : 0u);
        }
        s->mti = 0;
    }
    uint32_t y = s->mt[s->mti++];
    y ^= y >> 11;
    y ^= (y << 7) & 0x9D2C5680u;
    y ^= (y << 15) & 0xEFC60000u;
    y ^= y >> 18;
    return y;
}

// generate_canonical<float, 24>(mt19937): one 32-bit draw / 2^32, kept below 1
__device__ float mt_canonical(DevSampler* s) {
    float r = (float)mt_next(s) / 4294967296.0f;
    if (r >= 1.0f) r = __builtin_bit_cast(float, 0x3F7FFFFFu);  // largest float below 1
    return r;
}

__device__ void record_tok(DevSampler* s, int32_t tok) {
    // A full buffer keeps its last repeat_last entries (< kSampHist), the only
    // ones the penalty ever reads; below 2048 the reference's own trim (more
    // than 2 * repeat_last entries) comes first and this never runs but with
    // repeat_last == 0, where the history is never read.
    if (s->nh >= kSampHist) {
        const int keep = s->last;
        for (int i = 0; i < keep; ++i) s->hist[i] = s->hist[s->nh - keep + i];
        s->nh = keep;
    }
    s->hist[s->nh++] = tok;
    if (s->nh > s->last * 2) {
        for (int i = 0; i + s->last < s->nh; ++i) s->hist[i] = s->hist[i + s->last];
        s->nh -= s->last;
    }
}

struct SampScratch {
    float red[kST / 64];
    int ired[kST / 64];
    unsigned int hist[512];
    int bcast[8];
    float fb[4];  // [2]: the split transform's uniform, [3]: its top_p
    double dscan[kST];
    unsigned long long cand[kCandMax];
};

typedef const __attribute__((address_space(1))) float* g_cfp;

// f(i, x[i]) for the row elements this thread owns (i = tid, tid + kST, ...)
// in increasing i, as a plain strided loop would visit them, with the loads
// of kRowBatch elements issued together (indices clamped into the row): a
// pass over a 152K-entry row keeps eight loads in flight per thread instead
// of waiting on each. x is device memory.
constexpr int kRowBatch = 8;
template <class F> __device__ __forceinline__ void row_pass(const float* x, int n, F&& f) {
    const g_cfp gx = (g_cfp)x;
    for (int i0 = threadIdx.x; i0 < n; i0 += kRowBatch * kST) {
        float v[kRowBatch];
#pragma unroll
        for (int j = 0; j < kRowBatch; ++j) v[j] = gx[min(i0 + j * kST, n - 1)];
#pragma unroll
        for (int j = 0; j < kRowBatch; ++j)
            if (i0 + j * kST < n) f(i0 + j * kST, v[j]);
    }
}

// row_pass over two rows at once: f(i, x[i], y[i])
template <class F> __device__ __forceinline__ void row_pass2(const float* x, const float* y, int n, F&& f) {
    const g_cfp gx = (g_cfp)x, gy = (g_cfp)y;
    for (int i0 = threadIdx.x; i0 < n; i0 += kRowBatch * kST) {
        float u[kRowBatch], v[kRowBatch];
#pragma unroll
        for (int j = 0; j < kRowBatch; ++j) {
            const int i = min(i0 + j * kST, n - 1);
            u[j] = gx[i];
            v[j] = gy[i];
        }
#pragma unroll
        for (int j = 0; j < kRowBatch; ++j)
            if (i0 + j * kST < n) f(i0 + j * kST, u[j], v[j]);
    }
}

// f(i, w(i)) for i = b .. e-1 in order, the values of kRowBatch consecutive
// indices computed (loaded) together; f returns false to stop.
template <class W, class F> __device__ __forceinline__ void chunk_pass(int b, int e, W&& w, F&& f) {
    for (int i0 = b; i0 < e; i0 += kRowBatch) {
        float v[kRowBatch];
#pragma unroll
        for (int j = 0; j < kRowBatch; ++j) v[j] = w(min(i0 + j, e - 1));
#pragma unroll
        for (int j = 0; j < kRowBatch; ++j)
            if (i0 + j < e && !f(i0 + j, v[j])) return;
    }
}

__device__ float block_max(float v, SampScratch& sh) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = sh.red[0];
    for (int w = 1; w < kST / 64; ++w) m = fmaxf(m, sh.red[w]);
    __syncthreads();
    return m;
}

__device__ float block_sum(float v, SampScratch& sh) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    if ((threadIdx.x & 63) == 0) sh.red[threadIdx.x >> 6] = v;
    __syncthreads();
    float m = sh.red[0];
    for (int w = 1; w < kST / 64; ++w) m += sh.red[w];  // fixed order
    __syncthreads();
    return m;
}

// first index of the maximum over the block
__device__ int block_argmax(const float* x, int n, SampScratch& sh) {
    float bv = -INFINITY;
    int bi = 0x7FFFFFFF;
    row_pass(x, n, [&](int i, float v) {
        if (v > bv || (v == bv && i < bi)) {
            bv = v;
            bi = i;
        }
    });
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        sh.red[threadIdx.x >> 6] = bv;
        sh.ired[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    float v = sh.red[0];
    int idx = sh.ired[0];
    for (int w = 1; w < kST / 64; ++w)
        if (sh.red[w] > v || (sh.red[w] == v && sh.ired[w] < idx)) {
            v = sh.red[w];
            idx = sh.ired[w];
        }
    __syncthreads();
    return idx == 0x7FFFFFFF ? 0 : idx;
}

// ascending bitonic sort of sh.cand[0 .. m), m a power of two <= kCandMax
__device__ void bitonic_sort(SampScratch& sh, int m) {
    for (int size = 2; size <= m; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < m; i += kST) {
                const int j = i ^ stride;
                if (j > i) {
                    const bool up = (i & size) == 0;
                    const unsigned long long a = sh.cand[i], b = sh.cand[j];
                    if ((a > b) == up) {
                        sh.cand[i] = b;
                        sh.cand[j] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
}

// Repeat penalty (sampler.cpp:15-27) over the last repeat_last entries of
// history + extra (extra: proposals not yet recorded), one entry at a time so
// repeated ids compound. Up to kPenPar entries: each entry's logit is loaded
// by its own thread, lane 0 applies the penalties in entry order in LDS (an
// entry updates the value held at its id's first occurrence), and the first
// occurrences write the results back; the same operations in the same order
// as one lane walking the entries over the row, without a dependent global
// load per entry. More entries: that one-lane walk. Whole workgroup (sh.cand
// and sh.dscan serve as scratch).
constexpr int kPenPar = 256;
__device__ void penalize(const DevSampler* s, float* lg, int n, const int32_t* extra, int n_extra,
                         SampScratch& sh) {
    if (!(s->pen > 1.f)) return;
    const int L = s->nh + n_extra;
    const int start = L - s->last > 0 ? L - s->last : 0;
    const int m = L - start;
    const int tid = threadIdx.x;
    auto entry = [&](int i) { return i < s->nh ? s->hist[i] : extra[i - s->nh]; };
    if (m > kPenPar) {
        if (tid == 0)
            for (int i = start; i < L; ++i) {
                const int32_t id = entry(i);
                if (id < 0 || id >= n) continue;
                const float l = lg[id];
                lg[id] = l > 0.f ? l / s->pen : l * s->pen;
            }
        __syncthreads();
        return;
    }
    int* first = (int*)sh.dscan;  // first occurrence of each entry's id
    int32_t id = -1;
    if (tid < m) {
        id = entry(start + tid);
        const bool ok = id >= 0 && id < n;
        const float v = ok ? lg[id] : 0.f;
        sh.cand[tid] = ((unsigned long long)(uint32_t)(ok ? id : -1) << 32) | __builtin_bit_cast(uint32_t, v);
    }
    __syncthreads();
    if (tid < m) {
        int f = tid;
        for (int j = 0; j < tid; ++j)
            if ((int32_t)(sh.cand[j] >> 32) == (int32_t)(sh.cand[tid] >> 32)) {
                f = j;
                break;
            }
        first[tid] = f;
    }
    __syncthreads();
    if (tid == 0)
        for (int i = 0; i < m; ++i) {
            if ((int32_t)(sh.cand[i] >> 32) < 0) continue;
            const int f = first[i];
            const unsigned long long c = sh.cand[f];
            const float l = __builtin_bit_cast(float, (uint32_t)c);
            const float r = l > 0.f ? l / s->pen : l * s->pen;
            sh.cand[f] = (c & 0xFFFFFFFF00000000ull) | __builtin_bit_cast(uint32_t, r);
        }
    __syncthreads();
    if (tid < m && first[tid] == tid && id >= 0 && id < n) lg[id] = __builtin_bit_cast(float, (uint32_t)sh.cand[tid]);
    __syncthreads();
}

// lane i's value of v (i uniform over the wave)
__device__ __forceinline__ float rdlane(float v, int i) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), i));
}
__device__ __forceinline__ unsigned long long rdlane(unsigned long long v, int i) {
    const unsigned int lo = (unsigned int)__builtin_amdgcn_readlane((int)(unsigned int)v, i);
    const unsigned int hi = (unsigned int)__builtin_amdgcn_readlane((int)(unsigned int)(v >> 32), i);
    return ((unsigned long long)hi << 32) | lo;
}

// The parameters the split transform takes (T > 0, 1 <= top_k <= kTxK).
__device__ __forceinline__ bool tx_split(const DevSampler* s) {
    return s->temp > 0.f && s->top_k >= 1 && s->top_k <= kTxK;
}

// probability held in a candidate key (~bits(p) << 32 | index)
__device__ __forceinline__ float cand_p(unsigned long long c) { return __builtin_bit_cast(float, ~(uint32_t)(c >> 32)); }

// Temperature, softmax (p written over lg) and the top-k candidates sorted by
// (p desc, index asc) into sh.cand[0 .. k) (sampler.cpp:35-64). T > 0 only;
// scaled: lg already holds the logits divided by T. Returns k.
__device__ int topk_sorted(const DevSampler* s, float* lg, int n, SampScratch& sh, bool scaled = false) {
    const int tid = threadIdx.x;
    const float T = s->temp;
    // temperature (sampler.cpp:35-39) and the maximum in one pass
    const bool scale = T != 1.f && !scaled;
    const float inv_t = 1.f / T;
    float mx = -INFINITY;
    row_pass(lg, n, [&](int i, float l) {
        if (scale) {
            l *= inv_t;
            lg[i] = l;
        }
        mx = fmaxf(mx, l);
    });
    mx = block_max(mx, sh);
    // softmax (ops::softmax: e = exp(l - max), p = e * (1/sum))
    float sum = 0.f;
    row_pass(lg, n, [&](int i, float l) {
        const float e = expf(l - mx);
        lg[i] = e;
        sum += e;
    });
    sum = block_sum(sum, sh);
    const float inv_s = 1.f / sum;
    row_pass(lg, n, [&](int i, float e) { lg[i] = e * inv_s; });
    __syncthreads();
    // top-k threshold: exact radix select of the k-th largest p
    const int k = min(s->top_k > 0 ? s->top_k : n, min(n, kCandMax));
    unsigned int prefix = 0, mask = 0;
    int krem = k;
    // Four bits per pass (eight passes): each thread counts its own elements
    // into its own column of 16 counters (the candidate buffer serves as
    // scratch, [digit][thread]), so no two lanes ever add to one address;
    // wave d then adds up digit d's column sums.
    unsigned int* const cnt = (unsigned int*)sh.cand;
    static_assert(16 * kST * sizeof(unsigned int) <= sizeof(sh.cand), "digit counters fit the candidate buffer");
    static_assert(kST / 64 == 16, "one wave per digit");
    for (int shift = 28; shift >= 0; shift -= 4) {
#pragma unroll
        for (int d = 0; d < 16; ++d) cnt[d * kST + tid] = 0;
        row_pass(lg, n, [&](int, float p) {
            const unsigned int key = __builtin_bit_cast(unsigned int, p);
            if ((key & mask) == prefix) atomicAdd(&cnt[((key >> shift) & 15u) * kST + tid], 1u);
        });
        __syncthreads();
        {
            const int d = tid >> 6, l = tid & 63;
            unsigned int c = 0;
#pragma unroll
            for (int i = 0; i < kST / 64; ++i) c += cnt[d * kST + l * (kST / 64) + i];
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, 64);
            if (l == 0) sh.hist[d] = c;
        }
        __syncthreads();
        if (tid == 0) {
            int cum = 0, sel = 0;
            for (int b = 15; b >= 0; --b) {
                const int c = (int)sh.hist[b];
                if (cum + c >= krem) {
                    sel = b;
                    break;
                }
                cum += c;
            }
            sh.bcast[0] = sel;
            sh.bcast[1] = krem - cum;
        }
        __syncthreads();
        prefix |= (unsigned int)sh.bcast[0] << shift;
        mask |= 15u << shift;
        krem = sh.bcast[1];
        __syncthreads();
    }
    const unsigned int thr = prefix;  // bits of the k-th largest p; krem of its ties are kept
    // candidates: every p >= thr (key = ~bits(p) : index sorts p desc, index asc)
    if (tid == 0) sh.bcast[2] = 0;
    __syncthreads();
    row_pass(lg, n, [&](int i, float p) {
        const unsigned int key = __builtin_bit_cast(unsigned int, p);
        if (key >= thr) {
            const int slot = atomicAdd(&sh.bcast[2], 1);
            if (slot < kCandMax) sh.cand[slot] = ((unsigned long long)(~key) << 32) | (unsigned int)i;
        }
    });
    __syncthreads();
    int nc = sh.bcast[2];
    if (nc > kCandMax) {
        // more ties at the threshold than LDS holds: take every p > thr and
        // then the lowest-index ties, in index order
        __syncthreads();
        if (tid == 0) sh.bcast[2] = 0;
        __syncthreads();
        row_pass(lg, n, [&](int i, float p) {
            const unsigned int key = __builtin_bit_cast(unsigned int, p);
            if (key > thr) {
                const int slot = atomicAdd(&sh.bcast[2], 1);
                sh.cand[slot] = ((unsigned long long)(~key) << 32) | (unsigned int)i;
            }
        });
        __syncthreads();
        if (tid == 0) {
            int c = sh.bcast[2];
            for (int i = 0, got = 0; i < n && got < krem; ++i)
                if (__builtin_bit_cast(unsigned int, lg[i]) == thr) {
                    sh.cand[c++] = ((unsigned long long)(~thr) << 32) | (unsigned int)i;
                    ++got;
                }
            sh.bcast[2] = c;
        }
        __syncthreads();
        nc = sh.bcast[2];
    }
    int m = 1;
    while (m < nc) m <<= 1;
    for (int i = nc + tid; i < m; i += kST) sh.cand[i] = ~0ull;  // padding sorts last
    __syncthreads();
    bitonic_sort(sh, m);
    return k;
}

// Top-p cut over the sorted candidates (sampler.cpp:66-77): sh.bcast[4] = cut,
// sh.fb[0] = total kept mass. One lane; the caller synchronises.
__device__ void topp_cut(const DevSampler* s, const float* lg, int k, SampScratch& sh) {
    if (threadIdx.x != 0) return;
    float cum = 0.f;
    int cut = k;
    for (int i = 0; i < k; ++i) {
        cum += cand_p(sh.cand[i]);
        if (cum >= s->top_p) {
            cut = i + 1;
            break;
        }
    }
    float total = 0.f;
    for (int i = 0; i < cut; ++i) total += cand_p(sh.cand[i]);
    sh.bcast[4] = cut;
    sh.fb[0] = total;
}

// Sampler::sample on one row (core/sampler.cpp:91-97) without the record.
// Whole workgroup.
__device__ int32_t sample_row(DevSampler* s, float* lg, int n, SampScratch& sh) {
    const int tid = threadIdx.x;
    penalize(s, lg, n, nullptr, 0, sh);
    __syncthreads();
    if (s->temp <= 0.f) return block_argmax(lg, n, sh);  // sampler.cpp:50
    const int k = topk_sorted(s, lg, n, sh);
    topp_cut(s, lg, k, sh);
    // the draw (sampler.cpp:78-85), one lane
    if (tid == 0) {
        const int cut = sh.bcast[4];
        float r = mt_canonical(s) * sh.fb[0];
        int32_t tok = (int32_t)(sh.cand[0] & 0xFFFFFFFFu);
        for (int i = 0; i < cut; ++i) {
            const int32_t id = (int32_t)(sh.cand[i] & 0xFFFFFFFFu);
            r -= cand_p(sh.cand[i]);  // lg[id]
            if (r <= 0.f) {
                tok = id;
                break;
            }
        }
        sh.bcast[3] = tok;
    }
    __syncthreads();
    const int32_t tok = sh.bcast[3];
    __syncthreads();
    return tok;
}

// Top-p cut over the k sorted candidates in sh.cand, then p_out[id] = p / kept
// mass for the kept ones (zeros elsewhere when zero is set; the caller has
// cleared p_out otherwise). Whole workgroup.
__device__ void write_kept(const DevSampler* s, int k, float* p_out, int n, bool zero, SampScratch& sh) {
    const int tid = threadIdx.x;
    topp_cut(s, nullptr, k, sh);
    if (zero)
        for (int i = tid; i < n; i += kST) p_out[i] = 0.f;
    __syncthreads();
    const int cut = sh.bcast[4];
    const float total = sh.fb[0];
    for (int i = tid; i < cut; i += kST) {
        const int id = (int)(sh.cand[i] & 0xFFFFFFFFu);
        p_out[id] = cand_p(sh.cand[i]) / total;  // lg[id] / total
    }
    __syncthreads();
}

// The same transform as sampling, written out as a distribution: p_out holds
// the kept set renormalised (zeros elsewhere); T <= 0 puts all mass on the
// argmax. Whole workgroup.
__device__ void transform_row(const DevSampler* s, float* lg, int n, const int32_t* extra, int n_extra, float* p_out,
                              SampScratch& sh) {
    const int tid = threadIdx.x;
    penalize(s, lg, n, extra, n_extra, sh);
    __syncthreads();
    if (s->temp <= 0.f) {
        const int a = block_argmax(lg, n, sh);
        for (int i = tid; i < n; i += kST) p_out[i] = i == a ? 1.f : 0.f;
        __syncthreads();
        return;
    }
    const int k = topk_sorted(s, lg, n, sh);
    write_kept(s, k, p_out, n, true, sh);
}

// First index whose running sum of the positive parts of w(i) reaches
// target (r = target; r -= w(i) while w(i) > 0; stop at r <= 0), sums in
// double; falls back to the last positive index (0 if there is none).
// Whole workgroup.
template <typename W>
__device__ int block_pick(int n, W w, double target, SampScratch& sh) {
    const int tid = threadIdx.x;
    const int chunk = (n + kST - 1) / kST;
    const int b = min(n, tid * chunk), e = min(n, b + chunk);
    double loc = 0.0;
    int last = -1;
    chunk_pass(b, e, w, [&](int i, float d) {
        if (d > 0.f) {
            loc += (double)d;
            last = i;
        }
        return true;
    });
    sh.dscan[tid] = loc;
    if (tid == 0) {
        sh.bcast[5] = 0x7FFFFFFF;
        sh.bcast[6] = -1;
    }
    __syncthreads();
    if (tid == 0) {  // exclusive prefix in thread order
        double run = 0.0;
        for (int t = 0; t < kST; ++t) {
            const double v = sh.dscan[t];
            sh.dscan[t] = run;
            run += v;
        }
    }
    __syncthreads();
    const double prefix = sh.dscan[tid];
    if (last >= 0) {
        atomicMax(&sh.bcast[6], last);
        if (prefix < target && target <= prefix + loc) {
            double r = target - prefix;
            int got = last;  // rounding left r > 0: the chunk's last positive
            chunk_pass(b, e, w, [&](int i, float d) {
                if (!(d > 0.f)) return true;
                r -= (double)d;
                if (r <= 0.0) {
                    got = i;
                    return false;
                }
                return true;
            });
            atomicMin(&sh.bcast[5], got);
        } else if (target <= 0.0 && prefix == 0.0) {
            for (int i = b; i < e; ++i)
                if (w(i) > 0.f) {
                    atomicMin(&sh.bcast[5], i);
                    break;
                }
        }
    }
    __syncthreads();
    const int pick = sh.bcast[5] != 0x7FFFFFFF ? sh.bcast[5] : max(sh.bcast[6], 0);
    __syncthreads();
    return pick;
}

// min(1, p/q) acceptance of proposal x with residual resampling (no reference
// counterpart): accept when q[x] > 0 and u_acc * q[x] < p[x]; otherwise draw
// from norm(max(0, p - q)) with u_res (argmax of p when the residual is
// empty). Returns the emitted id; *accepted set on lane 0. Whole workgroup.
__device__ int32_t accept_resample(const float* p, const float* q, int n, int32_t x, float u_acc, float u_res,
                                   int* accepted, SampScratch& sh) {
    const float qx = q[x], px = p[x];
    if (qx > 0.f && u_acc * qx < px) {
        *accepted = 1;
        return x;
    }
    *accepted = 0;
    auto resid = [&](int i) { return p[i] - q[i]; };
    // total of the positive residual (double), then the draw
    double loc = 0.0;
    row_pass2(p, q, n, [&](int, float pv, float qv) {
        const float d = pv - qv;
        if (d > 0.f) loc += (double)d;
    });
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) loc += __shfl_xor(loc, o, 64);
    if ((threadIdx.x & 63) == 0) sh.dscan[threadIdx.x >> 6] = loc;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < kST / 64; ++w) tot += sh.dscan[w];
    __syncthreads();
    if (!(tot > 0.0)) return block_argmax(p, n, sh);
    return block_pick(n, resid, (double)u_res * tot, sh);
}

__global__ void k_sampler_init(DevSampler* s, uint32_t seed, float temp, float top_p, float pen, int top_k,
                               int last, const int32_t* hist, int n_hist) {
    if (threadIdx.x != 0) return;
    s->mt[0] = seed;
    for (int i = 1; i < 624; i++) s->mt[i] = 1812433253u * (s->mt[i - 1] ^ (s->mt[i - 1] >> 30)) + (uint32_t)i;
    s->mti = 624;
    s->temp = temp;
    s->top_p = top_p;
    s->pen = pen;
    s->top_k = top_k;
    s->last = last;
    s->nh = 0;
    for (int i = 0; i < n_hist; ++i) record_tok(s, hist[i]);
}

__global__ __launch_bounds__(kST) void k_sample(DevSampler* s, float* lg, int n, int32_t* out) {
    __shared__ SampScratch sh;
    const int32_t tok = sample_row(s, lg, n, sh);
    if (threadIdx.x == 0) {
        record_tok(s, tok);  // sampler.cpp:95
        *out = tok;
    }
}

// Sampler::set_params (sampler.hpp:37): new parameters, same generator and
// history; Sampler::reset (sampler.hpp:34): history cleared, same generator.
__global__ void k_sampler_set(DevSampler* s, int set, float temp, float top_p, float pen, int top_k, int last) {
    if (threadIdx.x != 0) return;
    if (set) {
        s->temp = temp;
        s->top_p = top_p;
        s->pen = pen;
        s->top_k = top_k;
        s->last = last;
    } else {
        s->nh = 0;
    }
}

__global__ void k_sampler_record(DevSampler* s, const int32_t* tok, int n) {
    if (threadIdx.x != 0) return;
    for (int i = 0; i < n; ++i) record_tok(s, tok[i]);
}

// Engine-style stochastic verify (core/engine.cpp:183-232) over the rows of
// one batched verify pass: row i is the target's logits at the i-th verify
// position. For each draft token: sample (records), record again (the
// Engine's second record, engine.cpp:194-195), stop at the first mismatch;
// when every draft token matched, sample the bonus row the same way. At most
// max_emit tokens are emitted (the caller's remaining budget; read from and
// decremented in *d_budget when given).
// out: [0] emitted, [1] accepted, [2] rows sampled (target forwards of the
// reference loop), [3] 1 if all drafts were accepted and the bonus emitted,
// [4 ..] the emitted ids. With d_pos / d_next the device round state advances.
// With split set and the split transform's parameters, the rows' kept sets
// were written by k_tx_max<true> / k_tx_exp / k_tx_final<2> (row i's window
// assumes proposals 0 .. i-1 accepted, the only case in which row i is
// sampled) and wave 0 draws from them: r = u * mass, r -= p down the sorted
// set, the first candidate if rounding leaves r > 0 (sampler.cpp:78-85).
__global__ __launch_bounds__(kST) void k_accept_engine(DevSampler* s, float* logits, int ld, int n_vocab,
                                                        const int32_t* draft, int n_draft, int max_emit,
                                                        int32_t* d_budget, int32_t* out, int32_t* d_pos,
                                                        int32_t* d_next, int split) {
    __shared__ SampScratch sh;
    if (split && tx_split(s)) {
        if (threadIdx.x >= 64) return;
        const int lane = threadIdx.x;
        const TxWork& w = s->tx;
        if (d_budget) max_emit = *d_budget;
        int emitted = 0, accepted = 0, rows = 0, all = 0;
        int32_t last_tok = 0;
        for (int i = 0; i <= n_draft && emitted < max_emit; ++i) {
            const int cut = w.cut[i];
            const float total = w.total[i];
            const uint2 ea = lane < cut ? w.kept[i][lane] : make_uint2(0u, 0u);
            const uint2 eb = lane + 64 < cut ? w.kept[i][lane + 64] : make_uint2(0u, 0u);
            float u = 0.f;
            if (lane == 0) u = mt_canonical(s);
            float rr = rdlane(u, 0) * total;
            int32_t tok = cut > 0 ? (int32_t)__builtin_amdgcn_readlane((int)ea.x, 0) : 0;
            for (int j = 0; j < cut; ++j) {
                const uint2 c = j < 64 ? make_uint2((unsigned int)__builtin_amdgcn_readlane((int)ea.x, j),
                                                    (unsigned int)__builtin_amdgcn_readlane((int)ea.y, j))
                                       : make_uint2((unsigned int)__builtin_amdgcn_readlane((int)eb.x, j - 64),
                                                    (unsigned int)__builtin_amdgcn_readlane((int)eb.y, j - 64));
                rr -= __builtin_bit_cast(float, c.y);
                if (rr <= 0.f) {
                    tok = (int32_t)c.x;
                    break;
                }
            }
            ++rows;
            if (lane == 0) {
                record_tok(s, tok);  // Sampler::sample's own record
                record_tok(s, tok);  // the Engine's second record
                out[4 + emitted] = tok;
            }
            ++emitted;
            last_tok = tok;
            if (i == n_draft) {
                all = 1;
                break;
            }
            if (tok != draft[i]) break;
            ++accepted;
        }
        if (lane == 0) {
            out[0] = emitted;
            out[1] = accepted;
            out[2] = rows;
            out[3] = all;
            if (d_pos) {
                *d_pos += emitted;
                *d_next = last_tok;
            }
            if (d_budget) *d_budget -= emitted;
        }
        return;
    }
    if (d_budget) max_emit = *d_budget;
    int emitted = 0, accepted = 0, rows = 0, all = 0;
    int32_t last_tok = 0;
    for (int i = 0; i <= n_draft && emitted < max_emit; ++i) {
        const int32_t tok = sample_row(s, logits + (size_t)i * ld, n_vocab, sh);
        ++rows;
        if (threadIdx.x == 0) {
            record_tok(s, tok);  // Sampler::sample's own record
            record_tok(s, tok);  // the Engine's second record
            out[4 + emitted] = tok;
        }
        __syncthreads();
        ++emitted;
        last_tok = tok;
        if (i == n_draft) {  // bonus row after a fully accepted round
            all = 1;
            break;
        }
        if (tok != draft[i]) break;
        ++accepted;
    }
    if (threadIdx.x == 0) {
        out[0] = emitted;
        out[1] = accepted;
        out[2] = rows;
        out[3] = all;
        if (d_pos) {
            *d_pos += emitted;
            *d_next = last_tok;
        }
        if (d_budget) *d_budget -= emitted;
    }
}

// Rows of logits -> distributions (kept set renormalised): row r uses the
// proposals extra[0 .. extra_base + r) as pending history for the penalty.
__global__ __launch_bounds__(kST) void k_transform(const DevSampler* s, float* lg, int ld, int n,
                                                    const int32_t* extra, int extra_base, float* p, int ldp) {
    __shared__ SampScratch sh;
    const int r = blockIdx.x;
    transform_row(s, lg + (size_t)r * ld, n, extra, extra_base + r, p + (size_t)r * ldp, sh);
}

__device__ float lane0_uniform(DevSampler* s, SampScratch& sh) {
    if (threadIdx.x == 0) sh.fb[1] = mt_canonical(s);
    __syncthreads();
    const float u = sh.fb[1];
    __syncthreads();
    return u;
}

__device__ double block_total(const float* p, int n, SampScratch& sh) {
    double loc = 0.0;
    row_pass(p, n, [&](int, float v) {
        if (v > 0.f) loc += (double)v;
    });
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) loc += __shfl_xor(loc, o, 64);
    if ((threadIdx.x & 63) == 0) sh.dscan[threadIdx.x >> 6] = loc;
    __syncthreads();
    double tot = 0.0;
    for (int w = 0; w < kST / 64; ++w) tot += sh.dscan[w];
    __syncthreads();
    return tot;
}

// One draw from a distribution p (u from the state's mt19937).
__global__ __launch_bounds__(kST) void k_draw(DevSampler* s, const float* p, int n, int32_t* out, int32_t* out2) {
    __shared__ SampScratch sh;
    const float u = lane0_uniform(s, sh);
    const double tot = block_total(p, n, sh);
    const int tok = block_pick(n, [&](int i) { return p[i]; }, (double)u * tot, sh);
    if (threadIdx.x == 0) {
        out[0] = tok;
        if (out2) out2[0] = tok;
    }
}

// ── the transform split over workgroups ─────────────────────────────────────
// Same results as transform_row (same kept set; the softmax sum is added in
// another order, so p may differ in its last bit) for T > 0 and
// 1 <= top_k <= kTxK, in three launches:
//  k_tx_max   (slice x row): repeat penalty of the ids in the slice, 1/T,
//             slice maximum;
//  k_tx_exp   (slice x row): e = expf(l - row max) as the one-workgroup
//             softmax forms it, slice sum, and the slice's candidates: every
//             e >= t (1 - 2^-20), t found by a radix search on the bits of e
//             such that at least min(top_k, positives) of the slice's e are
//             >= t. Any e below that bound has top_k others in its slice whose
//             p = e / sum is strictly larger, since both products are normal
//             floats rounded once and differ by more than two roundings, so
//             the row's top_k by (p desc, index asc) are all candidates;
//  k_tx_final (row): p = e * (1 / sum of the slice sums); a radix search
//             over the candidates' p down to a prefix the k-th largest p has
//             and at most max(k, 64) candidates reach; those sorted by (p
//             desc, index asc), the first k kept, top-p cut, p_out written;
//             optionally one draw from it. (Below t = 2^-100 the slice passes
//             every positive e on: p could then be subnormal.)
// Zero e (exp underflow) never enters: zero-probability candidates change
// neither the kept mass nor a draw. Other parameters (T <= 0, top_k 0 or
// above kTxK) take the one-workgroup transform in k_tx_max's first
// workgroup of each row, and a row with a slice of more than kTxCand
// candidates (ties) is redone by that transform in k_tx_final from the
// scaled logits the first launch left in the row.

// ENG (the Engine rule's rows, list mode): row r's window is the history
// plus extra[0], extra[0], ..., extra[r-1], extra[r-1] (the proposals an
// accepted prefix records twice each); other parameters are left to the
// one-workgroup acceptance kernel.
template <bool ENG>
__global__ __launch_bounds__(kST) void k_tx_max(DevSampler* s, float* lg, int ld, int n, const int32_t* extra,
                                                 int extra_base, float* p, int ldp) {
    __shared__ SampScratch sh;
    const int r = blockIdx.y, g = blockIdx.x, tid = threadIdx.x;
    float* row = lg + (size_t)r * ld;
    if (!tx_split(s)) {
        if (!ENG && g == 0) transform_row(s, row, n, extra, extra_base + r, p + (size_t)r * ldp, sh);
        return;
    }
    const int b = g * kTxSlice, e = min(n, b + kTxSlice);
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = b + tid + j * kST;
        v[j] = i < e ? row[i] : -INFINITY;
    }
    if (s->pen > 1.f) {
        // sampler.cpp:15-27: each occurrence of an id in the window divides
        // (l > 0) or multiplies its logit by the penalty, in window order; an
        // id's value sees only its own occurrences, so applying them c times
        // in a row is the same sequence of operations.
        int* hits = (int*)sh.cand;
#pragma unroll
        for (int j = 0; j < 4; ++j) hits[tid + j * kST] = 0;
        __syncthreads();
        const int L = s->nh + (ENG ? 2 * r : extra_base + r);
        const int start = L - s->last > 0 ? L - s->last : 0;
        for (int q = start + tid; q < L; q += kST) {
            const int32_t id = q < s->nh ? s->hist[q] : extra[(q - s->nh) >> (ENG ? 1 : 0)];
            if (id >= b && id < e) atomicAdd(&hits[id - b], 1);
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < 4; ++j)
            for (int c = hits[tid + j * kST]; c > 0; --c) v[j] = v[j] > 0.f ? v[j] / s->pen : v[j] * s->pen;
    }
    const float T = s->temp;
    if (T != 1.f) {
        const float inv_t = 1.f / T;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] *= inv_t;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = b + tid + j * kST;
        if (i < e) {
            row[i] = v[j];
            mx = fmaxf(mx, v[j]);
        }
    }
    mx = block_max(mx, sh);
    if (tid == 0) {
        s->tx.mx[r][g] = mx;
        if (g == 0) s->tx.ovf[r] = 0;
    }
}

// Radix steps over a workgroup, 4-bit digits: each wave counts its keys'
// digits into its own 16 counters of one half of wc (2 x 16 x 16 LDS
// counters, the half by pass parity, so one barrier per pass).
// radix_buf clears this wave's counters of the pass (before its radix_count
// calls: a wave's LDS operations complete in order).
__device__ __forceinline__ unsigned int* radix_buf(unsigned int* wc, int shift) {
    unsigned int* buf = wc + ((shift >> 2) & 1) * 256 + (threadIdx.x >> 6) * 16;
    if ((threadIdx.x & 63) < 16) buf[threadIdx.x & 63] = 0;
    return buf;
}
__device__ __forceinline__ void radix_count(unsigned int key, bool valid, unsigned int mask, unsigned int prefix,
                                            int shift, unsigned int* buf) {
    if (valid && (key & mask) == prefix) atomicAdd(&buf[(key >> shift) & 15u], 1u);
}

// The counters are added up and the digit of the want-th largest key among
// those matching the prefix is chosen (want >= 1). above: keys above the
// chosen digit's range (counting the ones already above the prefix); returns
// the keys >= the new prefix. Every wave adds the counters up and selects by
// itself.
__device__ int radix_step(int want, int& above, unsigned int& prefix, unsigned int& mask, int shift,
                          const unsigned int* wc) {
    const int lane = threadIdx.x & 63;
    static_assert(kST / 64 == 16, "sixteen waves");
    const unsigned int* buf = wc + ((shift >> 2) & 1) * 256;
    __syncthreads();
    // lane l: digit l & 15 over waves l >> 4, + 4, + 8, + 12, then over the
    // four lane groups: every lane holds the count of its digit
    const int d = lane & 15, g = lane >> 4;
    unsigned int t = buf[g * 16 + d] + buf[(g + 4) * 16 + d] + buf[(g + 8) * 16 + d] + buf[(g + 12) * 16 + d];
    t += __shfl_xor(t, 16, 64);
    t += __shfl_xor(t, 32, 64);
    // count of digits d .. 15
    unsigned int sfx = t;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) {
        const unsigned int v = __shfl_down(sfx, o, 16);
        if (d + o < 16) sfx += v;
    }
    // digits 0 .. sel reach want (the suffix counts fall with d)
    const int sel = max(__popcll(__ballot(lane < 16 && above + (int)sfx >= want)) - 1, 0);
    const int s_sel = (int)__shfl(sfx, sel, 64), t_sel = (int)__shfl(t, sel, 64);
    const int ge = above + s_sel;
    above += s_sel - t_sel;
    prefix |= (unsigned int)sel << shift;
    mask |= 15u << shift;
    return ge;
}

__global__ __launch_bounds__(kST) void k_tx_exp(DevSampler* s, const float* lg, int ld, int n, float* p, int ldp) {
    if (!tx_split(s)) return;
    __shared__ unsigned int wc[2 * 16 * 16];
    __shared__ float red[kST / 64];
    __shared__ int ired[kST / 64], slots;
    const int r = blockIdx.y, g = blockIdx.x, tid = threadIdx.x, lane = tid & 63, G = gridDim.x;
    TxWork& w = s->tx;
    float mx = lane < G ? w.mx[r][lane] : -INFINITY;  // G <= 64: one slice maximum per lane
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    const int b = g * kTxSlice, e = min(n, b + kTxSlice);
    const float* row = lg + (size_t)r * ld;
    float* prow = p + (size_t)r * ldp;
    float ev[4];
    float sum = 0.f;
    int npos = 0;  // positive e, + 2^16 x those below 2^-31 (top key nibble under 3)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int i = b + tid + j * kST;
        ev[j] = 0.f;
        if (i < e) {
            ev[j] = expf(row[i] - mx);
            if (p) prow[i] = 0.f;
            sum += ev[j];
            npos += ev[j] > 0.f ? (ev[j] < 0x1p-31f ? 0x10001 : 1) : 0;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        sum += __shfl_xor(sum, o, 64);
        npos += __shfl_xor(npos, o, 64);
    }
    if (lane == 0) {
        red[tid >> 6] = sum;
        ired[tid >> 6] = npos;
    }
    if (tid == 0) slots = 0;
    __syncthreads();
    npos = 0;
    for (int i = 0; i < kST / 64; ++i) npos += ired[i];
    const bool nib3 = (npos >> 16) == 0;  // every positive e has key nibble 3 (2^-31 <= e <= 1)
    npos &= 0xFFFF;
    if (tid == 0) {
        float t = red[0];
        for (int i = 1; i < kST / 64; ++i) t += red[i];  // fixed order
        w.sum[r][g] = t;
    }
    const int want = min(s->top_k, npos);
    unsigned int prefix = 0, mask = 0;
    if (want > 0) {
        const int stop = max(want, kTxStop);  // candidates the slice may pass on
        int above = 0;
        if (nib3) {
            prefix = 0x30000000u;
            mask = 0xF0000000u;
        }
        for (int shift = nib3 ? 24 : 28; shift >= 0; shift -= 4) {
            unsigned int* buf = radix_buf(wc, shift);
#pragma unroll
            for (int j = 0; j < 4; ++j)
                radix_count(__builtin_bit_cast(unsigned int, ev[j]), ev[j] > 0.f, mask, prefix, shift, buf);
            if (radix_step(want, above, prefix, mask, shift, wc) <= stop) break;
        }
        // bound: 2^-20 below the threshold; below 2^-100 every positive e
        // (p = e / sum could then be subnormal, where rounding is not relative)
        const float t = __builtin_bit_cast(float, prefix);
        const float tm = t < 0x1p-100f ? 0.f : t * (1.f - 0x1p-20f);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (ev[j] > 0.f && ev[j] >= tm) {
                const int slot = atomicAdd(&slots, 1);
                if (slot < kTxCand)
                    w.cand[r][g][slot] = make_uint2(__builtin_bit_cast(unsigned int, ev[j]), (unsigned int)(b + tid + j * kST));
            }
    }
    __syncthreads();
    if (tid == 0) {
        w.nc[r][g] = min(slots, kTxCand);
        if (slots > kTxCand) w.ovf[r] = 1;
    }
}

// Sorts the m <= kST distinct keys src[0 .. m) ascending into dst by rank
// (each key's count of smaller keys). Whole workgroup; src and dst distinct.
__device__ void rank_sort(const unsigned long long* src, unsigned long long* dst, int m) {
    const int tid = threadIdx.x;
    if (tid < m) {
        const unsigned long long k = src[tid];
        int rank = 0;
        for (int j = 0; j < m; ++j) rank += src[j] < k;
        dst[rank] = k;
    }
    __syncthreads();
}

// topp_cut on wave 0 for k <= 128 candidates: the same running float sum in
// candidate order, the values read from the lanes instead of one at a time
// from LDS. Ends with a workgroup barrier.
__device__ void topp_cut_wave(float top_p, int k, SampScratch& sh) {
    const int tid = threadIdx.x;
    if (tid < 64) {
        const float a = tid < k ? cand_p(sh.cand[tid]) : 0.f;
        const float b = tid + 64 < k ? cand_p(sh.cand[tid + 64]) : 0.f;
        float cum = 0.f;
        int cut = k;
        for (int i = 0; i < k; ++i) {
            cum += i < 64 ? rdlane(a, i) : rdlane(b, i - 64);
            if (cum >= top_p) {
                cut = i + 1;
                break;
            }
        }
        if (tid == 0) {
            sh.bcast[4] = cut;
            sh.fb[0] = cum;  // the kept mass: the same sum over the first cut
        }
    }
    __syncthreads();
}

// One draw from the kept set sh.cand[0 .. cut) (p_out[id] = p / total), as
// k_draw does over the whole row: u * (sum of p_out in index order, double),
// first index where the running sum reaches it, the last one if rounding
// leaves it short. The set is put in index order first. Whole workgroup.
__device__ int32_t draw_kept(float u, int cut, float total, SampScratch& sh) {
    const int tid = threadIdx.x;
    unsigned long long* byid = (unsigned long long*)sh.dscan;  // (index, p_out bits), kST entries
    unsigned long long* src = byid + kST / 2;
    static_assert(kTxK <= kST / 2, "kept set fits half of the scan buffer");
    if (tid < cut) {
        const unsigned long long c = sh.cand[tid];
        const float pv = cand_p(c) / total;
        src[tid] = ((c & 0xFFFFFFFFull) << 32) | __builtin_bit_cast(unsigned int, pv);
    }
    __syncthreads();
    rank_sort(src, byid, cut);
    if (tid < 64) {  // wave 0, the entries passed between lanes
        const unsigned long long ea = tid < cut ? byid[tid] : 0ull, eb = tid + 64 < cut ? byid[tid + 64] : 0ull;
        auto entry = [&](int i) { return i < 64 ? rdlane(ea, i) : rdlane(eb, i - 64); };
        double tot = 0.0;
        for (int i = 0; i < cut; ++i) {
            const float pv = __builtin_bit_cast(float, (unsigned int)entry(i));
            if (pv > 0.f) tot += (double)pv;
        }
        double rr = (double)u * tot;
        int tok = -1, last = -1;
        for (int i = 0; i < cut; ++i) {
            const unsigned long long c = entry(i);
            const float pv = __builtin_bit_cast(float, (unsigned int)c);
            if (!(pv > 0.f)) continue;
            last = (int)(c >> 32);
            rr -= (double)pv;
            if (rr <= 0.0) {
                tok = last;
                break;
            }
        }
        if (tid == 0) sh.bcast[3] = tok >= 0 ? tok : max(last, 0);
    }
    __syncthreads();
    const int32_t tok = sh.bcast[3];
    __syncthreads();
    return tok;
}

// The kept set sh.cand[0 .. sh.bcast[4]) (at most kTxK) and its mass
// sh.fb[0] into the state's list of row r.
__device__ void keep_list(TxWork& w, int r, SampScratch& sh) {
    const int cut = sh.bcast[4];
    for (int i = threadIdx.x; i < cut; i += kST) {
        const unsigned long long c = sh.cand[i];
        w.kept[r][i] = make_uint2((unsigned int)(c & 0xFFFFFFFFu), __builtin_bit_cast(unsigned int, cand_p(c)));
    }
    if (threadIdx.x == 0) {
        w.cut[r] = cut;
        w.total[r] = sh.fb[0];
    }
}

// The split transform's last step for row blockIdx.x. MODE 0: p written;
// 1: p written and one draw from it into out[0] (and out2[0]); 2 (list): the
// kept set, its mass and size go to the state's scratch for
// k_accept_engine, p is not written.
template <int MODE>
__global__ __launch_bounds__(kST) void k_tx_final(DevSampler* s, float* lg, int ld, int n, float* p, int ldp,
                                                   int32_t* out, int32_t* out2) {
    constexpr bool DRAW = MODE == 1, LIST = MODE == 2;
    __shared__ SampScratch sh;
    const int r = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    float* prow = p + (size_t)r * ldp;
    int32_t tok = -1;
    if (tx_split(s)) {
        TxWork& w = s->tx;
        const int G = (n + kTxSlice - 1) / kTxSlice;
        const float sv = lane < G ? w.sum[r][lane] : 0.f;  // loads issued together
        const int ncv = lane < G ? w.nc[r][lane] : 0;
        const bool ovf = w.ovf[r] != 0;
        if (tid == 0 && !ovf) {  // through LDS, so both are read before the merge's first barrier
            sh.fb[2] = DRAW ? mt_canonical(s) : 0.f;
            sh.fb[3] = s->top_p;
        }
        if (ovf) {
            const int k = topk_sorted(s, lg + (size_t)r * ld, n, sh, true);
            if (LIST) {
                topp_cut(s, nullptr, k, sh);
                __syncthreads();
                keep_list(w, r, sh);
            } else {
                write_kept(s, k, prow, n, false, sh);
            }
        } else {
            // the row sum over the slice sums (fixed order), as every wave forms it
            float sum = sv;
#pragma unroll
            for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
            const float inv_s = 1.f / sum;
            int* off = (int*)sh.dscan;  // off[0 .. G]: exclusive prefix of the slice counts
            if (tid == 0) sh.bcast[6] = 0;  // set when a candidate's p is below 2^-31
            if (tid < 64) {
                const int c = ncv;
                int inc = c;  // inclusive scan over the wave
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int t = __shfl_up(inc, o, 64);
                    if (tid >= o) inc += t;
                }
                if (tid <= G) off[tid] = inc - c;
            }
            __syncthreads();
            const int N = off[G];
            // gather, wave w taking slices w, w + 16, ...: key = ~bits(p) << 32 |
            // index (p desc, index asc)
            for (int g = tid >> 6; g < G; g += kST / 64) {
                const int c0 = off[g], nc = off[g + 1] - c0;
#pragma unroll
                for (int j = lane; j < kTxCand; j += 64)
                    if (j < nc) {
                        const uint2 c = w.cand[r][g][j];
                        const float pv = __builtin_bit_cast(float, c.x) * inv_s;
                        if (pv < 0x1p-31f) sh.bcast[6] = 1;
                        sh.cand[c0 + j] = ((unsigned long long)(~__builtin_bit_cast(unsigned int, pv)) << 32) | c.y;
                    }
            }
            __syncthreads();
            // a prefix of p bits that the k-th largest p has and at most
            // max(k, kRank) candidates reach (the k-th largest itself when ties
            // leave more)
            const int k = min(s->top_k, n);
            const int want = min(k, N);
            constexpr int kRank = 64;
            unsigned int prefix = 0, mask = 0;
            int above = 0;
            if (N > max(want, kRank)) {
                const bool nib3 = sh.bcast[6] == 0;  // p <= 1: key nibble 3 unless p < 2^-31
                if (nib3) {
                    prefix = 0x30000000u;
                    mask = 0xF0000000u;
                }
                for (int shift = nib3 ? 24 : 28; shift >= 0; shift -= 4) {
                    unsigned int* buf = radix_buf(sh.hist, shift);
                    for (int i = tid; i < N; i += kST)
                        radix_count(~(unsigned int)(sh.cand[i] >> 32), true, mask, prefix, shift, buf);
                    if (radix_step(want, above, prefix, mask, shift, sh.hist) <= max(want, kRank)) break;
                }
            }
            // every candidate of the row's top k has p >= thr; sorted, the first
            // k of them are the ones the one-workgroup transform sorts first
            const unsigned int thr = prefix;
            if (tid == 0) sh.bcast[2] = 0;
            __syncthreads();
            unsigned long long* sel = (unsigned long long*)sh.dscan + 32;  // after off[]
            constexpr int kSel = kST - 32;
            static_assert((kTxMaxG + 1) * sizeof(int) <= 32 * sizeof(double), "offsets before the selection");
            for (int i = tid; i < N; i += kST) {
                const unsigned long long c = sh.cand[i];
                if (~(unsigned int)(c >> 32) >= thr) {
                    const int slot = atomicAdd(&sh.bcast[2], 1);
                    if (slot < kSel) sel[slot] = c;
                }
            }
            __syncthreads();
            const int m0 = sh.bcast[2];
            if (m0 <= kSel) {
                rank_sort(sel, sh.cand, m0);
            } else {  // many ties at the threshold: sort the whole candidate list
                for (int i = tid; i < N; i += kST)
                    if (~(unsigned int)(sh.cand[i] >> 32) < thr) sh.cand[i] = ~0ull;
                int mp = 1;
                while (mp < N) mp <<= 1;
                for (int i = N + tid; i < mp; i += kST) sh.cand[i] = ~0ull;
                __syncthreads();
                bitonic_sort(sh, mp);
            }
            const int kk = min(k, m0);
            topp_cut_wave(sh.fb[3], kk, sh);
            const int cut = sh.bcast[4];
            const float total = sh.fb[0];
            if (LIST) {
                keep_list(w, r, sh);
            } else {
                for (int i = tid; i < cut; i += kST) {
                    const int id = (int)(sh.cand[i] & 0xFFFFFFFFu);
                    prow[id] = cand_p(sh.cand[i]) / total;
                }
            }
            if (DRAW) tok = draw_kept(sh.fb[2], cut, total, sh);
        }
    }
    if (DRAW) {
        if (tok < 0) {  // the transform was the one-workgroup one: draw over the row as k_draw does
            const float u = lane0_uniform(s, sh);
            const double tt = block_total(prow, n, sh);
            tok = block_pick(n, [&](int i) { return prow[i]; }, (double)u * tt, sh);
        }
        if (tid == 0) {
            out[0] = tok;
            if (out2) out2[0] = tok;
        }
    }
}

__global__ __launch_bounds__(kST) void k_accept_resample(const float* p, const float* q, int n, int32_t x,
                                                          float u_acc, float u_res, int32_t* out) {
    __shared__ SampScratch sh;
    int acc = 0;
    const int32_t tok = accept_resample(p, q, n, x, u_acc, u_res, &acc, sh);
    if (threadIdx.x == 0) {
        out[0] = tok;
        out[1] = acc;
    }
}

// Speculative sampling acceptance chain over one round (no reference
// counterpart; replaces the Engine rule in the north-star mode): for proposal
// i (drawn from the draft's q_i), accept with min(1, p_i/q_i) or emit a draw
// from norm(max(0, p_i - q_i)) and stop; when all k are accepted emit a draw
// from p_k. Uniforms come from the state's mt19937 (acceptance, then the
// residual or bonus draw); emitted ids are recorded once. Output layout as
// k_accept_engine.
__global__ __launch_bounds__(kST) void k_accept_chain(DevSampler* s, const float* p, int ldp, const float* q, int ldq,
                                                       int n, const int32_t* x, int k, int max_emit, int32_t* d_budget,
                                                       int32_t* out, int32_t* d_pos, int32_t* d_next) {
    __shared__ SampScratch sh;
    if (d_budget) max_emit = *d_budget;
    int emitted = 0, accepted = 0, all = 0;
    int32_t last_tok = 0;
    for (int i = 0; i <= k && emitted < max_emit; ++i) {
        const float* pi = p + (size_t)i * ldp;
        int32_t tok;
        if (i == k) {
            const float u = lane0_uniform(s, sh);
            const double tot = block_total(pi, n, sh);
            tok = block_pick(n, [&](int j) { return pi[j]; }, (double)u * tot, sh);
            all = 1;
        } else {
            const float ua = lane0_uniform(s, sh);
            const float* qi = q + (size_t)i * ldq;
            const float qx = qi[x[i]], px = pi[x[i]];
            if (qx > 0.f && ua * qx < px) {
                tok = x[i];
                ++accepted;
            } else {
                const float ur = lane0_uniform(s, sh);
                int acc = 0;
                tok = accept_resample(pi, qi, n, x[i], 1.f, ur, &acc, sh);  // u_acc = 1: the residual branch
            }
        }
        if (threadIdx.x == 0) {
            record_tok(s, tok);
            out[4 + emitted] = tok;
        }
        __syncthreads();
        ++emitted;
        last_tok = tok;
        if (i == k || tok != x[i] || i + 1 > accepted) break;
    }
    if (threadIdx.x == 0) {
        out[0] = emitted;
        out[1] = accepted;
        out[2] = emitted;
        out[3] = all;
        if (d_pos) {
            *d_pos += emitted;
            *d_next = last_tok;
        }
        if (d_budget) *d_budget -= emitted;
    }
}

// ── the acceptance chain split over workgroups ──────────────────────────────
// k_accept_chain's rule in three launches: k_chain_scan walks the
// acceptance tests in order on one wave (the uniforms in the same order,
// accepted ids recorded); it ends at the first rejection (residual draw from
// max(0, p_i - q_i)), after k acceptances (bonus draw from p_k) or at the
// emission limit (no draw). k_chain_part sums the draw's weights per slice of
// kTxSlice entries (double; contiguous runs of four per thread, then the
// threads in order); k_chain_pick finds the slice and then the entry where
// the running sum reaches u * total (first entry whose cumulative sum is
// >= the target; the last positive one when rounding leaves the target
// unreached; argmax of p_i when the residual is empty), records it and
// writes the outputs. The sums associate differently from the one-workgroup
// kernel's chunks; both are double sums of the same float weights.
__global__ __launch_bounds__(64) void k_chain_scan(DevSampler* s, const float* p, int ldp, const float* q, int ldq,
                                                   const int32_t* x, int k, int max_emit, const int32_t* d_budget,
                                                   int32_t* out) {
    const int lane = threadIdx.x;
    TxWork& w = s->tx;
    if (d_budget) max_emit = *d_budget;
    int emitted = 0, accepted = 0, mode = 0, row = -1;
    float u = 0.f;
    for (int i = 0; i <= k && emitted < max_emit; ++i) {
        float ua = 0.f;
        if (lane == 0) ua = mt_canonical(s);
        ua = rdlane(ua, 0);
        if (i == k) {
            mode = 2;
            row = k;
            u = ua;
            break;
        }
        const int32_t xi = x[i];
        const float qx = q[(size_t)i * ldq + xi], px = p[(size_t)i * ldp + xi];
        if (qx > 0.f && ua * qx < px) {
            if (lane == 0) {
                record_tok(s, xi);
                out[4 + emitted] = xi;
            }
            ++emitted;
            ++accepted;
            continue;
        }
        float ur = 0.f;
        if (lane == 0) ur = mt_canonical(s);
        mode = 1;
        row = i;
        u = rdlane(ur, 0);
        break;
    }
    if (lane == 0) {
        w.ch_mode = mode;
        w.ch_row = row;
        w.ch_u = u;
        w.ch_emitted = emitted;
        w.ch_accepted = accepted;
        w.ch_max = max_emit;
    }
}

// the draw's weight of entry j: positive part of p_i - q_i (residual) or p_k
__device__ __forceinline__ float chain_w(int mode, const float* pr, const float* qr, int j) {
    const float d = mode == 1 ? pr[j] - qr[j] : pr[j];
    return d > 0.f ? d : 0.f;
}

__global__ __launch_bounds__(kST) void k_chain_part(DevSampler* s, const float* p, int ldp, const float* q, int ldq,
                                                    int n) {
    TxWork& w = s->tx;
    const int mode = w.ch_mode;
    if (mode == 0) return;
    __shared__ double red[kST / 64];
    __shared__ int lred[kST / 64];
    const int g = blockIdx.x, tid = threadIdx.x, row = w.ch_row;
    const float* pr = p + (size_t)row * ldp;
    const float* qr = mode == 1 ? q + (size_t)row * ldq : nullptr;
    const int b = g * kTxSlice + 4 * tid;
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = b + j < n ? chain_w(mode, pr, qr, b + j) : 0.f;
    double loc = 0.0;
    int last = -1;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        if (v[j] > 0.f) {
            loc += (double)v[j];
            last = b + j;
        }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        loc += __shfl_xor(loc, o, 64);
        last = max(last, __shfl_xor(last, o, 64));
    }
    if ((tid & 63) == 0) {
        red[tid >> 6] = loc;
        lred[tid >> 6] = last;
    }
    __syncthreads();
    if (tid == 0) {
        double t = 0.0;
        int l = -1;
        for (int i = 0; i < kST / 64; ++i) {  // waves in order
            t += red[i];
            l = max(l, lred[i]);
        }
        w.ch_sum[g] = t;
        w.ch_last[g] = l;
    }
}

__global__ __launch_bounds__(kST) void k_chain_pick(DevSampler* s, const float* p, int ldp, const float* q, int ldq,
                                                    int n, int k, int32_t* d_budget, int32_t* out, int32_t* d_pos,
                                                    int32_t* d_next) {
    __shared__ SampScratch sh;
    TxWork& w = s->tx;
    const int tid = threadIdx.x, lane = tid & 63;
    const int mode = w.ch_mode, row = w.ch_row;
    int emitted = w.ch_emitted;
    const int accepted = w.ch_accepted;
    int32_t tok = -1;
    if (mode != 0) {
        const float* pr = p + (size_t)row * ldp;
        const float* qr = mode == 1 ? q + (size_t)row * ldq : nullptr;
        const int G = (n + kTxSlice - 1) / kTxSlice;
        // slice sums: exclusive prefix in slice order, total (every wave alike)
        const double sg = lane < G ? w.ch_sum[lane] : 0.0;
        const int lg_ = lane < G ? w.ch_last[lane] : -1;
        double inc = sg;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const double t = __shfl_up(inc, o, 64);
            if (lane >= o) inc += t;
        }
        const double pre = inc - sg;
        const double total = __shfl(inc, 63, 64);
        int lastpos = lg_;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) lastpos = max(lastpos, __shfl_xor(lastpos, o, 64));
        if (mode == 1 && !(total > 0.0)) {
            tok = block_argmax(pr, n, sh);  // empty residual
        } else {
            const double target = (double)w.ch_u * total;
            // the slice holding the target: first one with weight whose range
            // (pre, pre + sum] contains it (target <= 0: the first with weight)
            const bool hit = lane < G && sg > 0.0 && (target <= 0.0 ? pre == 0.0 : (pre < target && target <= inc));
            const unsigned long long hb = __ballot(hit);
            if (hb == 0) {
                tok = max(lastpos, 0);  // rounding left the target unreached
            } else {
                const int gs = __ffsll((long long)hb) - 1;
                const double r0 = target - __shfl(pre, gs, 64);
                // inside the slice: runs of four per thread, prefix in thread order
                const int b = gs * kTxSlice + 4 * tid;
                float v[4];
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = b + j < n ? chain_w(mode, pr, qr, b + j) : 0.f;
                double loc = 0.0;
#pragma unroll
                for (int j = 0; j < 4; ++j) loc += (double)v[j];
                sh.dscan[tid] = loc;
                if (tid == 0) sh.bcast[5] = 0x7FFFFFFF;
                __syncthreads();
                if (tid < 64) {  // exclusive prefix over the threads, 16 per lane
                    double run = 0.0;
                    for (int i = 0; i < kST / 64; ++i) run += sh.dscan[tid * (kST / 64) + i];
                    double sc = run;
#pragma unroll
                    for (int o = 1; o < 64; o <<= 1) {
                        const double t = __shfl_up(sc, o, 64);
                        if (tid >= o) sc += t;
                    }
                    double at = sc - run;
                    for (int i = 0; i < kST / 64; ++i) {
                        const double c = sh.dscan[tid * (kST / 64) + i];
                        sh.dscan[tid * (kST / 64) + i] = at;
                        at += c;
                    }
                }
                __syncthreads();
                const double tp = sh.dscan[tid];
                if (loc > 0.0 && (r0 <= 0.0 ? tp == 0.0 : (tp < r0 && r0 <= tp + loc))) {
                    double rr = r0 - tp;
                    int got = -1, lastp = -1;
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (v[j] > 0.f) {
                            lastp = b + j;
                            rr -= (double)v[j];
                            if (rr <= 0.0 && got < 0) got = b + j;
                        }
                    atomicMin(&sh.bcast[5], got >= 0 ? got : lastp);
                }
                __syncthreads();
                tok = sh.bcast[5] != 0x7FFFFFFF ? sh.bcast[5] : max(w.ch_last[gs], 0);
            }
        }
    }
    if (tid == 0) {
        int all = 0;
        if (mode != 0) {
            record_tok(s, tok);
            out[4 + emitted] = tok;
            ++emitted;
            all = mode == 2;
        }
        out[0] = emitted;
        out[1] = accepted;
        out[2] = emitted;
        out[3] = all;
        if (d_pos) {
            *d_pos += emitted;
            *d_next = emitted > 0 ? out[4 + emitted - 1] : 0;  // the last emitted id
        }
        if (d_budget) *d_budget -= emitted;
    }
}

__global__ void k_sampler_history(const DevSampler* s, int32_t* out, int cap, int32_t* n_out) {
    if (threadIdx.x != 0) return;
    const int n = s->nh < cap ? s->nh : cap;
    for (int i = 0; i < n; ++i) out[i] = s->hist[s->nh - n + i];
    *n_out = n;
}

}  // namespace orc

using namespace orc;

// Host record of the sampler states initialised with top_k = 0 ("all
// tokens") and T > 0: their vocabulary must fit the candidate sort
// (kCandMax). The state itself is device memory the host never reads back.
static std::mutex g_all_mu;
static std::unordered_set<const void*> g_all_tokens;

static int check_vocab(const void* d_state, int n_vocab, const char* who) {
    if (n_vocab <= kCandMax) return ORC_OK;
    std::lock_guard<std::mutex> lk(g_all_mu);
    if (g_all_tokens.count(d_state))
        return set_error(ORC_E_UNSUPPORTED, std::string(who) + ": top_k = 0 (all tokens) supports vocabularies up to " +
                                                std::to_string(kCandMax) + " tokens");
    return ORC_OK;
}

extern "C" size_t orc_sampler_state_bytes(void) { return sizeof(DevSampler); }

// Rows the split transform takes: at most kTxRows of at most kTxMaxG slices.
static bool tx_shape(int n, int rows) { return rows <= kTxRows && n <= kTxMaxG * kTxSlice; }

// The split transform: p (and, with out, one draw) or, without p, the kept
// lists of the Engine rule's rows (extra = the proposals).
static void launch_tx(DevSampler* st, float* lg, int ld, int n, int rows, const int32_t* extra, int extra_base,
                      float* p, int ldp, int32_t* out, int32_t* out2, hipStream_t s) {
    const dim3 grid((n + kTxSlice - 1) / kTxSlice, rows);
    if (p)
        hipLaunchKernelGGL(k_tx_max<false>, grid, dim3(kST), 0, s, st, lg, ld, n, extra, extra_base, p, ldp);
    else
        hipLaunchKernelGGL(k_tx_max<true>, grid, dim3(kST), 0, s, st, lg, ld, n, extra, 0, p, ldp);
    hipLaunchKernelGGL(k_tx_exp, grid, dim3(kST), 0, s, st, (const float*)lg, ld, n, p, ldp);
    if (!p)
        hipLaunchKernelGGL(k_tx_final<2>, dim3(rows), dim3(kST), 0, s, st, lg, ld, n, p, ldp, out, out2);
    else if (out)
        hipLaunchKernelGGL(k_tx_final<1>, dim3(rows), dim3(kST), 0, s, st, lg, ld, n, p, ldp, out, out2);
    else
        hipLaunchKernelGGL(k_tx_final<0>, dim3(rows), dim3(kST), 0, s, st, lg, ld, n, p, ldp, out, out2);
}

extern "C" int orc_sampler_init(void* d_state, float temperature, float top_p, int top_k, float repeat_penalty,
                                int repeat_last, uint64_t seed, const int32_t* d_hist, int n_hist,
                                orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || repeat_last < 0 || repeat_last >= kSampHist || n_hist < 0 || (n_hist && !d_hist) ||
        top_k < 0 || top_k > kCandMax)
        return set_error(ORC_E_INVALID, "sampler_init: bad args (0 <= top_k <= 16384, 0 <= repeat_last < 4096)");
    {
        std::lock_guard<std::mutex> lk(g_all_mu);
        if (top_k == 0 && temperature > 0.f) g_all_tokens.insert(d_state);  // T <= 0 sorts nothing (argmax)
        else g_all_tokens.erase(d_state);
    }
    hipLaunchKernelGGL(k_sampler_init, dim3(1), dim3(64), 0, resolve_stream(s), (DevSampler*)d_state,
                       (uint32_t)seed, temperature, top_p, repeat_penalty, top_k, repeat_last, d_hist, n_hist);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_sampler_set_params(void* d_state, float temperature, float top_p, int top_k, float repeat_penalty,
                                      int repeat_last, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || repeat_last < 0 || repeat_last >= kSampHist || top_k < 0 || top_k > kCandMax)
        return set_error(ORC_E_INVALID, "sampler_set_params: bad args (0 <= top_k <= 16384, 0 <= repeat_last < 4096)");
    {
        std::lock_guard<std::mutex> lk(g_all_mu);
        if (top_k == 0 && temperature > 0.f) g_all_tokens.insert(d_state);  // T <= 0 sorts nothing (argmax)
        else g_all_tokens.erase(d_state);
    }
    hipLaunchKernelGGL(k_sampler_set, dim3(1), dim3(64), 0, resolve_stream(s), (DevSampler*)d_state, 1, temperature,
                       top_p, repeat_penalty, top_k, repeat_last);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_sampler_clear_history(void* d_state, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state) return set_error(ORC_E_INVALID, "sampler_clear_history: null state");
    hipLaunchKernelGGL(k_sampler_set, dim3(1), dim3(64), 0, resolve_stream(s), (DevSampler*)d_state, 0, 0.f, 0.f, 0.f,
                       0, 0);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_sample(void* d_state, float* d_logits, int n_vocab, int32_t* d_out, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || !d_logits || !d_out || n_vocab <= 0) return set_error(ORC_E_INVALID, "sample: bad args");
    if (int rc = check_vocab(d_state, n_vocab, "sample")) return rc;
    hipLaunchKernelGGL(k_sample, dim3(1), dim3(kST), 0, resolve_stream(s), (DevSampler*)d_state, d_logits, n_vocab,
                       d_out);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_sampler_record(void* d_state, const int32_t* d_tok, int n, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || n < 0 || (n && !d_tok)) return set_error(ORC_E_INVALID, "sampler_record: bad args");
    if (!n) return ORC_OK;
    hipLaunchKernelGGL(k_sampler_record, dim3(1), dim3(64), 0, resolve_stream(s), (DevSampler*)d_state, d_tok, n);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_sampler_history(const void* d_state, int32_t* d_out, int cap, int32_t* d_n, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || !d_out || !d_n || cap <= 0) return set_error(ORC_E_INVALID, "sampler_history: bad args");
    hipLaunchKernelGGL(k_sampler_history, dim3(1), dim3(64), 0, resolve_stream(s), (const DevSampler*)d_state,
                       d_out, cap, d_n);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_spec_accept_engine(void* d_state, float* d_logits, int ld, int n_vocab, const int32_t* d_draft,
                                      int n_draft, int max_emit, int32_t* d_budget, int32_t* d_out, int32_t* d_pos,
                                      int32_t* d_next, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || !d_logits || !d_out || n_vocab <= 0 || ld < n_vocab || n_draft < 0 || (n_draft && !d_draft) ||
        (max_emit < 1 && !d_budget) || (!d_pos) != (!d_next))
        return set_error(ORC_E_INVALID, "accept_engine: bad args");
    if (int rc = check_vocab(d_state, n_vocab, "accept_engine")) return rc;
    const int split = tx_shape(n_vocab, n_draft + 1);
    if (split)
        launch_tx((DevSampler*)d_state, d_logits, ld, n_vocab, n_draft + 1, d_draft, 0, nullptr, 0, nullptr, nullptr,
                  resolve_stream(s));
    hipLaunchKernelGGL(k_accept_engine, dim3(1), dim3(kST), 0, resolve_stream(s), (DevSampler*)d_state, d_logits,
                       ld, n_vocab, d_draft, n_draft, max_emit, d_budget, d_out, d_pos, d_next, split);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_transform_probs(const void* d_state, float* d_logits, int ld, int n_vocab, int rows,
                                   const int32_t* d_extra, int extra_base, float* d_p, int ldp, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || !d_logits || !d_p || n_vocab <= 0 || rows < 1 || ld < n_vocab || ldp < n_vocab ||
        extra_base < 0 || ((extra_base + rows > 1) && !d_extra))
        return set_error(ORC_E_INVALID, "transform_probs: bad args");
    if (int rc = check_vocab(d_state, n_vocab, "transform_probs")) return rc;
    if (tx_shape(n_vocab, rows)) {
        launch_tx((DevSampler*)const_cast<void*>(d_state), d_logits, ld, n_vocab, rows, d_extra, extra_base, d_p, ldp,
                  nullptr, nullptr, resolve_stream(s));
    } else {
        hipLaunchKernelGGL(k_transform, dim3(rows), dim3(kST), 0, resolve_stream(s), (const DevSampler*)d_state,
                           d_logits, ld, n_vocab, d_extra, extra_base, d_p, ldp);
    }
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_transform_draw(void* d_state, float* d_logits, int n_vocab, const int32_t* d_extra, int n_extra,
                                  float* d_p, int32_t* d_out, int32_t* d_out2, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || !d_logits || !d_p || !d_out || n_vocab <= 0 || n_extra < 0 || (n_extra && !d_extra))
        return set_error(ORC_E_INVALID, "transform_draw: bad args");
    if (int rc = check_vocab(d_state, n_vocab, "transform_draw")) return rc;
    const hipStream_t st = resolve_stream(s);
    if (tx_shape(n_vocab, 1)) {
        launch_tx((DevSampler*)d_state, d_logits, n_vocab, n_vocab, 1, d_extra, n_extra, d_p, n_vocab, d_out, d_out2,
                  st);
    } else {
        hipLaunchKernelGGL(k_transform, dim3(1), dim3(kST), 0, st, (const DevSampler*)d_state, d_logits, n_vocab,
                           n_vocab, d_extra, n_extra, d_p, n_vocab);
        hipLaunchKernelGGL(k_draw, dim3(1), dim3(kST), 0, st, (DevSampler*)d_state, (const float*)d_p, n_vocab, d_out,
                           d_out2);
    }
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_draw(void* d_state, const float* d_p, int n_vocab, int32_t* d_out, int32_t* d_out2,
                        orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || !d_p || !d_out || n_vocab <= 0) return set_error(ORC_E_INVALID, "draw: bad args");
    hipLaunchKernelGGL(k_draw, dim3(1), dim3(kST), 0, resolve_stream(s), (DevSampler*)d_state, d_p, n_vocab, d_out,
                       d_out2);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_accept_resample(const float* d_p, const float* d_q, int n_vocab, int32_t x, float u_acc,
                                   float u_res, int32_t* d_out, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_p || !d_q || !d_out || n_vocab <= 0 || x < 0 || x >= n_vocab)
        return set_error(ORC_E_INVALID, "accept_resample: bad args");
    hipLaunchKernelGGL(k_accept_resample, dim3(1), dim3(kST), 0, resolve_stream(s), d_p, d_q, n_vocab, x, u_acc,
                       u_res, d_out);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_spec_accept_stochastic(void* d_state, const float* d_p, int ldp, const float* d_q, int ldq,
                                          int n_vocab, const int32_t* d_x, int k, int max_emit, int32_t* d_budget,
                                          int32_t* d_out, int32_t* d_pos, int32_t* d_next, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (!d_state || !d_p || !d_out || n_vocab <= 0 || ldp < n_vocab || k < 0 || (k && (!d_q || !d_x || ldq < n_vocab)) ||
        (max_emit < 1 && !d_budget) || (!d_pos) != (!d_next))
        return set_error(ORC_E_INVALID, "accept_stochastic: bad args");
    const hipStream_t st = resolve_stream(s);
    DevSampler* ds = (DevSampler*)d_state;
    if (n_vocab <= kTxMaxG * kTxSlice) {
        hipLaunchKernelGGL(k_chain_scan, dim3(1), dim3(64), 0, st, ds, d_p, ldp, d_q, ldq, d_x, k, max_emit,
                           (const int32_t*)d_budget, d_out);
        hipLaunchKernelGGL(k_chain_part, dim3((n_vocab + kTxSlice - 1) / kTxSlice), dim3(kST), 0, st, ds, d_p, ldp,
                           d_q, ldq, n_vocab);
        hipLaunchKernelGGL(k_chain_pick, dim3(1), dim3(kST), 0, st, ds, d_p, ldp, d_q, ldq, n_vocab, k, d_budget,
                           d_out, d_pos, d_next);
    } else {
        hipLaunchKernelGGL(k_accept_chain, dim3(1), dim3(kST), 0, st, ds, d_p, ldp, d_q, ldq, n_vocab, d_x, k,
                           max_emit, d_budget, d_out, d_pos, d_next);
    }
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

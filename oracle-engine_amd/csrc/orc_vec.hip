// Device kernels behind the reference's free functions on raw float arrays
// (namespace ops, core/ops.hpp:42-92): elementwise mul / add / copy, SiLU,
// softmax, dot, the two fp32 matmuls and RoPE on one position. The host
// mirror of namespace ops (host/ops.cpp) stages host arrays through these;
// rmsnorm and argmax use orc_rmsnorm and orc_argmax_noalloc.
//
// Numerics: fp32 throughout. Reductions (softmax sum, dot, matmul) run in a
// fixed order per launch shape (lane-strided partial sums, then a fixed
// butterfly), not the reference's 8-lane AVX order, so results agree with it
// to fp32 summation order. exp is the device expf.
#include "orc_internal.hpp"

namespace orc {

constexpr int kVT = 256;  // threads per block of the reductions

__global__ void k_vec_binary(int op, float* out, const float* a, const float* b, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (op == ORC_VEC_MUL) out[i] = a[i] * b[i];       // ops.cpp:339-354
    else if (op == ORC_VEC_ADD) out[i] = a[i] + b[i];  // ops.cpp:359-374
    else out[i] = a[i];                                // ops.cpp:379-381
}

// x / (1 + exp(-x)), ops.cpp:308-334
__global__ void k_vec_silu(float* x, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] / (1.f + expf(-x[i]));
}

// Block sum / max over kVT threads in a fixed order (wave butterfly, then the
// waves in index order).
__device__ float block_sum(float v, float* sh) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float s = 0.f;
    for (int i = 0; i < kVT / 64; ++i) s += sh[i];
    return s;
}
__device__ float block_max(float v, float* sh) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) sh[w] = v;
    __syncthreads();
    float m = sh[0];
    for (int i = 1; i < kVT / 64; ++i) m = fmaxf(m, sh[i]);
    return m;
}

// One block per row: x = exp(x - max) / sum, ops.cpp:386-435.
__global__ __launch_bounds__(kVT) void k_softmax(float* x, int n, int ld) {
    __shared__ float sh[kVT / 64];
    float* r = x + (size_t)blockIdx.x * ld;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += kVT) m = fmaxf(m, r[i]);
    m = block_max(m, sh);
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += kVT) {
        const float e = expf(r[i] - m);
        r[i] = e;
        s += e;
    }
    s = block_sum(s, sh);
    const float inv = 1.f / s;
    for (int i = threadIdx.x; i < n; i += kVT) r[i] *= inv;
}

// sum a[i] b[i], ops.cpp:102-143
__global__ __launch_bounds__(kVT) void k_dot(const float* a, const float* b, int n, float* out) {
    __shared__ float sh[kVT / 64];
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += kVT) s = __builtin_fmaf(a[i], b[i], s);
    s = block_sum(s, sh);
    if (threadIdx.x == 0) *out = s;
}

// out[i][j] = sum_l A[i][l] B'[l][j]: B' = B^T (B n x k, ops::matmul,
// ops.cpp:207-289) or B (k x n, ops::matmul_nn, ops.cpp:294-303). One wave
// per output; lanes stride over l, then a butterfly.
__global__ __launch_bounds__(kVT) void k_matmul(float* out, const float* A, const float* B, int m, int n, int k,
                                                int b_trans) {
    const int o = blockIdx.x * (kVT / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (o >= m * n) return;
    const int i = o / n, j = o % n;
    const float* ar = A + (size_t)i * k;
    float s = 0.f;
    if (b_trans) {
        const float* br = B + (size_t)j * k;
        for (int l = lane; l < k; l += 64) s = __builtin_fmaf(ar[l], br[l], s);
    } else {
        for (int l = lane; l < k; l += 64) s = __builtin_fmaf(ar[l], B[(size_t)l * n + j], s);
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) s += __shfl_xor(s, d, 64);
    if (lane == 0) out[(size_t)i * n + j] = s;
}

// Rotate-half RoPE of one position on n_heads q heads and n_kv k heads with
// the (cos, sin) pairs of the position, ops.cpp:440-485.
__global__ void k_rope_pos(float* q, float* k, int n_heads, int n_kv, int hd, const float* cs) {
    const int half = hd / 2;
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    const int h = t / half, i = t % half;
    if (h >= n_heads + n_kv) return;
    float* v = h < n_heads ? q + (size_t)h * hd : k + (size_t)(h - n_heads) * hd;
    const float c = cs[2 * i], s = cs[2 * i + 1];
    const float v0 = v[i], v1 = v[i + half];
    v[i] = v0 * c - v1 * s;
    v[i + half] = v0 * s + v1 * c;
}

}  // namespace orc

using namespace orc;

static int grid_of(int n, int t) { return (n + t - 1) / t; }

extern "C" int orc_vec_binary(int op, float* d_out, const float* d_a, const float* d_b, int n, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (op != ORC_VEC_MUL && op != ORC_VEC_ADD && op != ORC_VEC_COPY)
        return set_error(ORC_E_INVALID, "vec_binary: op must be ORC_VEC_MUL, ORC_VEC_ADD or ORC_VEC_COPY");
    if (n < 0 || (n && (!d_out || !d_a || (op != ORC_VEC_COPY && !d_b))))
        return set_error(ORC_E_INVALID, "vec_binary: bad args");
    if (!n) return ORC_OK;
    hipLaunchKernelGGL(k_vec_binary, dim3(grid_of(n, 256)), dim3(256), 0, resolve_stream(s), op, d_out, d_a, d_b, n);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_vec_silu(float* d_x, int n, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n < 0 || (n && !d_x)) return set_error(ORC_E_INVALID, "vec_silu: bad args");
    if (!n) return ORC_OK;
    hipLaunchKernelGGL(k_vec_silu, dim3(grid_of(n, 256)), dim3(256), 0, resolve_stream(s), d_x, n);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_softmax(float* d_x, int n, int n_rows, int ld, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n < 0 || n_rows < 0 || ((n && n_rows) && (!d_x || ld < n))) return set_error(ORC_E_INVALID, "softmax: bad args");
    if (!n || !n_rows) return ORC_OK;
    hipLaunchKernelGGL(k_softmax, dim3(n_rows), dim3(kVT), 0, resolve_stream(s), d_x, n, ld);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_dot(const float* d_a, const float* d_b, int n, float* d_out, orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n < 0 || !d_out || (n && (!d_a || !d_b))) return set_error(ORC_E_INVALID, "dot: bad args");
    hipLaunchKernelGGL(k_dot, dim3(1), dim3(kVT), 0, resolve_stream(s), d_a, d_b, n, d_out);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_matmul_f32(float* d_out, const float* d_a, const float* d_b, int m, int n, int k, int b_trans,
                              orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (m < 0 || n < 0 || k < 0 || ((int64_t)m * n > 0x7fffffff) || (m && n && (!d_out || (k && (!d_a || !d_b)))))
        return set_error(ORC_E_INVALID, "matmul_f32: bad args");
    if (!m || !n) return ORC_OK;
    hipLaunchKernelGGL(k_matmul, dim3(grid_of(m * n, kVT / 64)), dim3(kVT), 0, resolve_stream(s), d_out, d_a, d_b, m,
                       n, k, b_trans ? 1 : 0);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

extern "C" int orc_rope_pos(float* d_q, float* d_k, int n_heads, int n_kv_heads, int head_dim, const float* d_cs,
                            orc_stream_t s) {
    if (!initialized()) return set_error(ORC_E_NOINIT, "orc_init not called");
    if (n_heads < 0 || n_kv_heads < 0 || head_dim < 2 || !d_cs || (n_heads && !d_q) ||
        (n_kv_heads && !d_k))
        return set_error(ORC_E_INVALID, "rope_pos: bad args");
    const int n = (n_heads + n_kv_heads) * (head_dim / 2);
    if (!n) return ORC_OK;
    hipLaunchKernelGGL(k_rope_pos, dim3(grid_of(n, 256)), dim3(256), 0, resolve_stream(s), d_q, d_k, n_heads,
                       n_kv_heads, head_dim, d_cs);
    ORC_LAUNCH_CHECK();
    return ORC_OK;
}

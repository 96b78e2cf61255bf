// The reference's free functions on raw float arrays (core/ops.hpp:1-94),
// same names, signatures and in-place conventions, computed on the GPU: each
// call copies its host arrays into a reused device staging buffer, runs the
// kernel (liborc_hip: orc_rmsnorm, orc_vec_*, orc_softmax, orc_dot,
// orc_matmul_f32, orc_rope_pos, orc_argmax_noalloc) and copies the results
// back. Results match the reference's loops to fp32 summation order; argmax
// is exact (first index of the maximum). Thread-safe (one staging buffer
// under a lock). A device error is reported on stderr and leaves the output
// as the device wrote it (the reference's functions cannot fail).
#pragma once
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <vector>

// Row-major 2-D float array (core/ops.hpp:11-34).
struct Tensor {
    std::vector<float> data;
    int rows = 0;
    int cols = 0;

    Tensor() = default;
    Tensor(int r, int c) : data((size_t)r * c, 0.f), rows(r), cols(c) {}

    void resize(int r, int c) {
        rows = r;
        cols = c;
        data.assign((size_t)r * c, 0.f);
    }
    void zero() { std::fill(data.begin(), data.end(), 0.f); }

    float& at(int r, int c) { return data[(size_t)r * cols + c]; }
    float at(int r, int c) const { return data[(size_t)r * cols + c]; }

    float* ptr(int r = 0) { return data.data() + (size_t)r * cols; }
    const float* ptr(int r = 0) const { return data.data() + (size_t)r * cols; }

    int n_elems() const { return rows * cols; }
};

namespace ops {

// out = x / sqrt(mean(x^2) + eps) * weight (core/ops.hpp:42-43)
void rmsnorm(float* out, const float* x, const float* weight, int n, float eps = 1e-5f);
// out (m x n) = A (m x k) x B^T, B n x k (core/ops.hpp:49-50)
void matmul(float* out, const float* A, const float* B, int m, int n, int k);
// out (m x n) = A (m x k) x B, B k x n (core/ops.hpp:53-54)
void matmul_nn(float* out, const float* A, const float* B, int m, int n, int k);
// x = x * sigmoid(x) in place (core/ops.hpp:59)
void silu(float* x, int n);
// out = a * b (core/ops.hpp:64)
void mul(float* out, const float* a, const float* b, int n);
// a += b (core/ops.hpp:67)
void add(float* a, const float* b, int n);
// dst = src (core/ops.hpp:70)
void copy(float* dst, const float* src, int n);
// in-place softmax (core/ops.hpp:75)
void softmax(float* x, int n);
// rotate-half RoPE of position pos on q and k in place (core/ops.hpp:82-84)
void rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int pos, float freq_base = 500000.f);
// first index of the maximum; 0 for n <= 0 (core/ops.hpp:89)
int argmax(const float* x, int n);
// sum a[i] b[i] (core/ops.hpp:92)
float dot(const float* a, const float* b, int n);

}  // namespace ops

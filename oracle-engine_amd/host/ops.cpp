// namespace ops on host arrays, computed on the GPU (the declarations say how).
#include "ops.hpp"

#include "orc.h"

#include <cstdio>
#include <mutex>

namespace {

// Device staging shared by every call: grow-only, guarded by one lock (the
// copies in and out are synchronous, so a call leaves nothing in flight).
struct Stage {
    std::mutex mu;
    void* d = nullptr;
    size_t cap = 0;
    bool init = false;
};
Stage& stage() {
    static Stage s;
    return s;
}

// Holds the lock for one call; at(i) is the i-th float region of the layout
// given at construction (each region rounded up to 256 bytes).
class Call {
public:
    Call(std::initializer_list<size_t> floats) : lk_(stage().mu) {
        Stage& s = stage();
        if (!s.init) {
            ok_ = orc_init(0) == ORC_OK;
            s.init = ok_;
        }
        size_t off = 0;
        for (size_t n : floats) {
            off_.push_back(off);
            off += (n * sizeof(float) + 255) / 256 * 256;
        }
        if (ok_ && off > s.cap) {
            if (s.d) orc_free(s.d);
            s.d = nullptr;
            s.cap = 0;
            ok_ = orc_malloc(&s.d, off) == ORC_OK;
            if (ok_) s.cap = off;
        }
        if (!ok_) report("device staging");
    }
    bool ok() const { return ok_; }
    float* at(int i) const { return (float*)((char*)stage().d + off_[i]); }
    void put(int i, const float* h, size_t n) { check(orc_memcpy_h2d(at(i), h, n * sizeof(float), nullptr), "copy in"); }
    void get(float* h, int i, size_t n) { check(orc_memcpy_d2h(h, at(i), n * sizeof(float), nullptr), "copy out"); }
    void check(int rc, const char* what) {
        if (rc != ORC_OK && ok_) {
            ok_ = false;
            report(what);
        }
    }

private:
    std::lock_guard<std::mutex> lk_;
    std::vector<size_t> off_;
    bool ok_ = true;
    static void report(const char* what) { std::fprintf(stderr, "[ops] %s failed: %s\n", what, orc_last_error()); }
};

}  // namespace

namespace ops {

void rmsnorm(float* out, const float* x, const float* weight, int n, float eps) {  // ops.cpp:149-195
    if (n <= 0) return;
    Call c({(size_t)n, (size_t)n, (size_t)n});
    if (!c.ok()) return;
    c.put(0, x, n);
    c.put(1, weight, n);
    c.check(orc_rmsnorm(c.at(2), c.at(0), c.at(1), n, 1, eps, nullptr), "rmsnorm");
    if (c.ok()) c.get(out, 2, n);
}

static void mm(float* out, const float* A, const float* B, int m, int n, int k, int b_trans) {
    if (m <= 0 || n <= 0) return;
    const size_t na = (size_t)m * (k > 0 ? k : 0), nb = (size_t)n * (k > 0 ? k : 0), no = (size_t)m * n;
    Call c({na, nb, no});
    if (!c.ok()) return;
    if (na) c.put(0, A, na);
    if (nb) c.put(1, B, nb);
    c.check(orc_matmul_f32(c.at(2), c.at(0), c.at(1), m, n, k > 0 ? k : 0, b_trans, nullptr), "matmul");
    if (c.ok()) c.get(out, 2, no);
}

void matmul(float* out, const float* A, const float* B, int m, int n, int k) { mm(out, A, B, m, n, k, 1); }
void matmul_nn(float* out, const float* A, const float* B, int m, int n, int k) { mm(out, A, B, m, n, k, 0); }

void silu(float* x, int n) {  // ops.cpp:308-334
    if (n <= 0) return;
    Call c({(size_t)n});
    if (!c.ok()) return;
    c.put(0, x, n);
    c.check(orc_vec_silu(c.at(0), n, nullptr), "silu");
    if (c.ok()) c.get(x, 0, n);
}

static void binary(int op, float* out, const float* a, const float* b, int n) {
    if (n <= 0) return;
    Call c({(size_t)n, (size_t)n});
    if (!c.ok()) return;
    c.put(0, a, n);
    if (b) c.put(1, b, n);
    c.check(orc_vec_binary(op, c.at(0), c.at(0), b ? c.at(1) : nullptr, n, nullptr), "elementwise");
    if (c.ok()) c.get(out, 0, n);
}

void mul(float* out, const float* a, const float* b, int n) { binary(ORC_VEC_MUL, out, a, b, n); }
void add(float* a, const float* b, int n) { binary(ORC_VEC_ADD, a, a, b, n); }
void copy(float* dst, const float* src, int n) { binary(ORC_VEC_COPY, dst, src, nullptr, n); }

void softmax(float* x, int n) {  // ops.cpp:386-435
    if (n <= 0) return;
    Call c({(size_t)n});
    if (!c.ok()) return;
    c.put(0, x, n);
    c.check(orc_softmax(c.at(0), n, 1, n, nullptr), "softmax");
    if (c.ok()) c.get(x, 0, n);
}

void rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int pos, float freq_base) {
    // ops.cpp:440-485: the position's angles with the reference's float
    // arithmetic on the host, the rotation on the device; an odd head_dim
    // rotates the pairs (i, i + head_dim / 2) and leaves the last value
    if (head_dim < 2 || n_heads < 0 || n_kv_heads < 0) return;
    const int half = head_dim / 2;
    std::vector<float> cs((size_t)2 * half);
    for (int i = 0; i < half; ++i) {
        const float theta = (float)pos / std::pow(freq_base, (float)(2 * i) / (float)head_dim);
        cs[2 * i] = std::cos(theta);
        cs[2 * i + 1] = std::sin(theta);
    }
    const size_t nq = (size_t)n_heads * head_dim, nk = (size_t)n_kv_heads * head_dim;
    Call c({nq, nk, cs.size()});
    if (!c.ok()) return;
    if (nq) c.put(0, q, nq);
    if (nk) c.put(1, k, nk);
    c.put(2, cs.data(), cs.size());
    c.check(orc_rope_pos(c.at(0), c.at(1), n_heads, n_kv_heads, head_dim, c.at(2), nullptr), "rope");
    if (c.ok() && nq) c.get(q, 0, nq);
    if (c.ok() && nk) c.get(k, 1, nk);
}

int argmax(const float* x, int n) {  // ops.cpp:490-497
    if (n <= 0) return 0;
    Call c({(size_t)n, 1});
    if (!c.ok()) return 0;
    c.put(0, x, n);
    c.check(orc_argmax_noalloc(c.at(0), 1, n, n, (int32_t*)c.at(1), nullptr), "argmax");
    int32_t id = 0;
    if (c.ok()) c.check(orc_memcpy_d2h(&id, c.at(1), sizeof(id), nullptr), "copy out");
    return id;
}

float dot(const float* a, const float* b, int n) {  // ops.cpp:102-143
    if (n <= 0) return 0.f;
    Call c({(size_t)n, (size_t)n, 1});
    if (!c.ok()) return 0.f;
    c.put(0, a, n);
    c.put(1, b, n);
    c.check(orc_dot(c.at(0), c.at(1), n, c.at(2), nullptr), "dot");
    float r = 0.f;
    if (c.ok()) c.get(&r, 2, 1);
    return r;
}

}  // namespace ops

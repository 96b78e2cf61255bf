#include "spec.hpp"

#include <algorithm>
#include <cstdio>

DecodeSession::DecodeSession(int max_tokens, int max_k) : max_tokens_(max_tokens), max_k_(max_k) {
    orc_malloc((void**)&d_hist_, (size_t)(max_tokens + 2) * 4);
    orc_malloc((void**)&d_vin_, (size_t)(max_k + 2) * 4);
    orc_malloc((void**)&d_tgt_, (size_t)(max_k + 2) * 4);
    orc_malloc((void**)&d_acc_, 4 * 4);
}

DecodeSession::~DecodeSession() {
    orc_free(d_hist_);
    orc_free(d_vin_);
    orc_free(d_tgt_);
    orc_free(d_acc_);
}

int DecodeSession::prefill(Model& m, const int32_t* prompt, int n_prompt) {
    if (n_prompt < 2) return 0;
    m.forward_prefill(prompt, n_prompt - 1, 0, nullptr);
    return 0;
}

// The argmax of step s is written straight into the input slot of step s+1,
// so the whole chain is enqueued without a host round trip.
int DecodeSession::greedy(Model& m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out) {
    if (n_gen > max_tokens_ || n_prompt < 1) return ORC_E_INVALID;
    int pos = n_prompt - 1;
    if (pos + n_gen > (int)m.cfg.ctx_len) return ORC_E_INVALID;
    int32_t first = prompt[n_prompt - 1];
    if (first < 0 || first >= (int32_t)m.cfg.n_vocab) first = 0;
    if (int rc = orc_memcpy_h2d(d_hist_, &first, 4, nullptr)) return rc;
    for (int s = 0; s < n_gen; ++s)
        if (int rc = m.forward_dev(d_hist_ + s, 1, pos + s, true, d_hist_ + s + 1)) return rc;
    if (int rc = orc_memcpy_d2h(out, d_hist_ + 1, (size_t)n_gen * 4, nullptr)) return rc;
    return n_gen;
}

int DecodeSession::spec_greedy(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                               int32_t* out, SpecStats* st) {
    if (k < 1 || k > max_k_ || n_prompt < 1) return ORC_E_INVALID;
    if (dft.cfg.n_vocab != tgt.cfg.n_vocab) return ORC_E_INVALID;  // bench_engine.cpp:290-293
    SpecStats local;
    SpecStats& S = st ? *st : local;
    int pos = n_prompt - 1, ng = 0;
    int32_t next = prompt[n_prompt - 1];
    if (next < 0 || next >= (int32_t)tgt.cfg.n_vocab) next = 0;
    const int ctx = (int)std::min(tgt.cfg.ctx_len, dft.cfg.ctx_len);
    std::vector<int32_t> ids(k + 2);
    while (ng < n_gen && pos + k + 1 <= ctx) {
        if (int rc = orc_memcpy_h2d(d_vin_, &next, 4, nullptr)) return rc;
        // (a) k greedy draft proposals; draft step i writes d_i into d_vin[i+1]
        for (int i = 0; i < k; ++i)
            if (int rc = dft.forward_dev(d_vin_ + i, 1, pos + i, true, d_vin_ + i + 1)) return rc;
        S.proposed += k;
        // (b) one (k+1)-token verify pass of the target over [next, d0 .. d_{k-1}]
        if (int rc = tgt.forward_dev(d_vin_, k + 1, pos, true, d_tgt_)) return rc;
        S.passes++;
        S.rounds++;
        // (c) acceptance on the device; ids and count to the host
        if (int rc = orc_spec_accept_greedy(d_tgt_, d_vin_ + 1, k, d_acc_, nullptr)) return rc;
        int32_t acc[2];
        if (int rc = orc_memcpy_d2h(ids.data(), d_tgt_, (size_t)(k + 1) * 4, nullptr)) return rc;
        if (int rc = orc_memcpy_d2h(acc, d_acc_, 8, nullptr)) return rc;
        const int a = acc[0];
        // emitted tokens are tgt[0..a]: a accepted draft tokens, then the
        // mismatch or the bonus token, capped at n_gen
        bool capped = false;
        for (int i = 0; i <= a; ++i) {
            out[ng++] = ids[i];
            if (i < a) S.accepted++;
            if (ng >= n_gen) { capped = true; break; }
        }
        next = ids[a];
        if (a == k && !capped) {
            // all accepted: the draft still lacks d_{k-1} at position pos+k
            if (int rc = dft.forward_dev(d_vin_ + k, 1, pos + k, false, nullptr)) return rc;
        }
        pos += a + 1;
    }
    orc_stream_sync(nullptr);
    return ng;
}

#include "spec.hpp"

#include <algorithm>
#include <cstdio>

DecodeSession::DecodeSession(int max_tokens, int max_k) : max_tokens_(max_tokens), max_k_(max_k) {
    // orc_init is idempotent; the session may be created before any model is
    // loaded. A failed step leaves the session unusable: every loop then
    // returns the recorded error instead of launching on null buffers.
    auto need = [&](int rc, const char* what) {
        if (rc != ORC_OK && init_rc_ == ORC_OK) {
            init_rc_ = rc;
            init_err_ = std::string("DecodeSession: ") + what + ": " + orc_last_error();
        }
    };
    need(orc_init(0), "orc_init");
    if (max_tokens < 1 || max_k < 1) {
        init_rc_ = ORC_E_INVALID;
        init_err_ = "DecodeSession: max_tokens and max_k must be positive";
        return;
    }
    need(orc_malloc((void**)&d_hist_, (size_t)(max_tokens + 2) * 4), "device allocation");
    need(orc_malloc((void**)&d_vin_, (size_t)(max_k + 2) * 4), "device allocation");
    need(orc_malloc((void**)&d_tgt_, (size_t)(max_k + 2) * 4), "device allocation");
    need(orc_malloc((void**)&d_acc_, (size_t)(max_k + 4) * 4), "device allocation");
    need(orc_malloc((void**)&d_pos_, 4 * 4), "device allocation");
    need(orc_malloc((void**)&d_tok_, 4 * 4), "device allocation");
    need(orc_malloc(&d_samp_, orc_sampler_state_bytes()), "device allocation");
    need(orc_malloc((void**)&d_eout_, (size_t)(max_k + 8) * 4), "device allocation");
    need(orc_malloc((void**)&d_budget_, 4), "device allocation");
}

DecodeSession::~DecodeSession() {
    for (int i = 0; i < kBands; ++i) {
        drop(greedy_g_[i]);
        drop(spec_g_[i]);
        drop(eng_g_[i]);
        drop(smp_g_[i]);
    }
    orc_free(d_p_);
    orc_free(d_q_);
    orc_free(d_samp_);
    orc_free(d_eout_);
    orc_free(d_budget_);
    orc_free(d_hist_);
    orc_free(d_vin_);
    orc_free(d_tgt_);
    orc_free(d_acc_);
    orc_free(d_pos_);
    orc_free(d_tok_);
}

void DecodeSession::drop(Captured& c) {
    orc_graph_destroy(c.g);
    orc_graph_destroy(c.fill);
    c = Captured();
}

// Position bound recorded into a run's graphs: the run's last position + 1
// rounded up to a power of two (at least 512), capped at the context. It
// sizes the attention grids of short runs.
static int graph_limit(int need, int ctx) {
    int lim = 512;
    while (lim < need && lim < ctx) lim *= 2;
    return std::min(lim, ctx);
}

// Band of a replay whose positions lie in [p_lo, p_hi]: 0 when all attend to
// at most T = orc_attn_wg_limit() positions (p < T), 2 when none does, 1 when
// they straddle T; the limit of bands 1 and 2 is the run's.
DecodeSession::Band DecodeSession::band_of(int p_lo, int p_hi, int run_lim, int ctx) {
    const int T = orc_attn_wg_limit();
    if (p_hi < T) return {0, 0, std::min(T, ctx)};
    if (p_lo >= T) return {2, T, run_lim};
    return {1, 0, run_lim};
}

DecodeSession::Captured& DecodeSession::slot(Captured (&set)[kBands], const Band& b, uint64_t a, uint64_t bb, int k) {
    Captured& c = set[b.idx];
    if (c.a != a || c.b != bb || c.k != k || c.floor != b.floor || c.lim != b.lim || !c.g) {
        drop(c);
        c.floor = b.floor;
        c.lim = b.lim;
    }
    return c;
}

// Sets the position band of the models for the passes being captured and
// clears it again when the capture is done.
struct BandScope {
    Model *a, *b;
    BandScope(Model& x, Model* y, int floor, int lim) : a(&x), b(y) {
        a->set_pos_band(floor, lim);
        if (b) b->set_pos_band(floor, lim);
    }
    ~BandScope() {
        a->set_pos_band(0, 0);
        if (b) b->set_pos_band(0, 0);
    }
};

// Ends a capture that failed part-way so the stream leaves capture mode.
static int abort_capture(int rc) {
    orc_graph_t g = nullptr;
    if (orc_graph_end(nullptr, &g) == 0) orc_graph_destroy(g);
    return rc;
}

// One captured greedy step: forward at *d_pos with input d_tok[0], argmax
// into d_tok[1], then append / advance on the device.
int DecodeSession::greedy_graphed(Model& m, int pos, int32_t first, int n_gen, int32_t* out) {
    const int ctx = (int)m.cfg.ctx_len;
    const int run_lim = graph_limit(pos + n_gen + 1, ctx);
    const int32_t state[2] = {pos, 0};
    if (int rc = orc_memcpy_h2d(d_pos_, state, 8, nullptr)) return rc;
    if (int rc = orc_memcpy_h2d(d_tok_, &first, 4, nullptr)) return rc;
    for (int s = 0; s < n_gen; ++s) {
        const Band b = band_of(pos + s, pos + s, run_lim, ctx);
        Captured& c = slot(greedy_g_, b, m.uid(), 0, 1);
        if (!c.g) {
            BandScope bs(m, nullptr, b.floor, b.lim);
            if (int rc = orc_graph_begin(nullptr)) return rc;
            if (int rc = m.forward_dev_at(d_tok_, 1, d_pos_, 0, true, d_tok_ + 1)) return abort_capture(rc);
            if (int rc = orc_decode_advance(d_tok_, d_hist_, d_pos_, d_pos_ + 1, nullptr)) return abort_capture(rc);
            if (int rc = orc_graph_end(nullptr, &c.g)) return rc;
            c.a = m.uid();
            c.b = 0;
            c.k = 1;
        }
        if (int rc = orc_graph_launch(c.g, nullptr)) return rc;
    }
    if (int rc = orc_memcpy_d2h(out, d_hist_, (size_t)n_gen * 4, nullptr)) return rc;
    return n_gen;
}

// The speculative-greedy loop (benchmark/bench_engine.cpp:310-356). A round
// at position pos drafts ndt = min(k, dctx - 1 - pos) tokens (the draft's
// context), verifies nver = min(ndt + 1, tctx - pos) inputs in one target
// pass (the target's context) and compares the first min(ndt, nver) drafts;
// it emits the accepted drafts, then the mismatch, or, when every draft was
// accepted, the verify pass held a bonus row (nver = ndt + 1) and
// pos + ndt + 1 < tctx - 1, the bonus token (and refills the draft's KV at
// pos + ndt); the loop runs while pos < tctx - 1. Rounds with ndt = k and
// nver = k + 1 replay one captured graph (k draft steps at *d_pos + i, the
// (k+1)-token verify at *d_pos, acceptance, which advances *d_pos and writes
// the next input into d_vin[0]; a second graph refills the draft); the
// shorter rounds at the end of a context run from the host at host
// positions.
int DecodeSession::spec_rounds(Model& tgt, Model& dft, int pos, int32_t next, int n_gen, int k, int32_t* out,
                               SpecStats& S) {
    const int tctx = (int)tgt.cfg.ctx_len, dctx = (int)dft.cfg.ctx_len, ctx = std::min(tctx, dctx);
    const int run_lim = graph_limit(pos + n_gen + k + 2, ctx);
    std::vector<int32_t> h(k + 3), ids(k + 2);
    bool dev_state = false;  // *d_pos / d_vin[0] hold pos / next
    int ng = 0;
    while (ng < n_gen && pos < tctx - 1) {
        const int ndt = std::min(k, dctx - 1 - pos);
        if (ndt < 1) break;
        const int nver = std::min(ndt + 1, tctx - pos);
        const int ncmp = std::min(ndt, nver);
        const bool graphed = graphs_ && ndt == k && nver == k + 1;
        Captured* c = nullptr;
        int a;
        const int32_t* em;  // the round's target argmaxes from the first emitted token on
        if (graphed) {
            // the round's passes reach positions pos .. pos + k (the refill included)
            const Band b = band_of(pos, pos + k, run_lim, ctx);
            c = &slot(spec_g_, b, tgt.uid(), dft.uid(), k);
            if (!c->g) {
                BandScope bs(tgt, &dft, b.floor, b.lim);
                if (int rc = orc_graph_begin(nullptr)) return rc;
                for (int i = 0; i < k; ++i)
                    if (int rc = dft.forward_dev_at(d_vin_ + i, 1, d_pos_, i, true, d_vin_ + i + 1))
                        return abort_capture(rc);
                if (int rc = tgt.forward_dev_at(d_vin_, k + 1, d_pos_, 0, true, d_tgt_)) return abort_capture(rc);
                if (int rc = orc_spec_accept_greedy_at(d_tgt_, d_vin_ + 1, k, d_acc_, d_pos_, d_vin_, nullptr))
                    return abort_capture(rc);
                if (int rc = orc_graph_end(nullptr, &c->g)) return rc;
                if (int rc = orc_graph_begin(nullptr)) return rc;
                if (int rc = dft.forward_dev_at(d_vin_ + k, 1, d_pos_, -1, false, nullptr)) return abort_capture(rc);
                if (int rc = orc_graph_end(nullptr, &c->fill)) return rc;
                c->a = tgt.uid();
                c->b = dft.uid();
                c->k = k;
            }
            if (!dev_state) {
                if (int rc = orc_memcpy_h2d(d_pos_, &pos, 4, nullptr)) return rc;
                if (int rc = orc_memcpy_h2d(d_vin_, &next, 4, nullptr)) return rc;
                dev_state = true;
            }
            if (int rc = orc_graph_launch(c->g, nullptr)) return rc;
            if (int rc = orc_memcpy_d2h(h.data(), d_acc_, (size_t)(k + 3) * 4, nullptr)) return rc;
            a = h[0];
            em = h.data() + 2;
        } else {
            if (int rc = orc_memcpy_h2d(d_vin_, &next, 4, nullptr)) return rc;
            dev_state = false;
            // (a) ndt greedy draft proposals; draft step i writes d_i into d_vin[i+1]
            for (int i = 0; i < ndt; ++i)
                if (int rc = dft.forward_dev(d_vin_ + i, 1, pos + i, true, d_vin_ + i + 1)) return rc;
            // (b) one nver-token verify pass of the target over [next, d0 .. d_{nver-2}]
            if (int rc = tgt.forward_dev(d_vin_, nver, pos, true, d_tgt_)) return rc;
            // (c) acceptance of the first ncmp drafts on the device; ids and count to the host
            if (int rc = orc_spec_accept_greedy(d_tgt_, d_vin_ + 1, ncmp, d_acc_, nullptr)) return rc;
            int32_t acc[2];
            if (int rc = orc_memcpy_d2h(ids.data(), d_tgt_, (size_t)nver * 4, nullptr)) return rc;
            if (int rc = orc_memcpy_d2h(acc, d_acc_, 8, nullptr)) return rc;
            a = acc[0];
            em = ids.data();
        }
        S.proposed += ndt;
        S.passes++;
        S.rounds++;
        // em[0 .. a-1] are the accepted drafts, em[a] the mismatch or (a = ndt < nver) the bonus
        bool stop = false;
        for (int i = 0; i < a && !stop; ++i) {
            out[ng++] = em[i];
            S.accepted++;
            stop = ng >= n_gen;
        }
        if (!stop) {
            if (a < ncmp) {
                out[ng++] = em[a];
                next = em[a];
            } else if (ndt < nver && pos + ndt + 1 < tctx - 1) {
                out[ng++] = em[ndt];
                next = em[ndt];
                // every proposal accepted: the draft still lacks d_{ndt-1} at pos + ndt
                if (graphed) {
                    if (int rc = orc_graph_launch(c->fill, nullptr)) return rc;
                } else if (int rc = dft.forward_dev(d_vin_ + ndt, 1, pos + ndt, false, nullptr)) {
                    return rc;
                }
            } else {
                stop = true;  // the bonus falls at the end of the context: the loop ends here
            }
        }
        pos += a + 1;
        if (stop) break;
    }
    orc_stream_sync(nullptr);
    return ng;
}

int DecodeSession::prefill(Model& m, const int32_t* prompt, int n_prompt) {
    if (init_rc_ != ORC_OK) return unusable();
    if (n_prompt < 1 || !prompt) return invalid("empty prompt");
    if (n_prompt > (int)m.cfg.ctx_len)
        return invalid("prompt of " + std::to_string(n_prompt) + " tokens does not fit the " +
                       std::to_string(m.cfg.ctx_len) + "-position context");
    if (n_prompt < 2) return 0;
    m.forward_prefill(prompt, n_prompt - 1, 0, nullptr);
    if (m.last_error()[0]) return invalid(std::string("prefill failed: ") + m.last_error());
    return 0;
}

// The argmax of step s is written straight into the input slot of step s+1,
// so the whole chain is enqueued without a host round trip.
int DecodeSession::greedy(Model& m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out) {
    if (init_rc_ != ORC_OK) return unusable();
    if (n_gen > max_tokens_ || n_prompt < 1) return invalid("greedy: bad prompt or more tokens than the session holds");
    int pos = n_prompt - 1;
    if (pos + n_gen > (int)m.cfg.ctx_len) return invalid("greedy: prompt + generated tokens exceed the context");
    int32_t first = prompt[n_prompt - 1];
    if (first < 0 || first >= (int32_t)m.cfg.n_vocab) first = 0;
    if (graphs_) return greedy_graphed(m, pos, first, n_gen, out);
    if (int rc = orc_memcpy_h2d(d_hist_, &first, 4, nullptr)) return rc;
    for (int s = 0; s < n_gen; ++s)
        if (int rc = m.forward_dev(d_hist_ + s, 1, pos + s, true, d_hist_ + s + 1)) return rc;
    if (int rc = orc_memcpy_d2h(out, d_hist_ + 1, (size_t)n_gen * 4, nullptr)) return rc;
    return n_gen;
}

int DecodeSession::spec_greedy(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                               int32_t* out, SpecStats* st) {
    if (init_rc_ != ORC_OK) return unusable();
    if (k < 1 || k > max_k_ || n_prompt < 1) return invalid("spec_greedy: bad k or prompt");
    if (dft.cfg.n_vocab != tgt.cfg.n_vocab)  // bench_engine.cpp:290-293
        return invalid("spec_greedy: draft and target vocabularies differ");
    SpecStats local;
    SpecStats& S = st ? *st : local;
    const int pos = n_prompt - 1;
    int32_t next = prompt[n_prompt - 1];
    if (next < 0 || next >= (int32_t)tgt.cfg.n_vocab) next = 0;
    return spec_rounds(tgt, dft, pos, next, n_gen, k, out, S);
}

// engine.cpp:115-125: reset both models, prefill prompt[0 .. n-2] on each
// and initialise the device sampler with those ids recorded. ids = the
// prompt with out-of-range ids clamped to 0 (model.cpp:352-356).
int DecodeSession::begin_sampled(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, const SamplerConfig& sc,
                                 std::vector<int32_t>& ids) {
    const int V = (int)tgt.cfg.n_vocab;
    if (n_prompt > (int)std::min(tgt.cfg.ctx_len, dft.cfg.ctx_len))
        return invalid("prompt of " + std::to_string(n_prompt) + " tokens does not fit the context");
    ids.assign(prompt, prompt + n_prompt);
    for (auto& t : ids)
        if (t < 0 || t >= V) t = 0;
    tgt.reset();
    dft.reset();
    if (n_prompt > 1) {
        tgt.forward_prefill(ids.data(), n_prompt - 1, 0, nullptr);
        if (tgt.last_error()[0]) return invalid(std::string("target prefill failed: ") + tgt.last_error());
        dft.forward_prefill(ids.data(), n_prompt - 1, 0, nullptr);
        if (dft.last_error()[0]) return invalid(std::string("draft prefill failed: ") + dft.last_error());
    }
    int32_t* d_ph = nullptr;
    if (n_prompt > 1) {
        if (int rc = orc_malloc((void**)&d_ph, (size_t)(n_prompt - 1) * 4)) return rc;
        if (int rc = orc_memcpy_h2d(d_ph, ids.data(), (size_t)(n_prompt - 1) * 4, nullptr)) {
            orc_free(d_ph);
            return rc;
        }
    }
    int rc = orc_sampler_init(d_samp_, sc.temperature, sc.top_p, sc.top_k, sc.repeat_penalty, sc.repeat_last, sc.seed,
                              d_ph, n_prompt - 1, nullptr);
    orc_stream_sync(nullptr);
    orc_free(d_ph);
    return rc;
}

int DecodeSession::spec_engine(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                               const SamplerConfig& sc, int32_t* out, SpecStats* st) {
    if (init_rc_ != ORC_OK) return unusable();
    if (k < 1 || k > max_k_ || n_prompt < 1 || n_gen < 1) return invalid("spec_engine: bad k, prompt or length");
    if (dft.cfg.n_vocab != tgt.cfg.n_vocab) return invalid("spec_engine: draft and target vocabularies differ");
    // engine.cpp:155-160 lets a draft of a longer context propose tokens the
    // target can no longer verify; this loop supports draft contexts up to
    // the target's
    if (dft.cfg.ctx_len > tgt.cfg.ctx_len) return invalid("spec_engine: draft context longer than the target's");
    SpecStats local;
    SpecStats& S = st ? *st : local;
    const int V = (int)tgt.cfg.n_vocab;
    const int ctx = (int)std::min(tgt.cfg.ctx_len, dft.cfg.ctx_len);
    std::vector<int32_t> ids;
    int rc = begin_sampled(tgt, dft, prompt, n_prompt, sc, ids);
    if (rc) return rc;
    int pos = n_prompt - 1;

    const int run_lim = graph_limit(pos + n_gen + k + 2, ctx);
    const int32_t next = ids[n_prompt - 1];
    if ((rc = orc_memcpy_h2d(d_pos_, &pos, 4, nullptr))) return rc;
    if ((rc = orc_memcpy_h2d(d_vin_, &next, 4, nullptr))) return rc;
    if ((rc = orc_memcpy_h2d(d_budget_, &n_gen, 4, nullptr))) return rc;
    std::vector<int32_t> h(k + 5);
    int ng = 0;
    Captured* c = nullptr;
    // engine.cpp:140-240: a round drafts ndt = min(k, ctx - 1 - pos) tokens and
    // samples the bonus (an extra target position pos + ndt) only while
    // pos + ndt < ctx - 1; the loop runs while pos < ctx - 1. Rounds with
    // ndt = k replay the captured graphs.
    const int tctx = (int)tgt.cfg.ctx_len;
    while (ng < n_gen && pos < tctx - 1) {
        const int ndt = std::min(k, ctx - 1 - pos);
        if (ndt < 1) break;
        const bool graphed = graphs_ && ndt == k;
        if (graphed) {
            const Band b = band_of(pos, pos + k, run_lim, ctx);  // positions pos .. pos + k this round
            c = &slot(eng_g_, b, tgt.uid(), dft.uid(), k);
            if (!c->g) {
                BandScope bs(tgt, &dft, b.floor, b.lim);
                if ((rc = orc_graph_begin(nullptr))) return rc;
                for (int i = 0; i < k; ++i)
                    if ((rc = dft.forward_dev_at(d_vin_ + i, 1, d_pos_, i, true, d_vin_ + i + 1)))
                        return abort_capture(rc);
                if ((rc = tgt.forward_dev_at(d_vin_, k + 1, d_pos_, 0, true, nullptr))) return abort_capture(rc);
                if ((rc = orc_spec_accept_engine(d_samp_, tgt.d_logits(), V, V, d_vin_ + 1, k, 0, d_budget_, d_eout_,
                                                 d_pos_, d_vin_, nullptr)))
                    return abort_capture(rc);
                if ((rc = orc_graph_end(nullptr, &c->g))) return rc;
                if ((rc = orc_graph_begin(nullptr))) return rc;
                if ((rc = dft.forward_dev_at(d_vin_ + k, 1, d_pos_, -1, false, nullptr))) return abort_capture(rc);
                if ((rc = orc_graph_end(nullptr, &c->fill))) return rc;
                c->a = tgt.uid();
                c->b = dft.uid();
                c->k = k;
            }
            if ((rc = orc_graph_launch(c->g, nullptr))) return rc;
        } else {
            for (int i = 0; i < ndt; ++i)
                if ((rc = dft.forward_dev_at(d_vin_ + i, 1, d_pos_, i, true, d_vin_ + i + 1))) return rc;
            if ((rc = tgt.forward_dev_at(d_vin_, ndt + 1, d_pos_, 0, true, nullptr))) return rc;
            if ((rc = orc_spec_accept_engine(d_samp_, tgt.d_logits(), V, V, d_vin_ + 1, ndt, 0, d_budget_, d_eout_,
                                             d_pos_, d_vin_, nullptr)))
                return rc;
        }
        if ((rc = orc_memcpy_d2h(h.data(), d_eout_, (size_t)(ndt + 5) * 4, nullptr))) return rc;
        int emitted = h[0], passes = h[2];
        // a bonus at the end of the context is not sampled by the reference:
        // its token and target pass are dropped and the loop ends
        const bool bonus = h[3] && emitted == ndt + 1;
        const bool at_end = bonus && pos + ndt >= tctx - 1;
        if (at_end) {
            --emitted;
            --passes;
        }
        S.accepted += h[1];
        S.proposed += ndt;
        S.passes += passes;
        S.rounds++;
        for (int i = 0; i < emitted && ng < n_gen; ++i) out[ng++] = h[4 + i];
        if (at_end) break;
        if (h[3] && ng < n_gen) {  // every proposal accepted: the draft lacks d_{ndt-1} (engine.cpp:230)
            if (graphed) {
                if ((rc = orc_graph_launch(c->fill, nullptr))) return rc;
            } else if ((rc = dft.forward_dev_at(d_vin_ + ndt, 1, d_pos_, -1, false, nullptr))) {
                return rc;
            }
        }
        pos += emitted;
    }
    orc_stream_sync(nullptr);
    return ng;
}

// One round of speculative sampling: k draft steps, each followed by the
// sampler transform of its logits (pending proposals d_vin[1 .. i] in the
// penalty window) into q_i and a draw x_i = d_vin[i+1]; one batched target
// pass over d_vin[0 .. k]; the transform of its k+1 rows into p; the
// acceptance chain, which advances *d_pos and writes the next input to d_vin[0].
int DecodeSession::sampled_round(Model& tgt, Model& dft, int k, int V) {
    for (int i = 0; i < k; ++i) {
        float* q = d_q_ + (size_t)i * V;
        if (int rc = dft.forward_dev_at(d_vin_ + i, 1, d_pos_, i, true, nullptr)) return rc;
        if (int rc = orc_transform_draw(d_samp_, dft.d_logits(), V, d_vin_ + 1, i, q, d_vin_ + i + 1, nullptr, nullptr))
            return rc;
    }
    if (int rc = tgt.forward_dev_at(d_vin_, k + 1, d_pos_, 0, true, nullptr)) return rc;
    if (int rc = orc_transform_probs(d_samp_, tgt.d_logits(), V, V, k + 1, d_vin_ + 1, 0, d_p_, V, nullptr)) return rc;
    return orc_spec_accept_stochastic(d_samp_, d_p_, V, d_q_, V, V, d_vin_ + 1, k, 0, d_budget_, d_eout_, d_pos_,
                                      d_vin_, nullptr);
}

int DecodeSession::spec_sampled(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                                const SamplerConfig& sc, int32_t* out, SpecStats* st) {
    if (init_rc_ != ORC_OK) return unusable();
    if (k < 1 || k > max_k_ || n_prompt < 1 || n_gen < 1) return invalid("spec_sampled: bad k, prompt or length");
    if (dft.cfg.n_vocab != tgt.cfg.n_vocab) return invalid("spec_sampled: draft and target vocabularies differ");
    SpecStats local;
    SpecStats& S = st ? *st : local;
    const int V = (int)tgt.cfg.n_vocab;
    const int ctx = (int)std::min(tgt.cfg.ctx_len, dft.cfg.ctx_len);
    const size_t need = (size_t)(max_k_ + 1) * V;
    if (need > pq_cap_) {  // p: k+1 rows, q: k rows of the vocabulary
        orc_free(d_p_);
        orc_free(d_q_);
        d_p_ = d_q_ = nullptr;
        pq_cap_ = 0;
        for (Captured& c : smp_g_) drop(c);
        if (int rc = orc_malloc((void**)&d_p_, need * 4)) return rc;
        if (int rc = orc_malloc((void**)&d_q_, need * 4)) return rc;
        pq_cap_ = need;
    }
    std::vector<int32_t> ids;
    int rc = begin_sampled(tgt, dft, prompt, n_prompt, sc, ids);
    if (rc) return rc;
    int pos = n_prompt - 1;

    const int run_lim = graph_limit(pos + n_gen + k + 2, ctx);
    const int32_t next = ids[n_prompt - 1];
    if ((rc = orc_memcpy_h2d(d_pos_, &pos, 4, nullptr))) return rc;
    if ((rc = orc_memcpy_h2d(d_vin_, &next, 4, nullptr))) return rc;
    if ((rc = orc_memcpy_h2d(d_budget_, &n_gen, 4, nullptr))) return rc;
    std::vector<int32_t> h(k + 5);
    int ng = 0;
    Captured* c = nullptr;
    while (ng < n_gen && pos + k + 1 <= ctx) {
        if (graphs_) {
            const Band b = band_of(pos, pos + k, run_lim, ctx);  // positions pos .. pos + k this round
            c = &slot(smp_g_, b, tgt.uid(), dft.uid(), k);
            if (!c->g) {
                BandScope bs(tgt, &dft, b.floor, b.lim);
                if ((rc = orc_graph_begin(nullptr))) return rc;
                if ((rc = sampled_round(tgt, dft, k, V))) return abort_capture(rc);
                if ((rc = orc_graph_end(nullptr, &c->g))) return rc;
                if ((rc = orc_graph_begin(nullptr))) return rc;
                if ((rc = dft.forward_dev_at(d_vin_ + k, 1, d_pos_, -1, false, nullptr))) return abort_capture(rc);
                if ((rc = orc_graph_end(nullptr, &c->fill))) return rc;
                c->a = tgt.uid();
                c->b = dft.uid();
                c->k = k;
            }
            rc = orc_graph_launch(c->g, nullptr);
        } else {
            rc = sampled_round(tgt, dft, k, V);
        }
        if (rc) return rc;
        if ((rc = orc_memcpy_d2h(h.data(), d_eout_, (size_t)(k + 5) * 4, nullptr))) return rc;
        const int emitted = h[0];
        S.accepted += h[1];
        S.proposed += k;
        S.passes += 1;
        S.rounds++;
        for (int i = 0; i < emitted && ng < n_gen; ++i) out[ng++] = h[4 + i];
        if (h[3] && ng < n_gen) {  // every proposal accepted: the draft lacks x_{k-1}
            if (graphs_) {
                if ((rc = orc_graph_launch(c->fill, nullptr))) return rc;
            } else if ((rc = dft.forward_dev_at(d_vin_ + k, 1, d_pos_, -1, false, nullptr))) {
                return rc;
            }
        }
        pos += emitted;
    }
    orc_stream_sync(nullptr);
    return ng;
}

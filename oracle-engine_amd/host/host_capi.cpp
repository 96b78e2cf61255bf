// C API of the host library (include/oracle_host.h).
#include "oracle_host.h"

#include "model.hpp"
#include "spec.hpp"

#include <cstring>
#include <memory>
#include <string>

struct orch_model {
    Model m;
    std::string err;
};

namespace {
thread_local std::string g_load_err;
DecodeSession& session() {
    static DecodeSession s;  // device scratch for the decode loops, created on first use
    return s;
}
int fail(orch_model* h, int rc) {
    h->err = h->m.last_error()[0] ? h->m.last_error() : orc_last_error();
    return rc ? rc : -1;
}
}  // namespace

extern "C" orch_model* orch_load(const char* path, int ctx_len) {
    auto h = std::make_unique<orch_model>();
    if (!h->m.load(path, ctx_len)) {
        g_load_err = h->m.last_error();
        return nullptr;
    }
    return h.release();
}

extern "C" void orch_free(orch_model* m) { delete m; }

extern "C" const char* orch_error(const orch_model* m) { return m ? m->err.c_str() : g_load_err.c_str(); }

extern "C" int orch_cfg(const orch_model* h, int32_t* c, float* rope) {
    const ModelConfig& g = h->m.cfg;
    c[0] = (int32_t)g.n_vocab; c[1] = (int32_t)g.n_layers; c[2] = (int32_t)g.n_heads; c[3] = (int32_t)g.n_kv_heads;
    c[4] = (int32_t)g.embed_dim; c[5] = (int32_t)g.ffn_hidden; c[6] = (int32_t)g.head_dim; c[7] = (int32_t)g.ctx_len;
    c[8] = h->m.gguf().has_tensor("blk.0.attn_q.bias") ? 1 : 0;
    c[9] = h->m.gguf().has_tensor("output.weight") ? 0 : 1;
    if (rope) *rope = g.rope_freq;
    return 0;
}

extern "C" int orch_reset(orch_model* h) {
    h->m.reset();
    return 0;
}

extern "C" int orch_forward(orch_model* h, int32_t tok, int pos, float* logits) {
    const float* l = h->m.forward(tok, pos, logits != nullptr);
    if (logits) {
        if (!l) return fail(h, -1);
        std::memcpy(logits, l, (size_t)h->m.cfg.n_vocab * 4);
    }
    return 0;
}

extern "C" int orch_forward_batch(orch_model* h, const int32_t* toks, int n, int sp, float* logits) {
    if (n <= 0 || sp < 0 || sp + n > (int)h->m.cfg.ctx_len) {
        h->err = "positions exceed the context length";
        return -1;
    }
    h->m.forward_prefill(toks, n, sp, logits);
    if (h->m.last_error()[0]) return fail(h, -1);
    return 0;
}

extern "C" int orch_greedy(orch_model* h, const int32_t* prompt, int np, int n_gen, int32_t* out, int prefill) {
    if (prefill) {
        h->m.reset();
        session().prefill(h->m, prompt, np);
    }
    int rc = session().greedy(h->m, prompt, np, n_gen, out);
    return rc < 0 ? fail(h, rc) : rc;
}

extern "C" int orch_spec_greedy(orch_model* t, orch_model* d, const int32_t* prompt, int np, int n_gen, int k,
                                int32_t* out, int64_t* stats, int prefill) {
    if (prefill) {
        t->m.reset();
        d->m.reset();
        session().prefill(t->m, prompt, np);
        session().prefill(d->m, prompt, np);
    }
    SpecStats st;
    int rc = session().spec_greedy(t->m, d->m, prompt, np, n_gen, k, out, &st);
    if (stats) {
        stats[0] = st.accepted;
        stats[1] = st.proposed;
        stats[2] = st.passes;
        stats[3] = st.rounds;
    }
    return rc < 0 ? fail(t, rc) : rc;
}

extern "C" double orch_weight_bytes(const orch_model* h, int logits) { return h->m.weight_bytes(logits != 0); }

extern "C" int orch_sync(void) { return orc_device_sync(); }

extern "C" int orch_set_graphs(int on) {
    const int prev = session().graphs() ? 1 : 0;
    session().set_graphs(on != 0);
    return prev;
}


static SamplerConfig sampler_config(const float* sampler, const int32_t* isampler, uint64_t seed) {
    SamplerConfig sc;
    sc.temperature = sampler[0];
    sc.top_p = sampler[1];
    sc.repeat_penalty = sampler[2];
    sc.top_k = isampler[0];
    sc.repeat_last = isampler[1];
    sc.seed = seed;
    return sc;
}

extern "C" int orch_spec_engine(orch_model* t, orch_model* d, const int32_t* prompt, int np, int n_gen, int k,
                                const float* sampler, const int32_t* isampler, uint64_t seed, int32_t* out,
                                int64_t* stats) {
    if (!t || !d || !prompt || !out || !sampler || !isampler) return -1;
    SpecStats st;
    const int rc = session().spec_engine(t->m, d->m, prompt, np, n_gen, k, sampler_config(sampler, isampler, seed),
                                         out, &st);
    if (rc < 0) return fail(t, rc);
    if (stats) {
        stats[0] = st.accepted;
        stats[1] = st.proposed;
        stats[2] = st.passes;
    }
    return rc;
}

extern "C" int orch_spec_sampled(orch_model* t, orch_model* d, const int32_t* prompt, int np, int n_gen, int k,
                                 const float* sampler, const int32_t* isampler, uint64_t seed, int32_t* out,
                                 int64_t* stats) {
    if (!t || !d || !prompt || !out || !sampler || !isampler) return -1;
    SpecStats st;
    const int rc = session().spec_sampled(t->m, d->m, prompt, np, n_gen, k, sampler_config(sampler, isampler, seed),
                                          out, &st);
    if (rc < 0) return fail(t, rc);
    if (stats) {
        stats[0] = st.accepted;
        stats[1] = st.proposed;
        stats[2] = st.passes;
    }
    return rc;
}

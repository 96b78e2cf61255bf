// C API of the host library (include/oracle_host.h).
#include "oracle_host.h"

#include "engine.hpp"
#include "model.hpp"
#include "ops.hpp"
#include "sampler.hpp"
#include "spec.hpp"

#include <algorithm>
#include <cstring>
#include <memory>
#include <string>

struct orch_model {
    Model m;
    std::string err;
};

namespace {
thread_local std::string g_load_err;
// Device scratch and captured graphs of the decode loops: one session per
// calling thread (created on its first decode call, released when the thread
// ends), so threads that decode different models never share them. One
// model must still not be used by two threads at once (its activations and
// KV cache are single-stream state, as the reference's Model is).
DecodeSession& session() {
    thread_local DecodeSession s;
    return s;
}
int fail(orch_model* h, int rc) {
    h->err = session().error()[0] ? session().error() : h->m.last_error()[0] ? h->m.last_error() : orc_last_error();
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
    if (!h || !prompt || !out) return -1;
    session().clear_error();
    if (prefill) {
        h->m.reset();
        if (int rc = session().prefill(h->m, prompt, np)) return fail(h, rc);
    }
    int rc = session().greedy(h->m, prompt, np, n_gen, out);
    return rc < 0 ? fail(h, rc) : rc;
}

extern "C" int orch_spec_greedy(orch_model* t, orch_model* d, const int32_t* prompt, int np, int n_gen, int k,
                                int32_t* out, int64_t* stats, int prefill) {
    if (!t || !d || !prompt || !out) return -1;
    session().clear_error();
    if (prefill) {
        t->m.reset();
        d->m.reset();
        if (int rc = session().prefill(t->m, prompt, np)) return fail(t, rc);
        if (int rc = session().prefill(d->m, prompt, np)) return fail(t, rc);
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
    session().clear_error();
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
    session().clear_error();
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

// ── GGUFParser drop-ins of a loaded model (tests of the parser API) ─────────
extern "C" int orch_gguf_device_type(const orch_model* h, const char* tensor) {
    return h && tensor ? h->m.gguf().device_type(tensor) : -1;
}

extern "C" int orch_gguf_gemm(orch_model* h, const char* tensor, const float* x, int n_tok, int j0, int j1,
                              float* out) {
    if (!h || !tensor || !x || !out || n_tok < 1) return -1;
    const GGUFParser& g = h->m.gguf();
    if (!g.has_tensor(tensor) || g.tensor_info(tensor).shape.size() != 2) {
        h->err = std::string("no 2-D tensor ") + tensor;
        return -1;
    }
    const int n_in = (int)g.tensor_info(tensor).shape[0];
    const bool ok = n_tok == 1 ? g.gemv_q_range(tensor, out, x, j0, j1, n_in)
                  : j0 == 0 ? g.gemm_q(tensor, out, x, n_tok, j1, n_in) : false;
    if (!ok) {
        h->err = std::string("gemv_q / gemm_q failed on ") + tensor + ": " + orc_last_error();
        return -1;
    }
    return 0;
}

extern "C" int orch_gguf_dequant_row(orch_model* h, const char* tensor, int64_t row, float* out) {
    if (!h || !tensor || !out || !h->m.gguf().has_tensor(tensor)) return -1;
    h->m.gguf().dequantize_row(tensor, row, out);
    return 0;
}

// ── the rest of the Model surface ───────────────────────────────────────────
extern "C" int orch_embed_tokens(orch_model* h, const int32_t* tokens, int n, float* out) {
    if (!h || !tokens || !out || n <= 0) return -1;
    const std::vector<float> e = h->m.embed_tokens(std::vector<int32_t>(tokens, tokens + n));
    if (e.empty()) return fail(h, -1);
    std::memcpy(out, e.data(), e.size() * 4);
    return 0;
}

extern "C" int orch_save_state(orch_model* h, const char* path, int pos) {
    return h && path && h->m.save_state(path, pos) ? 0 : -1;
}

extern "C" int orch_load_state(orch_model* h, const char* path, int* pos) {
    if (!h || !path || !pos) return -1;
    return h->m.load_state(path, *pos) ? 0 : -1;
}

struct orch_kv_snapshot {
    Model::KVSnapshot s;
};

extern "C" orch_kv_snapshot* orch_snapshot_kv(orch_model* h, int pos) {
    if (!h) return nullptr;
    auto s = std::make_unique<orch_kv_snapshot>();
    s->s = h->m.snapshot_kv(pos);
    return s->s.bytes ? s.release() : nullptr;
}

extern "C" int orch_restore_kv(orch_model* h, const orch_kv_snapshot* s) {
    if (!h || !s) return -1;
    h->m.restore_kv(s->s);
    return h->m.last_error()[0] ? fail(h, -1) : 0;
}

extern "C" int orch_snapshot_pos(const orch_kv_snapshot* s) { return s ? s->s.pos : -1; }
extern "C" void orch_snapshot_free(orch_kv_snapshot* s) { delete s; }
extern "C" int orch_norm_cache_matches(orch_model* h) { return h && h->m.test_norm_cache_matches() ? 1 : 0; }

// ── namespace ops ────────────────────────────────────────────────────────────
extern "C" void orch_ops_rmsnorm(float* out, const float* x, const float* w, int n, float eps) {
    ops::rmsnorm(out, x, w, n, eps);
}
extern "C" void orch_ops_matmul(float* out, const float* a, const float* b, int m, int n, int k) {
    ops::matmul(out, a, b, m, n, k);
}
extern "C" void orch_ops_matmul_nn(float* out, const float* a, const float* b, int m, int n, int k) {
    ops::matmul_nn(out, a, b, m, n, k);
}
extern "C" void orch_ops_silu(float* x, int n) { ops::silu(x, n); }
extern "C" void orch_ops_mul(float* out, const float* a, const float* b, int n) { ops::mul(out, a, b, n); }
extern "C" void orch_ops_add(float* a, const float* b, int n) { ops::add(a, b, n); }
extern "C" void orch_ops_copy(float* dst, const float* src, int n) { ops::copy(dst, src, n); }
extern "C" void orch_ops_softmax(float* x, int n) { ops::softmax(x, n); }
extern "C" void orch_ops_rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int pos,
                              float freq_base) {
    ops::rope(q, k, n_heads, n_kv_heads, head_dim, pos, freq_base);
}
extern "C" int orch_ops_argmax(const float* x, int n) { return ops::argmax(x, n); }
extern "C" float orch_ops_dot(const float* a, const float* b, int n) { return ops::dot(a, b, n); }

// ── Sampler ──────────────────────────────────────────────────────────────────
struct orch_sampler {
    Sampler s;
    explicit orch_sampler(const SamplerParams& p, uint64_t seed) : s(p, seed) {}
};

static SamplerParams sparams(float temperature, float top_p, int top_k, float repeat_pen, int repeat_last) {
    SamplerParams p;
    p.temperature = temperature;
    p.top_p = top_p;
    p.top_k = top_k;
    p.repeat_pen = repeat_pen;
    p.repeat_last = repeat_last;
    return p;
}

extern "C" orch_sampler* orch_sampler_new(float temperature, float top_p, int top_k, float repeat_pen,
                                          int repeat_last, uint64_t seed) {
    auto h = std::make_unique<orch_sampler>(sparams(temperature, top_p, top_k, repeat_pen, repeat_last), seed);
    return h->s.device_state() && h->s.error().empty() ? h.release() : nullptr;
}
extern "C" void orch_sampler_free(orch_sampler* s) { delete s; }
extern "C" int32_t orch_sampler_sample(orch_sampler* s, float* logits, int n_vocab) {
    return s ? s->s.sample(logits, n_vocab) : -1;
}
extern "C" void orch_sampler_record(orch_sampler* s, int32_t id) {
    if (s) s->s.record(id);
}
extern "C" void orch_sampler_reset(orch_sampler* s) {
    if (s) s->s.reset();
}
extern "C" void orch_sampler_set_params(orch_sampler* s, float temperature, float top_p, int top_k,
                                        float repeat_pen, int repeat_last) {
    if (s) s->s.set_params(sparams(temperature, top_p, top_k, repeat_pen, repeat_last));
}

// ── Engine and Tokenizer ─────────────────────────────────────────────────────
struct orch_engine {
    Engine e;
    std::string err;
};

extern "C" orch_engine* orch_engine_new(const char* model_path, const char* draft_path) {
    auto h = std::make_unique<orch_engine>();
    if (!model_path || !h->e.load(model_path) || (draft_path && !h->e.load_draft(draft_path))) {
        g_load_err = h->e.last_error();
        return nullptr;
    }
    return h.release();
}
extern "C" void orch_engine_free(orch_engine* e) { delete e; }
extern "C" const char* orch_engine_error(const orch_engine* e) {
    return e ? e->e.last_error().c_str() : g_load_err.c_str();
}
extern "C" void orch_engine_set_seed(orch_engine* e, uint64_t seed) {
    if (e) e->e.set_seed(seed);
}

extern "C" int64_t orch_engine_generate(orch_engine* h, const char* const* roles, const char* const* contents,
                                        int n_msgs, int n_predict, float temperature, float top_p,
                                        float repeat_penalty, int repeat_last_n, uint8_t* out, int64_t cap) {
    if (!h || n_msgs < 0 || (n_msgs && (!roles || !contents)) || !out || cap < 0) return -1;
    std::vector<Message> msgs;
    for (int i = 0; i < n_msgs; ++i) msgs.push_back({roles[i], contents[i]});
    GenParams gp;
    gp.n_predict = n_predict;
    gp.temperature = temperature;
    gp.top_p = top_p;
    gp.repeat_penalty = repeat_penalty;
    gp.repeat_last_n = repeat_last_n;
    int64_t w = 0;
    bool fit = true;
    const std::string resp = h->e.generate(msgs, gp, [&](const std::string& p) {
        const uint32_t n = (uint32_t)p.size();
        if (w + 4 + (int64_t)n > cap) {
            fit = false;
            return;
        }
        std::memcpy(out + w, &n, 4);
        std::memcpy(out + w + 4, p.data(), n);
        w += 4 + n;
    });
    if (!fit) return -1;
    // a refused prompt is an empty reply, as the reference's; a device failure is an error
    if (!h->e.last_error().empty() && h->e.last_error() != "prompt too long for the context") return -1;
    return w;
}

extern "C" int orch_engine_embed(orch_engine* h, const char* text, float* out) {
    if (!h || !text || !out) return -1;
    const std::vector<float> v = h->e.embed(text);
    if (v.empty()) return -1;
    std::memcpy(out, v.data(), v.size() * 4);
    return 0;
}

struct orch_tokenizer {
    GGUFParser g;
    Tokenizer t;
};

extern "C" orch_tokenizer* orch_tokenizer_load(const char* path) {
    auto h = std::make_unique<orch_tokenizer>();
    if (!path || !h->g.load_meta(path) || !h->t.load(h->g)) return nullptr;
    return h.release();
}
extern "C" void orch_tokenizer_free(orch_tokenizer* t) { delete t; }

extern "C" int orch_tok_encode(orch_tokenizer* h, const char* text, int64_t len, int add_bos, int32_t* out, int cap) {
    if (!h || (len && !text) || len < 0 || !out) return -1;
    const auto ids = h->t.encode(std::string(text, (size_t)len), add_bos != 0);
    if ((int64_t)ids.size() > cap) return -1;
    std::memcpy(out, ids.data(), ids.size() * 4);
    return (int)ids.size();
}

extern "C" int orch_tok_decode_one(orch_tokenizer* h, int32_t id, char* out, int cap) {
    if (!h || !out) return -1;
    const std::string p = h->t.decode_one(id);
    std::memcpy(out, p.data(), std::min<size_t>(p.size(), (size_t)std::max(cap, 0)));
    return (int)p.size();
}

extern "C" int32_t orch_tok_special_id(orch_tokenizer* h, const char* name) {
    return h && name ? h->t.special_id(name) : -1;
}
extern "C" int32_t orch_tok_bos_eos(orch_tokenizer* h, int which) {
    return h ? (which ? h->t.eos_id() : h->t.bos_id()) : -1;
}

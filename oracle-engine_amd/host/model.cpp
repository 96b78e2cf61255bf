#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

Model::~Model() { free_dev(); }

bool Model::fail(const std::string& m) {
    err_ = m;
    std::fprintf(stderr, "[Model] %s\n", m.c_str());
    return false;
}

void Model::free_dev() {
    for (void* p : {(void*)d_x_, (void*)d_qkv_, (void*)d_attn_, (void*)d_h_, (void*)d_logits_, (void*)d_k_,
                    (void*)d_v_, (void*)d_rope_, (void*)d_ids_, (void*)d_am_, d_attn_ws_, d_am_ws_})
        if (p) orc_free(p);
    d_x_ = d_qkv_ = d_attn_ = d_h_ = d_logits_ = d_k_ = d_v_ = d_rope_ = nullptr;
    d_ids_ = d_am_ = nullptr;
    d_attn_ws_ = d_am_ws_ = nullptr;
}

// Config derivation and tensor binding: core/model.cpp:17-154.
bool Model::load(const std::string& path, int ctx_len) {
    free_dev();
    loaded_ = false;
    if (orc_init(0) != 0) return fail(std::string("orc_init: ") + orc_last_error());
    if (!gguf_.load(path)) return fail("cannot load " + path);
    const std::string arch = gguf_.meta_str("general.architecture", "llama");
    auto key = [&](const char* k) { return arch + "." + k; };
    if (gguf_.meta_u32(key("expert_count"), 0) > 0) return fail("MoE architecture not supported (" + arch + ")");
    if (gguf_.has_meta(key("ssm.state_size")) || gguf_.has_meta(key("ssm.conv_kernel")))
        return fail("SSM architecture not supported (" + arch + ")");
    if (arch.find("vl") != std::string::npos || arch.find("clip") != std::string::npos)
        return fail("vision-language architecture not supported (" + arch + ")");
    cfg = ModelConfig{};
    cfg.n_vocab = gguf_.meta_u32("llama.vocab_size", gguf_.meta_u32(key("vocab_size"), 32000));
    cfg.n_layers = gguf_.meta_u32(key("block_count"), 32);
    cfg.n_heads = gguf_.meta_u32(key("attention.head_count"), 32);
    cfg.n_kv_heads = gguf_.meta_u32(key("attention.head_count_kv"), cfg.n_heads);
    cfg.embed_dim = gguf_.meta_u32(key("embedding_length"), 4096);
    cfg.ffn_hidden = gguf_.meta_u32(key("feed_forward_length"), 11008);
    cfg.rope_freq = gguf_.meta_f32(key("rope.freq_base"), 500000.f);
    cfg.head_dim = gguf_.meta_u32(key("attention.key_length"), cfg.embed_dim / cfg.n_heads);
    cfg.rms_eps = gguf_.meta_f32(key("attention.layer_norm_rms_epsilon"), 1e-5f);
    cfg.qk_norm = gguf_.has_tensor("blk.0.attn_q_norm.weight");
    cfg.ctx_len = ctx_len > 0 ? (uint32_t)ctx_len : 512u;
    const char* vsrc = gguf_.has_tensor("output.weight") ? "output.weight"
                     : gguf_.has_tensor("token_embd.weight") ? "token_embd.weight" : nullptr;
    if (vsrc) {
        const auto& sh = gguf_.tensor_info(vsrc).shape;
        uint64_t a = sh.size() > 0 ? sh[0] : 0, b = sh.size() > 1 ? sh[1] : 0;
        cfg.n_vocab = (uint32_t)std::max(a, b);
    }
    if (cfg.n_kv_heads == 0 || cfg.n_heads % cfg.n_kv_heads) return fail("bad head counts");
    if (cfg.head_dim != 64 && cfg.head_dim != 128) return fail("head_dim must be 64 or 128");

    auto mat = [&](const std::string& name, Mat& m, int n_in, int n_out) -> bool {
        if (!gguf_.has_tensor(name)) return fail("missing tensor " + name);
        const TensorInfo& ti = gguf_.tensor_info(name);
        m.type = (int)ti.type;
        m.d = gguf_.tensor_device(name);
        m.n_in = (int)ti.shape[0];
        m.n_out = ti.shape.size() > 1 ? (int)ti.shape[1] : 1;
        if (m.n_in != n_in || m.n_out != n_out)
            return fail("tensor " + name + " has an unexpected shape");
        // quantized blocks, or dense F32 / F16 / BF16 rows (the reference's
        // dequantize + ops::matmul fallback, core/model.cpp:370-381)
        if (m.type != ORC_Q4_0 && m.type != ORC_Q8_0 && m.type != ORC_Q4_K && m.type != ORC_Q6_K &&
            m.type != ORC_F32 && m.type != ORC_F16 && m.type != ORC_BF16)
            return fail("tensor " + name + ": weight type " + ggml_type_name(ti.type) +
                        " is not supported by the device GEMM");
        if ((m.type == ORC_F32 || m.type == ORC_F16 || m.type == ORC_BF16) && m.n_in % 32)
            return fail("tensor " + name + ": dense rows must hold a multiple of 32 values");
        return true;
    };
    // Norm weights and biases: n floats read from the tensor's first byte
    // whatever type it declares, as the reference's load_norm_n memcpy's
    // 4 n raw bytes (core/model.cpp:317-320); the read must stay inside the
    // data section.
    auto vec = [&](const std::string& name, int n, bool required) -> const float* {
        if (!gguf_.has_tensor(name)) {
            if (required) fail("missing tensor " + name);
            return nullptr;
        }
        const TensorInfo& ti = gguf_.tensor_info(name);
        if (ti.offset + 4 * (uint64_t)n > gguf_.data_bytes() || (ti.offset & 3)) {
            fail("tensor " + name + ": " + std::to_string(n) + " floats from its offset leave the data section");
            return nullptr;
        }
        return (const float*)gguf_.tensor_device(name);
    };
    const int D = cfg.embed_dim, NQ = cfg.n_q_total(), NKV = cfg.n_kv_total(), FF = cfg.ffn_hidden, V = cfg.n_vocab;
    if (!mat("token_embd.weight", embd_, D, V)) return false;
    if (!mat(gguf_.has_tensor("output.weight") ? "output.weight" : "token_embd.weight", head_, D, V)) return false;
    if (!(out_norm_ = vec("output_norm.weight", D, true))) return false;
    layers_.assign(cfg.n_layers, Layer{});
    const bool bias = gguf_.has_tensor("blk.0.attn_q.bias");
    for (uint32_t l = 0; l < cfg.n_layers; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        Layer& L = layers_[l];
        if (!mat(b + "attn_q.weight", L.q, D, NQ) || !mat(b + "attn_k.weight", L.k, D, NKV) ||
            !mat(b + "attn_v.weight", L.v, D, NKV) || !mat(b + "attn_output.weight", L.o, NQ, D) ||
            !mat(b + "ffn_gate.weight", L.gate, D, FF) || !mat(b + "ffn_up.weight", L.up, D, FF) ||
            !mat(b + "ffn_down.weight", L.down, FF, D))
            return false;
        if (L.gate.type != L.up.type) return fail("ffn_gate and ffn_up must share a type");
        if (!(L.attn_norm = vec(b + "attn_norm.weight", D, true)) || !(L.ffn_norm = vec(b + "ffn_norm.weight", D, true)))
            return false;
        if (bias) {
            if (!(L.bq = vec(b + "attn_q.bias", NQ, true)) || !(L.bk = vec(b + "attn_k.bias", NKV, true)) ||
                !(L.bv = vec(b + "attn_v.bias", NKV, true)))
                return false;
        }
        // QK-norm weights, head_dim raw floats each (core/model.cpp:129-137)
        if (cfg.qk_norm && (!(L.q_norm = vec(b + "attn_q_norm.weight", (int)cfg.head_dim, true)) ||
                            !(L.k_norm = vec(b + "attn_k_norm.weight", (int)cfg.head_dim, true))))
            return false;
    }

    // Q8_0 matrices whose rows hold a multiple of 256 values are regrouped
    // once into the aligned ORC_Q8_0_X8 layout (same bytes, same results);
    // the token embedding keeps the GGUF layout for the row gather. The
    // parser records the new layout, so its own drop-ins read it correctly.
    {
        std::vector<std::pair<Mat*, std::string>> ms{{&head_, "output.weight"}};
        for (uint32_t l = 0; l < cfg.n_layers; ++l) {
            Layer& L = layers_[l];
            const std::string b = "blk." + std::to_string(l) + ".";
            for (auto mn : {std::make_pair(&L.q, "attn_q"), std::make_pair(&L.k, "attn_k"),
                            std::make_pair(&L.v, "attn_v"), std::make_pair(&L.o, "attn_output"),
                            std::make_pair(&L.gate, "ffn_gate"), std::make_pair(&L.up, "ffn_up"),
                            std::make_pair(&L.down, "ffn_down")})
                ms.push_back({mn.first, b + mn.second + ".weight"});
        }
        for (auto& mn : ms) {
            Mat* m = mn.first;
            if (m->type != ORC_Q8_0 || m->n_in % 256 || m->d == embd_.d || ((uintptr_t)m->d & 15)) continue;
            if (!gguf_.regroup_q8_0(mn.second))
                return fail("q8_0 regroup of " + mn.second + ": " + orc_last_error());
            m->type = ORC_Q8_0_X8;
        }
        orc_stream_sync(nullptr);
    }

    // device buffers
    const int B = kMaxBatch, BP = kPrefillBatch, C = (int)cfg.ctx_len, QKV = NQ + 2 * NKV;
    auto alloc = [&](void** p, size_t n) { return orc_malloc(p, n) == 0; };
    const size_t kv = (size_t)cfg.n_layers * NKV * C * sizeof(float);
    if (!alloc((void**)&d_x_, (size_t)BP * D * 4) || !alloc((void**)&d_qkv_, (size_t)BP * QKV * 4) ||
        !alloc((void**)&d_attn_, (size_t)BP * NQ * 4) || !alloc((void**)&d_h_, (size_t)BP * FF * 4) ||
        !alloc((void**)&d_logits_, (size_t)B * V * 4) || !alloc((void**)&d_k_, kv) || !alloc((void**)&d_v_, kv) ||
        !alloc((void**)&d_rope_, (size_t)C * cfg.head_dim * 4) || !alloc((void**)&d_ids_, (size_t)BP * 4) ||
        !alloc((void**)&d_am_, (size_t)B * 4) ||
        !alloc(&d_attn_ws_, std::max(orc_attn_workspace(B, cfg.n_heads, cfg.head_dim, C),
                                     orc_attn_fused_workspace(cfg.n_heads, cfg.n_kv_heads, cfg.head_dim))) ||
        !alloc(&d_am_ws_, orc_argmax_workspace(B, V)))
        return fail(std::string("device allocation failed: ") + orc_last_error());
    // RoPE table with the reference's float arithmetic (ops.cpp:461-466):
    // theta = pos / powf(base, 2i/hd), then cosf/sinf.
    {
        const int half = cfg.head_dim / 2;
        std::vector<float> tab((size_t)C * half * 2);
        std::vector<float> den(half);
        for (int i = 0; i < half; ++i) den[i] = std::pow(cfg.rope_freq, (float)(2 * i) / (float)cfg.head_dim);
        for (int p = 0; p < C; ++p)
            for (int i = 0; i < half; ++i) {
                const float th = (float)p / den[i];
                tab[((size_t)p * half + i) * 2 + 0] = std::cos(th);
                tab[((size_t)p * half + i) * 2 + 1] = std::sin(th);
            }
        if (orc_memcpy_h2d(d_rope_, tab.data(), tab.size() * 4, nullptr)) return fail(orc_last_error());
    }
    logits_.assign((size_t)V, 0.f);
    loaded_ = true;
    reset();
    fused_attn_ = cfg.n_heads % cfg.n_kv_heads == 0 && cfg.n_heads / cfg.n_kv_heads <= 8 &&
                  (cfg.head_dim == 64 || cfg.head_dim == 128);
    static uint64_t next_uid = 0;
    uid_ = ++next_uid;
    return true;
}

void Model::reset() {
    if (!d_k_) return;
    const size_t kv = (size_t)cfg.n_layers * cfg.n_kv_total() * cfg.ctx_len * sizeof(float);
    orc_fill(d_k_, 0, kv, nullptr);
    orc_fill(d_v_, 0, kv, nullptr);
    orc_stream_sync(nullptr);
}

void Model::warmup() {  // core/model.cpp:238-245
    for (int i = 0; i < 2; ++i) {
        forward(0, 0, true);
        reset();
    }
}

int Model::gemm_segs(const std::vector<std::pair<const Mat*, std::pair<float*, const float*>>>& segs, int n,
                     const float* x, int ldx, int ldy, const float* norm, int epi, orc_stream_t s) {
    // Q4_K and Q6_K matrices of whole 16-row tiles: one mixed launch
    bool mixed = segs.size() > 1 && segs.size() <= 3 && (epi == ORC_EPI_STORE || epi == ORC_EPI_ACCUM);
    bool types_differ = false;
    for (const auto& sg : segs) {
        const Mat& m = *sg.first;
        mixed = mixed && (m.type == ORC_Q4_K || m.type == ORC_Q6_K) && m.n_out % 16 == 0 && m.n_out < 65536;
        types_differ = types_differ || m.type != segs[0].first->type;
    }
    if (mixed && types_differ) {
        orc_seg sg[3];
        int ty[3];
        for (size_t k = 0; k < segs.size(); ++k) {
            sg[k].d_w = segs[k].first->d;
            sg[k].n_out = segs[k].first->n_out;
            sg[k].d_y = segs[k].second.first;
            sg[k].d_bias = segs[k].second.second;
            ty[k] = segs[k].first->type;
        }
        return orc_gemm_fused_mixed(ty, sg, (int)segs.size(), n, segs[0].first->n_in, x, ldx, ldy, norm,
                                    norm ? 1e-5f : 0.f, epi, s);
    }
    // one fused launch per run of consecutive same-type matrices
    size_t i = 0;
    while (i < segs.size()) {
        size_t j = i;
        orc_seg sg[3];
        int k = 0;
        while (j < segs.size() && k < 3 && segs[j].first->type == segs[i].first->type) {
            sg[k].d_w = segs[j].first->d;
            sg[k].n_out = segs[j].first->n_out;
            sg[k].d_y = segs[j].second.first;
            sg[k].d_bias = segs[j].second.second;
            ++k;
            ++j;
        }
        if (int rc = orc_gemm_fused(segs[i].first->type, sg, k, n, segs[i].first->n_in, x, ldx, ldy, norm,
                                    norm ? 1e-5f : 0.f, epi, s))
            return rc;
        i = j;
    }
    return 0;
}

int Model::chunk_dev(const int32_t* d_ids, int n, const int32_t* d_pos, int sp, bool logits, int32_t* d_argmax,
                     orc_stream_t s) {
    const int D = cfg.embed_dim, NQ = cfg.n_q_total(), NKV = cfg.n_kv_total(), FF = cfg.ffn_hidden;
    const int QKV = NQ + 2 * NKV, C = cfg.ctx_len, V = cfg.n_vocab;
    int rc;
#define CK(e) if ((rc = (e)) != 0) return rc
    CK(orc_embed(embd_.type, embd_.d, D, V, d_ids, n, d_x_, D, s));
    for (uint32_t l = 0; l < cfg.n_layers; ++l) {
        const Layer& L = layers_[l];
        float* kc = d_k_ + (size_t)l * NKV * C;
        float* vc = d_v_ + (size_t)l * NKV * C;
        // pre-norm + Q|K|V (+bias) -> qkv rows [q | k | v]   (model.cpp:366-388)
        CK(gemm_segs({{&L.q, {d_qkv_, L.bq}}, {&L.k, {d_qkv_ + NQ, L.bk}}, {&L.v, {d_qkv_ + NQ + NKV, L.bv}}}, n,
                     d_x_, D, QKV, L.attn_norm, ORC_EPI_STORE, s));
        // QK-norm (Qwen3): per-head RMSNorm of q and k, after the bias and
        // before RoPE, with the model's epsilon (model.cpp:390-399, 584-593)
        if (cfg.qk_norm)
            CK(orc_qk_norm(d_qkv_, QKV, n, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, L.q_norm, L.k_norm, cfg.rms_eps,
                           s));
        // RoPE + KV store (model.cpp:401-408), attention (model.cpp:410-435).
        // Prefill passes of kPrefillAttnMin tokens or more (host positions):
        // one launch over the pass (query blocks, online softmax; the
        // prefill attention of model.cpp:595-626). Otherwise launches of at
        // most kMaxBatch tokens, in order: each stores its tokens' K / V rows
        // before the next attends to them.
        if (fused_attn_ && !d_pos && n >= kPrefillAttnMin) {
            CK(orc_attn_prefill(d_qkv_, QKV, n, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, sp, d_rope_, kc, vc, C,
                                d_attn_, NQ, s));
        } else for (int a0 = 0; a0 < n; a0 += kMaxBatch) {
            const int an = std::min(kMaxBatch, n - a0);
            float* qkv = d_qkv_ + (size_t)a0 * QKV;
            float* att = d_attn_ + (size_t)a0 * NQ;
            if (fused_attn_) {  // one launch: rotate, store K/V, attend
                const bool band = d_pos && pos_limit_ > 0;  // a capture that declared its positions
                const int lim = band && pos_limit_ < C ? pos_limit_ : C;
                const int flo = band && pos_floor_ < lim ? pos_floor_ : 0;
                CK(orc_attn_fused_at(qkv, QKV, an, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, d_pos, sp + a0,
                                     d_rope_, kc, vc, C, flo, lim, att, NQ, d_attn_ws_, s));
            } else {
                CK(orc_rope_kv_store_at(qkv, QKV, an, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, d_pos, sp + a0,
                                        d_rope_, kc, vc, C, s));
                CK(orc_attn_gqa_at(qkv, QKV, an, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, d_pos, sp + a0, kc, vc,
                                   C, att, NQ, d_attn_ws_, s));
            }
        }
        // x += O attn   (model.cpp:438-444)
        CK(gemm_segs({{&L.o, {d_x_, nullptr}}}, n, d_attn_, NQ, D, nullptr, ORC_EPI_ACCUM, s));
        // h = silu(gate xn) * up xn   (model.cpp:449-464)
        CK(gemm_segs({{&L.gate, {d_h_, nullptr}}, {&L.up, {d_h_, nullptr}}}, n, d_x_, D, FF, L.ffn_norm,
                     ORC_EPI_SWIGLU, s));
        // x += down h   (model.cpp:467-473)
        CK(gemm_segs({{&L.down, {d_x_, nullptr}}}, n, d_h_, FF, D, nullptr, ORC_EPI_ACCUM, s));
    }
    if (logits) {  // final norm + LM head (model.cpp:479-492)
        CK(gemm_segs({{&head_, {d_logits_, nullptr}}}, n, d_x_, D, V, out_norm_, ORC_EPI_STORE, s));
        if (d_argmax) CK(orc_argmax(d_logits_, n, V, V, d_argmax, d_am_ws_, s));
    }
#undef CK
    return 0;
}

int Model::forward_dev(const int32_t* d_ids, int n, int sp, bool logits, int32_t* d_argmax, orc_stream_t s) {
    if (!loaded_) return ORC_E_INVALID;
    if (n <= 0) return 0;
    if (sp < 0 || sp + n > (int)cfg.ctx_len) {
        err_ = "positions exceed the context length";
        return ORC_E_INVALID;
    }
    if (n > kMaxBatch && logits) {
        err_ = "logits for more than kMaxBatch tokens per call";
        return ORC_E_INVALID;
    }
    const int chunk = logits ? kMaxBatch : kPrefillBatch;
    for (int t0 = 0; t0 < n; t0 += chunk) {
        const int m = std::min(chunk, n - t0);
        if (int rc = chunk_dev(d_ids + t0, m, nullptr, sp + t0, logits, d_argmax ? d_argmax + t0 : nullptr, s)) {
            err_ = orc_last_error();
            return rc;
        }
    }
    return 0;
}

int Model::forward_dev_at(const int32_t* d_ids, int n, const int32_t* d_pos, int pos_off, bool logits,
                          int32_t* d_argmax, orc_stream_t s) {
    if (!loaded_) return ORC_E_INVALID;
    if (n <= 0) return 0;
    if (n > kMaxBatch) {
        err_ = "forward_dev_at: more than kMaxBatch tokens";
        return ORC_E_INVALID;
    }
    if (int rc = chunk_dev(d_ids, n, d_pos, pos_off, logits, d_argmax, s)) {
        err_ = orc_last_error();
        return rc;
    }
    return 0;
}

const float* Model::forward(int32_t token_id, int pos, bool compute_logits) {  // model.cpp:340-495
    if (!loaded_) return nullptr;
    if (token_id < 0 || token_id >= (int32_t)cfg.n_vocab) {
        std::fprintf(stderr, "[Model] token id %d out of range, using 0\n", token_id);
        token_id = 0;
    }
    if (orc_memcpy_h2d(d_ids_, &token_id, 4, nullptr)) return nullptr;
    if (forward_dev(d_ids_, 1, pos, compute_logits, nullptr, nullptr)) return nullptr;
    if (!compute_logits) {
        orc_stream_sync(nullptr);
        return nullptr;
    }
    if (orc_memcpy_d2h(logits_.data(), d_logits_, (size_t)cfg.n_vocab * 4, nullptr)) return nullptr;
    return logits_.data();
}

void Model::forward_prefill(const int32_t* tokens, int n, int sp, float* out_logits) {  // model.cpp:510-674
    if (!loaded_ || n <= 0) return;
    err_.clear();
    std::vector<int32_t> ids(tokens, tokens + n);
    for (auto& t : ids)
        if (t < 0 || t >= (int32_t)cfg.n_vocab) {
            std::fprintf(stderr, "[Model] forward_prefill: token id %d out of range, using 0\n", t);
            t = 0;
        }
    const int chunk = out_logits ? kMaxBatch : kPrefillBatch;  // logits rows fit kMaxBatch tokens
    for (int t0 = 0; t0 < n; t0 += chunk) {
        const int m = std::min(chunk, n - t0);
        if (orc_memcpy_h2d(d_ids_, ids.data() + t0, (size_t)m * 4, nullptr)) return;
        if (chunk_dev(d_ids_, m, nullptr, sp + t0, out_logits != nullptr, nullptr, nullptr)) {
            err_ = orc_last_error();
            std::fprintf(stderr, "[Model] forward_prefill failed: %s\n", err_.c_str());
            return;
        }
        if (out_logits)
            orc_memcpy_d2h(out_logits + (size_t)t0 * cfg.n_vocab, d_logits_, (size_t)m * cfg.n_vocab * 4, nullptr);
    }
    orc_stream_sync(nullptr);
}

// ── embedding, KV snapshot and .orkv files ──────────────────────────────────

std::vector<float> Model::embed_tokens(const std::vector<int32_t>& tokens) {  // model.cpp:248-270
    if (tokens.empty() || !loaded_) return {};
    const int D = cfg.embed_dim, n = (int)tokens.size();
    if (n > (int)cfg.ctx_len) {
        fail("embed_tokens: more tokens than the context holds");
        return {};
    }
    std::vector<int32_t> ids(tokens);
    for (auto& t : ids)
        if (t < 0 || t >= (int32_t)cfg.n_vocab) t = 0;  // model.cpp:352-356
    std::vector<float> acc((size_t)D, 0.f), xs((size_t)kPrefillBatch * D);
    reset();
    for (int t0 = 0; t0 < n; t0 += kPrefillBatch) {
        const int m = std::min(kPrefillBatch, n - t0);
        if (orc_memcpy_h2d(d_ids_, ids.data() + t0, (size_t)m * 4, nullptr) ||
            chunk_dev(d_ids_, m, nullptr, t0, false, nullptr, nullptr) ||
            orc_memcpy_d2h(xs.data(), d_x_, (size_t)m * D * 4, nullptr)) {
            fail(std::string("embed_tokens: ") + orc_last_error());
            reset();
            return {};
        }
        for (int t = 0; t < m; ++t)
            for (int d = 0; d < D; ++d) acc[d] += xs[(size_t)t * D + d];
    }
    const float inv_n = 1.f / n;
    float norm2 = 0.f;
    for (int d = 0; d < D; ++d) {
        acc[d] *= inv_n;
        norm2 += acc[d] * acc[d];
    }
    const float inv_norm = 1.f / (std::sqrt(norm2) + 1e-9f);
    for (float& v : acc) v *= inv_norm;
    reset();
    return acc;
}

Model::KVSnapshot Model::snapshot_kv(int pos) const {
    KVSnapshot s;
    s.pos = pos;
    if (!loaded_) return s;
    const size_t bytes = (size_t)cfg.n_layers * cfg.n_kv_total() * cfg.ctx_len * sizeof(float);
    void *k = nullptr, *v = nullptr;
    if (orc_malloc(&k, bytes) || orc_malloc(&v, bytes)) {
        if (k) orc_free(k);
        std::fprintf(stderr, "[Model] snapshot_kv: %s\n", orc_last_error());
        return s;
    }
    s.k.reset(k, [](void* q) { orc_free(q); });
    s.v.reset(v, [](void* q) { orc_free(q); });
    if (orc_memcpy_d2d(k, d_k_, bytes, nullptr) || orc_memcpy_d2d(v, d_v_, bytes, nullptr) ||
        orc_stream_sync(nullptr)) {
        std::fprintf(stderr, "[Model] snapshot_kv: %s\n", orc_last_error());
        return KVSnapshot{nullptr, nullptr, 0, pos};
    }
    s.bytes = bytes;
    return s;
}

void Model::restore_kv(const KVSnapshot& snap) {
    err_.clear();
    const size_t bytes = (size_t)cfg.n_layers * cfg.n_kv_total() * cfg.ctx_len * sizeof(float);
    if (!loaded_ || !snap.k || !snap.v || snap.bytes != bytes) {
        fail("restore_kv: the snapshot is empty or of another shape");
        return;
    }
    if (orc_memcpy_d2d(d_k_, snap.k.get(), bytes, nullptr) || orc_memcpy_d2d(d_v_, snap.v.get(), bytes, nullptr) ||
        orc_stream_sync(nullptr))
        fail(std::string("restore_kv: ") + orc_last_error());
}

static constexpr uint32_t kOrkvMagic = 0x564B524Fu;  // "ORKV" little-endian (model.cpp:11-12)
static constexpr uint32_t kOrkvVersion = 2u;
static_assert(sizeof(ModelConfig) == 44, "ModelConfig must keep the reference's layout");

// Device KV [layer][kv_head][pos][hd] <-> file [layer][pos][kv_head * hd],
// one layer at a time through host buffers.
bool Model::save_state(const std::string& path, int pos) const {  // model.cpp:156-181
    if (!loaded_) return false;
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) {
        std::fprintf(stderr, "[Model] save_state: cannot open %s\n", path.c_str());
        return false;
    }
    const size_t C = cfg.ctx_len, H = cfg.n_kv_heads, hd = cfg.head_dim, per = C * H * hd;
    const uint32_t ipos = (uint32_t)pos;
    const uint64_t n = (uint64_t)cfg.n_layers * per;
    bool ok = std::fwrite(&kOrkvMagic, 4, 1, f) == 1 && std::fwrite(&kOrkvVersion, 4, 1, f) == 1 &&
              std::fwrite(&cfg, sizeof(ModelConfig), 1, f) == 1 && std::fwrite(&ipos, 4, 1, f) == 1 &&
              std::fwrite(&n, 8, 1, f) == 1;
    std::vector<float> dev(per), file(per);
    for (int which = 0; which < 2 && ok; ++which) {
        const float* src = which ? d_v_ : d_k_;
        for (uint32_t l = 0; l < cfg.n_layers && ok; ++l) {
            ok = orc_memcpy_d2h(dev.data(), src + l * per, per * 4, nullptr) == 0;
            for (size_t h = 0; ok && h < H; ++h)
                for (size_t p = 0; p < C; ++p)
                    std::memcpy(&file[(p * H + h) * hd], &dev[(h * C + p) * hd], hd * 4);
            ok = ok && std::fwrite(file.data(), 4, per, f) == per;
        }
    }
    std::fclose(f);
    if (!ok) std::fprintf(stderr, "[Model] save_state: incomplete write to %s\n", path.c_str());
    return ok;
}

bool Model::load_state(const std::string& path, int& pos) {  // model.cpp:184-236
    if (!loaded_) return false;
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    auto bad = [&](const char* why) {
        std::fprintf(stderr, "[Model] load_state: %s (%s)\n", why, path.c_str());
        std::fclose(f);
        return false;
    };
    uint32_t magic = 0, ver = 0;
    if (std::fread(&magic, 4, 1, f) != 1 || std::fread(&ver, 4, 1, f) != 1 || magic != kOrkvMagic ||
        ver != kOrkvVersion)
        return bad("not a compatible .orkv file");
    ModelConfig lc;
    if (std::fread(&lc, sizeof(ModelConfig), 1, f) != 1) return bad("truncated header");
    if (lc.n_layers != cfg.n_layers || lc.embed_dim != cfg.embed_dim || lc.ctx_len != cfg.ctx_len ||
        lc.n_kv_heads != cfg.n_kv_heads || lc.head_dim != cfg.head_dim)
        return bad("configuration differs from the loaded model (layers/embed/ctx/kv_heads/head_dim)");
    uint32_t ipos = 0;
    uint64_t n = 0;
    if (std::fread(&ipos, 4, 1, f) != 1 || std::fread(&n, 8, 1, f) != 1) return bad("truncated header");
    const size_t C = cfg.ctx_len, H = cfg.n_kv_heads, hd = cfg.head_dim, per = C * H * hd;
    if (n != (uint64_t)cfg.n_layers * per) return bad("KV size does not match the configuration");
    // read everything before touching the device cache (a truncated file
    // leaves it as it was)
    std::vector<float> file(2 * n);
    if (std::fread(file.data(), 4, 2 * n, f) != 2 * n) return bad("truncated KV data");
    std::fclose(f);
    std::vector<float> dev(per);
    for (int which = 0; which < 2; ++which) {
        float* dst = which ? d_v_ : d_k_;
        for (uint32_t l = 0; l < cfg.n_layers; ++l) {
            const float* src = file.data() + (size_t)which * n + (size_t)l * per;
            for (size_t h = 0; h < H; ++h)
                for (size_t p = 0; p < C; ++p) std::memcpy(&dev[(h * C + p) * hd], &src[(p * H + h) * hd], hd * 4);
            if (orc_memcpy_h2d(dst + l * per, dev.data(), per * 4, nullptr))
                return fail(std::string("load_state: ") + orc_last_error());
        }
    }
    pos = (int)ipos;
    return true;
}

bool Model::test_norm_cache_matches() {  // core/model.hpp:119-121, core/model.cpp:296-313
    if (!loaded_) return false;
    const int D = cfg.embed_dim, Hd = cfg.head_dim;
    std::vector<float> dev((size_t)std::max(D, Hd));
    auto same = [&](const std::string& name, const float* d, int n) {
        const uint8_t* raw = gguf_.tensor_raw(name);
        return raw && d && orc_memcpy_d2h(dev.data(), d, (size_t)n * 4, nullptr) == 0 &&
               std::memcmp(dev.data(), raw, (size_t)n * 4) == 0;
    };
    if (!same("output_norm.weight", out_norm_, D)) return false;
    for (uint32_t l = 0; l < cfg.n_layers; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        if (!same(b + "attn_norm.weight", layers_[l].attn_norm, D) ||
            !same(b + "ffn_norm.weight", layers_[l].ffn_norm, D))
            return false;
        if (cfg.qk_norm && (!same(b + "attn_q_norm.weight", layers_[l].q_norm, Hd) ||
                            !same(b + "attn_k_norm.weight", layers_[l].k_norm, Hd)))
            return false;
    }
    return true;
}

double Model::weight_bytes(bool logits) const {
    double b = 0;
    auto mb = [](const Mat& m) { return (double)orc_row_bytes(m.type, m.n_in) * m.n_out; };
    for (const Layer& L : layers_) b += mb(L.q) + mb(L.k) + mb(L.v) + mb(L.o) + mb(L.gate) + mb(L.up) + mb(L.down);
    if (logits) b += mb(head_);
    return b;
}

double Model::decode_bytes(int pos, bool logits) const {
    const double kv = 2.0 * 4.0 * cfg.n_layers * cfg.n_kv_total();
    return weight_bytes(logits) + kv * (pos + 1) + kv;  // read K,V for positions <= pos; write this position
}

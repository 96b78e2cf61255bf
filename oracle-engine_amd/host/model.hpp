// Model — the reference's transformer API (core/model.hpp:10-121) with every
// weight, activation and the KV cache resident in HBM.
//
// Drop-in surface: ModelConfig, load, forward(token, pos, compute_logits)
// returning host logits, forward_prefill / forward_batch, reset, warmup, cfg,
// gguf(). The hot path uses the *_dev entry points: tokens, logits and argmax
// ids stay on the device, and a step is a fixed sequence of fused kernels:
//   embed -> per layer [ norm+QKV(+bias) | RoPE+KV store | GQA attention |
//   O-proj += residual | norm+gate/up+SwiGLU | down += residual ] ->
//   norm+LM head -> argmax.
// One decode step and one (k+1)-token verify pass run the same kernels, and the
// GEMM is batch-invariant, so verify logits equal decode logits bit for bit.
#pragma once
#include "gguf_parser.hpp"
#include "orc.h"

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

// core/model.hpp:10-27; the same field order and types, so the .orkv
// header (which stores the struct's bytes) is interchangeable.
struct ModelConfig {
    uint32_t n_vocab = 0;
    uint32_t n_layers = 0;
    uint32_t n_heads = 0;
    uint32_t n_kv_heads = 0;
    uint32_t embed_dim = 0;
    uint32_t ffn_hidden = 0;
    uint32_t head_dim = 0;
    uint32_t ctx_len = 512;
    float rope_freq = 500000.f;
    float rms_eps = 1e-5f;
    bool qk_norm = false;
    uint32_t n_gqa() const { return n_heads / n_kv_heads; }
    uint32_t n_q_total() const { return n_heads * head_dim; }
    uint32_t n_kv_total() const { return n_kv_heads * head_dim; }
};

class Model {
public:
    ModelConfig cfg;
    static constexpr int kMaxBatch = 16;      // tokens per device pass with logits (verify)
    static constexpr int kPrefillBatch = 1024;  // tokens per device pass without logits (prefill)
    // Passes of this many tokens or more run orc_attn_prefill (the prompts of
    // the 127-255-id configurations keep the verify path's attention).
    static constexpr int kPrefillAttnMin = 256;

    Model() = default;
    ~Model();
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    // Loads and uploads the model. ctx_len = 0 keeps the reference's 512
    // (core/model.cpp:64); a larger value sizes the device KV cache for it.
    bool load(const std::string& gguf_path, int ctx_len = 0);
    bool is_loaded() const { return loaded_; }
    // Distinct for every successful load of any Model in the process (keys
    // captured graphs, which bake in this model's device buffers).
    uint64_t uid() const { return uid_; }

    // Reference-compatible host API.
    const float* forward(int32_t token_id, int pos, bool compute_logits = true);
    void forward_prefill(const int32_t* tokens, int n, int start_pos = 0, float* out_logits = nullptr);
    void forward_batch(const int32_t* tokens, int n, int start_pos, float* out_logits) {
        forward_prefill(tokens, n, start_pos, out_logits);
    }
    void reset();
    void warmup();
    const GGUFParser& gguf() const { return gguf_; }

    // core/model.hpp:100 / model.cpp:248-270: the mean over the tokens of the
    // hidden state after the last layer (before the final norm), L2
    // normalised (1 / (|acc| + 1e-9)); the KV cache is cleared before and
    // after. The tokens run as batched passes; the pooling follows the
    // reference's float order on the host. Empty on error.
    std::vector<float> embed_tokens(const std::vector<int32_t>& tokens);

    // core/model.hpp:103-105: a copy of the whole KV cache, here in device
    // memory (a device-to-device copy each way). restore_kv takes only a
    // snapshot of this model's shape; pos is carried for the caller.
    struct KVSnapshot {
        std::shared_ptr<void> k, v;
        size_t bytes = 0;
        int pos = 0;
    };
    KVSnapshot snapshot_kv(int pos) const;
    void restore_kv(const KVSnapshot& snap);

    // core/model.hpp:108-116 / model.cpp:156-236: the reference's .orkv file
    // (magic "ORKV", version 2, the ModelConfig bytes, pos, then the K and V
    // caches as [layer][pos][kv_head x head_dim] floats), converted from and
    // to the device layout [layer][kv_head][pos][head_dim]. load_state
    // rejects the files the reference rejects.
    bool save_state(const std::string& path, int pos) const;
    bool load_state(const std::string& path, int& pos);

    // core/model.hpp:120: the norm weights the device reads equal the file's.
    bool test_norm_cache_matches();

    // Device hot path. d_ids: n token ids in HBM at positions start_pos..;
    // when compute_logits, logits of every position go to d_logits() and, if
    // d_argmax is non-null, the first-index argmax of each row to d_argmax.
    // Returns 0 or an ORC_E_* code. Nothing crosses to the host.
    int forward_dev(const int32_t* d_ids, int n, int start_pos, bool compute_logits, int32_t* d_argmax,
                    orc_stream_t s = nullptr);
    // As forward_dev with the first position read on the device (*d_pos +
    // pos_off), so a captured graph of the call replays at any position; the
    // caller keeps positions inside the context. n <= kMaxBatch.
    int forward_dev_at(const int32_t* d_ids, int n, const int32_t* d_pos, int pos_off, bool compute_logits,
                       int32_t* d_argmax, orc_stream_t s = nullptr);
    // Bounds on the device positions of the passes recorded while they are set
    // (a captured graph replays them at later positions): floor <= position <
    // limit; 0, 0: none. They size the attention grids; results do not depend
    // on them.
    void set_pos_band(int floor, int limit) {
        pos_floor_ = floor;
        pos_limit_ = limit;
    }
    float* d_logits() const { return d_logits_; }
    const char* last_error() const { return err_.c_str(); }

    // Bytes read from HBM by one decode step at position pos (weights + LM
    // head + KV), for roofline reports.
    double decode_bytes(int pos, bool logits = true) const;
    double weight_bytes(bool logits = true) const;

private:
    struct Mat {
        int type = -1;
        const uint8_t* d = nullptr;
        int n_in = 0, n_out = 0;
    };
    struct Layer {
        Mat q, k, v, o, gate, up, down;
        const float *attn_norm = nullptr, *ffn_norm = nullptr, *bq = nullptr, *bk = nullptr, *bv = nullptr;
        const float *q_norm = nullptr, *k_norm = nullptr;  // QK-norm weights (head_dim each)
    };
    GGUFParser gguf_;
    bool loaded_ = false;
    uint64_t uid_ = 0;
    bool fused_attn_ = false;  // one-launch RoPE + KV store + attention supports this shape
    int pos_floor_ = 0, pos_limit_ = 0;
    std::vector<Layer> layers_;
    Mat embd_, head_;
    const float* out_norm_ = nullptr;
    float *d_x_ = nullptr, *d_qkv_ = nullptr, *d_attn_ = nullptr, *d_h_ = nullptr, *d_logits_ = nullptr;
    float *d_k_ = nullptr, *d_v_ = nullptr, *d_rope_ = nullptr;
    int32_t *d_ids_ = nullptr, *d_am_ = nullptr;
    void *d_attn_ws_ = nullptr, *d_am_ws_ = nullptr;
    std::vector<float> logits_;
    std::string err_;

    bool fail(const std::string& m);
    int chunk_dev(const int32_t* d_ids, int n, const int32_t* d_pos, int start_pos, bool logits, int32_t* d_argmax,
                  orc_stream_t s);
    int gemm_segs(const std::vector<std::pair<const Mat*, std::pair<float*, const float*>>>& segs, int n,
                  const float* x, int ldx, int ldy, const float* norm, int epi, orc_stream_t s);
    void free_dev();
};

/*
 * oracle_host.h — C API of the C++ host (liboracle_host.so) that mirrors the
 * reference's Model / harness API on top of orc.h. It exists so that
 * non-C++ callers (the Python tests and bench.py, a ctypes/cgo binding) can
 * drive whole decode loops; C++ callers use host/model.hpp and host/spec.hpp
 * directly. Every entry point names the reference API it exposes.
 */
#ifndef ORACLE_HOST_H
#define ORACLE_HOST_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct orch_model orch_model;

/* Model::load (core/model.cpp:17-96); ctx_len 0 keeps the reference's 512. */
orch_model* orch_load(const char* gguf_path, int ctx_len);
void orch_free(orch_model* m);
/* Message of the last failure (load or call), "" if none. */
const char* orch_error(const orch_model* m);
/* cfg[0..9] = n_vocab, n_layers, n_heads, n_kv_heads, embed_dim, ffn_hidden,
 * head_dim, ctx_len, has_qkv_bias, tied_head (ModelConfig, core/model.hpp:10-27). */
int orch_cfg(const orch_model* m, int32_t* cfg, float* rope_freq);
/* Model::reset (core/model.hpp:92). */
int orch_reset(orch_model* m);
/* Model::forward (core/model.cpp:340-495); logits may be NULL (no LM head). */
int orch_forward(orch_model* m, int32_t token, int pos, float* logits);
/* Model::forward_prefill / forward_batch (core/model.cpp:510-674); logits
 * [n][n_vocab] may be NULL. */
int orch_forward_batch(orch_model* m, const int32_t* tokens, int n, int start_pos, float* logits);
/* Harness greedy decode (benchmark/bench_engine.cpp:221-243): if prefill,
 * reset + batched prefill of n_prompt-1 tokens; then n_gen argmax steps.
 * Returns tokens written (<0 on error). */
int orch_greedy(orch_model* m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out, int prefill);
/* Harness speculative greedy decode (benchmark/bench_engine.cpp:285-363)
 * with draft length k; stats[0..3] = accepted, proposed, target passes,
 * rounds. Returns tokens written. */
int orch_spec_greedy(orch_model* tgt, orch_model* dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                     int32_t* out, int64_t* stats, int prefill);
/* The Engine's stochastic speculative loop (core/engine.cpp:100-240) with
 * the device sampler: resets both models, prefills n_prompt-1 tokens (also
 * recorded in the sampler history), greedy draft of k, target sampling at
 * every verify position (sample + the Engine's second record), accept while
 * equal, refill the draft when all k match. sampler = temperature, top_p,
 * repeat_penalty; isampler = top_k, repeat_last; seed as std::mt19937 takes
 * it. stats[0..2] = accepted, proposed, target forwards. Returns tokens
 * written. */
int orch_spec_engine(orch_model* tgt, orch_model* dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                     const float* sampler, const int32_t* isampler, uint64_t seed, int32_t* out, int64_t* stats);
/* Speculative sampling with the exact-distribution rule (no reference
 * counterpart; the reference's Engine accepts on equal samples, as
 * orch_spec_engine does). Same reset, prefill, recorded prompt and sampler
 * arguments as orch_spec_engine. Per round the draft proposes k ids, each
 * drawn from its logits through the sampler transform (penalty window =
 * history + the round's earlier proposals); the target scores the round in
 * one batched pass; proposal i is accepted with min(1, p_i/q_i); the first
 * rejection emits a draw from norm(max(0, p_i - q_i)); a fully accepted round
 * emits a bonus draw from p_k. Every emitted id is recorded once. The emitted
 * stream is distributed as sampling the target alone. stats[0..2] =
 * accepted, proposed, target passes. Returns tokens written. */
int orch_spec_sampled(orch_model* tgt, orch_model* dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                      const float* sampler, const int32_t* isampler, uint64_t seed, int32_t* out, int64_t* stats);
/* Decode loops replay captured HIP graphs (on, the default) or launch every
 * kernel from the host (off); the token streams are identical. Drops the
 * graphs captured so far (the next loop captures them again, e.g. with
 * kernel timing events once orc_prof_enable is on). Returns the previous
 * setting. No reference counterpart. */
int orch_set_graphs(int on);
/* Quantized weight bytes one decode step streams (layers + LM head if logits). */
double orch_weight_bytes(const orch_model* m, int logits);
/* Block the host until all device work of the library has finished. */
int orch_sync(void);

/* The model's GGUFParser drop-ins on host buffers (model.gguf() in C++):
 * n_tok = 1: GGUFParser::gemv_q_range(tensor, out, x, j0, j1, n_in) — out[j]
 * for j in [j0, j1) (core/gguf_parser.cpp:868-911); n_tok > 1 (j0 = 0):
 * GGUFParser::gemm_q(tensor, out, x, n_tok, j1, n_in) — out[t * j1 + j]
 * (core/gguf_parser.cpp:919-997). They read the tensor in the layout its HBM
 * bytes hold after Model::load (orch_gguf_device_type: the GGML type, or
 * ORC_Q8_0_X8 = 258 for a regrouped Q8_0 matrix). */
int orch_gguf_device_type(const orch_model* m, const char* tensor);
int orch_gguf_gemm(orch_model* m, const char* tensor, const float* x, int n_tok, int j0, int j1, float* out);
/* GGUFParser::dequantize_row (core/gguf_parser.cpp:443-482): row `row` of the
 * tensor as fp32 into out (shape[0] floats), bit-exact. */
int orch_gguf_dequant_row(orch_model* m, const char* tensor, int64_t row, float* out);

/* ── the rest of the reference's Model surface ─────────────────────────────── */
/* Model::embed_tokens (core/model.cpp:248-270): embed_dim floats into out. */
int orch_embed_tokens(orch_model* m, const int32_t* tokens, int n, float* out);
/* Model::save_state / load_state (core/model.cpp:156-236), the .orkv file. */
int orch_save_state(orch_model* m, const char* path, int pos);
int orch_load_state(orch_model* m, const char* path, int* pos);
/* Model::snapshot_kv / restore_kv (core/model.hpp:103-105) through a handle. */
typedef struct orch_kv_snapshot orch_kv_snapshot;
orch_kv_snapshot* orch_snapshot_kv(orch_model* m, int pos);
int orch_restore_kv(orch_model* m, const orch_kv_snapshot* s);
int orch_snapshot_pos(const orch_kv_snapshot* s);
void orch_snapshot_free(orch_kv_snapshot* s);
/* Model::test_norm_cache_matches (core/model.hpp:119-121): 1 if equal. */
int orch_norm_cache_matches(orch_model* m);

/* ── namespace ops on host arrays (core/ops.hpp:42-92), run on the GPU ─────── */
void orch_ops_rmsnorm(float* out, const float* x, const float* w, int n, float eps);
void orch_ops_matmul(float* out, const float* a, const float* b, int m, int n, int k);
void orch_ops_matmul_nn(float* out, const float* a, const float* b, int m, int n, int k);
void orch_ops_silu(float* x, int n);
void orch_ops_mul(float* out, const float* a, const float* b, int n);
void orch_ops_add(float* a, const float* b, int n);
void orch_ops_copy(float* dst, const float* src, int n);
void orch_ops_softmax(float* x, int n);
void orch_ops_rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int pos, float freq_base);
int orch_ops_argmax(const float* x, int n);
float orch_ops_dot(const float* a, const float* b, int n);

/* ── Engine (core/engine.hpp:35-76) and Tokenizer (core/tokenizer.hpp:17-44) ── */
typedef struct orch_engine orch_engine;
/* Engine::load, then Engine::load_draft when draft_path is not NULL. */
orch_engine* orch_engine_new(const char* model_path, const char* draft_path);
void orch_engine_free(orch_engine* e);
const char* orch_engine_error(const orch_engine* e);
/* A fixed sampler seed for the following generate calls. */
void orch_engine_set_seed(orch_engine* e, uint64_t seed);
/* Engine::generate over n_msgs (roles[i], contents[i]) with GenParams
 * {n_predict, temperature, top_p, repeat_penalty, repeat_last_n}. The on_token
 * pieces go to out as (uint32 byte length, bytes) records; returns the bytes
 * written, or -1 (the pieces did not fit cap, or the engine failed). */
int64_t orch_engine_generate(orch_engine* e, const char* const* roles, const char* const* contents, int n_msgs,
                             int n_predict, float temperature, float top_p, float repeat_penalty, int repeat_last_n,
                             uint8_t* out, int64_t cap);
/* Engine::embed: embed_dim floats into out. */
int orch_engine_embed(orch_engine* e, const char* text, float* out);
/* A Tokenizer loaded from a GGUF's metadata alone (GGUFParser::load_meta:
 * no weights uploaded, no GPU needed). */
typedef struct orch_tokenizer orch_tokenizer;
orch_tokenizer* orch_tokenizer_load(const char* gguf_path);
void orch_tokenizer_free(orch_tokenizer* t);
/* Tokenizer::encode of text (len bytes): ids written (at most cap), or -1. */
int orch_tok_encode(orch_tokenizer* t, const char* text, int64_t len, int add_bos, int32_t* out, int cap);
/* Tokenizer::decode_one: the piece's byte length (written up to cap bytes). */
int orch_tok_decode_one(orch_tokenizer* t, int32_t id, char* out, int cap);
/* Tokenizer::special_id; bos_id (which = 0) or eos_id (which = 1). */
int32_t orch_tok_special_id(orch_tokenizer* t, const char* name);
int32_t orch_tok_bos_eos(orch_tokenizer* t, int which);

/* ── Sampler (core/sampler.hpp:24-48) on a device state ──────────────────────── */
typedef struct orch_sampler orch_sampler;
orch_sampler* orch_sampler_new(float temperature, float top_p, int top_k, float repeat_pen, int repeat_last,
                               uint64_t seed);
void orch_sampler_free(orch_sampler* s);
int32_t orch_sampler_sample(orch_sampler* s, float* logits, int n_vocab);
void orch_sampler_record(orch_sampler* s, int32_t id);
void orch_sampler_reset(orch_sampler* s);
void orch_sampler_set_params(orch_sampler* s, float temperature, float top_p, int top_k, float repeat_pen,
                             int repeat_last);

#ifdef __cplusplus
}
#endif
#endif

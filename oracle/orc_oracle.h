/*
 * orc_oracle — CPU restatement of ORACLE's speculative-decoding hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the parity checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product (the HIP library and its C++ host) never links or calls it.
 *
 * Every function states the reference file:line it restates. All arithmetic is
 * fp32 as in the reference; the decode path restates gemv_q (fused quantized
 * dots) and the verify path restates gemm_q (fp32 dequant, then fp32 dots),
 * because the reference rounds the two differently.
 */
#ifndef ORC_ORACLE_H
#define ORC_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (core/gguf_parser.hpp:9-24). */
enum { ORCO_F32 = 0, ORCO_F16 = 1, ORCO_Q4_0 = 2, ORCO_Q8_0 = 8, ORCO_Q4_K = 12, ORCO_Q6_K = 14, ORCO_BF16 = 30 };

float orco_fp16(uint16_t h);                                       /* gguf_parser.cpp:1002-1022 */
uint64_t orco_row_bytes(int type, int64_t n_el);                   /* gguf_parser.cpp:61-75 */
int orco_dequant(int type, const uint8_t* src, int64_t n, float* out); /* gguf_parser.cpp:420-482,1029-1154 */
float orco_dot(int type, const uint8_t* row, int n_in, const float* x); /* gguf_parser.cpp:496-866 */
int orco_gemv(int type, const uint8_t* w, int n_out, int n_in, const float* x, float* y);   /* :873-911 */
int orco_gemm(int type, const uint8_t* w, int n_tok, int n_out, int n_in, const float* x, float* y); /* :919-997 */

void orco_rmsnorm(float* out, const float* x, const float* w, int n, float eps); /* ops.cpp:149-195 */
void orco_rope(float* q, float* k, int n_heads, int n_kv_heads, int head_dim, int pos, float base); /* ops.cpp:440-485 */
void orco_softmax(float* x, int n);                                /* ops.cpp:386-435 */
void orco_silu(float* x, int n);                                   /* ops.cpp:308-334 */
int orco_argmax(const float* x, int n);                            /* ops.cpp:490-497 */
/* Causal GQA attention of one query token at position `pos` over a KV cache
 * laid out [ctx][n_kv_heads*head_dim] (model.cpp:410-435). */
void orco_attention(const float* q, const float* kc, const float* vc, int n_heads, int n_kv_heads, int head_dim,
                    int pos, float* out);

/* Model: GGUF load + config derivation (model.cpp:17-96), decode forward
 * (model.cpp:340-495) and batched forward (model.cpp:510-674). ctx_len is a
 * parameter (the reference fixes it to 512, model.cpp:64). */
typedef struct orco_model orco_model;
orco_model* orco_model_load(const char* path, int ctx_len);
void orco_model_free(orco_model* m);
/* cfg[0..9] = n_vocab, n_layers, n_heads, n_kv_heads, embed_dim, ffn_hidden, head_dim, ctx_len, has_bias, tied */
void orco_model_cfg(const orco_model* m, int32_t* cfg, float* rope_freq);
void orco_model_reset(orco_model* m);
/* Decode one token; writes n_vocab logits when `logits` is non-NULL. Returns 0 on success. */
int orco_model_forward(orco_model* m, int32_t token, int pos, float* logits);
/* Batched forward of n tokens at start_pos.. ; logits [n][n_vocab] when non-NULL. */
int orco_model_forward_batch(orco_model* m, const int32_t* tokens, int n, int start_pos, float* logits);
/* The last hidden state (after the final norm of the last forward), embed_dim floats. */
const float* orco_model_hidden(const orco_model* m);

/* Greedy decode with the harness protocol (bench_engine.cpp:221-243): batched
 * prefill of n_prompt-1 tokens, then n_gen decode steps. Returns n_gen. */
int orco_greedy(orco_model* m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out);
/* Speculative greedy with batched verify (bench_engine.cpp:300-356).
 * stats[0..2] = accepted, proposed, target passes. Returns tokens written. */
int orco_spec_greedy(orco_model* tgt, orco_model* dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                     int32_t* out, int64_t* stats);

/* std::mt19937 (32-bit seed) and the reference Sampler (sampler.cpp:7-105). */
typedef struct orco_sampler orco_sampler;
orco_sampler* orco_sampler_new(float temperature, float top_p, int top_k, float repeat_pen, int repeat_last,
                               uint64_t seed);
void orco_sampler_free(orco_sampler* s);
void orco_sampler_record(orco_sampler* s, int32_t tok);
int32_t orco_sampler_sample(orco_sampler* s, float* logits, int n_vocab); /* mutates logits, records */
uint32_t orco_mt_next(orco_sampler* s);                                     /* raw engine output */
/* The history window the penalty reads (most recent last); returns its length. */
int orco_sampler_history(const orco_sampler* s, int32_t* out, int cap);
/* Engine-style stochastic spec (engine.cpp:150-240) with a fixed seed; stats as above. */
int orco_spec_engine(orco_model* tgt, orco_model* dft, const int32_t* ids, int n_ids, int n_predict, int k,
                     orco_sampler* s, int32_t* out, int64_t* stats);

/* Probability transform used by both sampling schemes: penalty, temperature,
 * softmax, top-k (stable: lower index wins ties), top-p cut. Writes the
 * renormalised distribution over the kept set into p (zeros elsewhere).
 * Returns the size of the kept set. (sampler.cpp:15-86) */
int orco_transform_probs(const float* logits, int n, const int32_t* hist, int n_hist, float temperature,
                         float top_p, int top_k, float repeat_pen, float* p);
/* min(1, p/q) acceptance with residual resampling for one proposal `x`
 * (no reference counterpart): returns x when u_acc < p[x]/q[x], else a draw
 * from norm(max(0, p - q)) using u_res. */
int32_t orco_accept_resample(const float* p, const float* q, int n, int32_t x, float u_acc, float u_res,
                             int* accepted);
/* One draw from non-negative weights with the uniform u (first index where
 * the double running sum reaches u * total). */
int32_t orco_pick(const float* w, int n, float u);
/* One round's acceptance chain over rows p[0..k] and q[0..k-1] (n floats
 * each) for the proposals x[0..k-1]: u_acc per proposal from the sampler's
 * mt19937, accept when q_i[x_i] > 0 and u_acc * q_i[x_i] < p_i[x_i], else one
 * more uniform for the residual draw and stop; after k acceptances a bonus
 * draw from p_k. At most max_emit ids; each emitted id is recorded. Returns
 * the number emitted. */
int orco_accept_chain(orco_sampler* s, const float* p, const float* q, int n, const int32_t* x, int k, int max_emit,
                      int32_t* out, int* accepted, int* all);
/* Speculative sampling loop (no reference counterpart; the round shape is
 * bench_engine.cpp:300-356): the draft proposes x_i ~ q_i (its logits through
 * the sampler transform, pending proposals in the penalty window), the target
 * scores next, x_0..x_{k-1} in one batch, proposal i is accepted with
 * min(1, p_i/q_i), a rejection emits a residual draw, a fully accepted round
 * a bonus draw from p_k. Uniforms from the sampler's mt19937 in this order:
 * the k proposal draws, then per proposal u_acc (and u_res on rejection),
 * then the bonus. Emitted ids are recorded once; prompt[0..np-2] is
 * prefilled and recorded first (engine.cpp:115-125). Rounds run while
 * pos + k + 1 <= the smaller context. stats: accepted, proposed, rounds. */
int orco_spec_sampled(orco_model* tgt, orco_model* dft, const int32_t* prompt, int np, int n_gen, int k,
                      orco_sampler* s, int32_t* out, int64_t* stats);

#ifdef __cplusplus
}
#endif
#endif

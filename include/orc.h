/*
 * orc.h — C ABI of the MI355X (gfx950) kernels behind ORACLE's
 * speculative-decoding hot path.
 *
 * The reference (Titouan935/oracle-engine) has no FFI: its hot path is the C++
 * API of core/gguf_parser.hpp, core/ops.hpp, core/model.hpp and
 * core/sampler.hpp, linked statically. Each entry point below names the
 * reference function or loop it replaces (file:line in the reference tree).
 * The C++ host in oracle-engine_amd/host keeps that C++ API and calls only
 * these functions.
 *
 * Conventions
 *  - Every function returns 0 on success or a negative ORC_E_* code; the
 *    message of the last error on the calling thread is orc_last_error().
 *  - Pointers named d_* are device (HBM) pointers; h_* are host pointers.
 *  - All kernels are stream-ordered on `stream` (NULL = the library's default
 *    stream created by orc_init). Nothing allocates in a kernel entry point.
 *  - Floating-point data is fp32; quantized weights are raw GGML blocks exactly
 *    as stored in the GGUF file (type ids as in core/gguf_parser.hpp:9-24).
 *  - Matrices follow GGUF: a weight with shape [n_in, n_out] is n_out rows of
 *    n_in elements, rows contiguous; activations X are [n_tok][ldx] row-major.
 */
#ifndef ORC_H
#define ORC_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* error codes */
#define ORC_OK 0
#define ORC_E_INVALID (-1)     /* bad argument (shape, type, pointer) */
#define ORC_E_UNSUPPORTED (-2) /* quantization type or shape not supported */
#define ORC_E_HIP (-3)         /* a HIP runtime call failed */
#define ORC_E_NOINIT (-4)      /* orc_init was not called */

/* GGML type ids (core/gguf_parser.hpp:9-24) */
#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 30 /* dense weights: F32, F16 and BF16 rows run the vector GEMV */
#define ORC_Q4_0 2
#define ORC_Q8_0 8
#define ORC_Q4_K 12
#define ORC_Q6_K 14
/* Device layout of Q8_0 weights regrouped by orc_q8_0_regroup (no GGML
 * counterpart): every 8 consecutive blocks of a row (272 bytes) hold their 8
 * fp16 scales first (16 bytes), then their 8 x 32 int8 codes (256 bytes), so
 * every code load is 16-byte aligned. Same bytes per row as Q8_0; rows of a
 * multiple of 256 values. The GEMM entry points take it as a weight type and
 * give results bit-identical to the same matrix as Q8_0. */
#define ORC_Q8_0_X8 258

typedef void* orc_stream_t; /* a hipStream_t */
typedef void* orc_graph_t;  /* an instantiated hipGraphExec_t */
typedef void* orc_event_t;  /* a hipEvent_t */

/* ── runtime ─────────────────────────────────────────────────────────────── */
/* Select `device`, create the default stream. Replaces nothing in the
 * reference (CPU-only); called once by the host before any other entry point. */
int orc_init(int device);
int orc_shutdown(void);
const char* orc_last_error(void);
/* Device name, compute-unit count and HBM bytes (for reports). */
int orc_device_info(char* name, int name_cap, int* n_cu, size_t* hbm_bytes);

int orc_malloc(void** d_ptr, size_t bytes);
int orc_free(void* d_ptr);
int orc_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes, orc_stream_t stream);
int orc_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes, orc_stream_t stream);
int orc_memcpy_d2d(void* d_dst, const void* d_src, size_t bytes, orc_stream_t stream);
/* Fill with a byte value using a kernel (graph-capture safe). */
int orc_fill(void* d_dst, int byte_value, size_t bytes, orc_stream_t stream);
/* Allocate device memory and copy `bytes` raw GGUF bytes into it, unchanged.
 * Replaces the RAM preload of the data section (core/gguf_parser.cpp:112-138). */
int orc_upload(const void* h_src, size_t bytes, void** d_ptr);
int orc_stream_create(orc_stream_t* stream);
int orc_stream_destroy(orc_stream_t stream);
int orc_stream_sync(orc_stream_t stream);
int orc_device_sync(void);
/* Stream capture into a replayable graph (one decode step / one verify round). */
int orc_graph_begin(orc_stream_t stream);
int orc_graph_end(orc_stream_t stream, orc_graph_t* graph);
int orc_graph_launch(orc_graph_t graph, orc_stream_t stream);
int orc_graph_destroy(orc_graph_t graph);
int orc_event_create(orc_event_t* ev);
int orc_event_destroy(orc_event_t ev);
int orc_event_record(orc_event_t ev, orc_stream_t stream);
int orc_event_elapsed_ms(orc_event_t start, orc_event_t stop, float* ms);

/* ── quant codecs ────────────────────────────────────────────────────────── */
/* Bytes of one row of n_el elements of `type` (core/gguf_parser.cpp:61-75). */
int64_t orc_row_bytes(int type, int64_t n_el);
/* Regroups n_blocks8 groups of 8 consecutive Q8_0 blocks (272 bytes each,
 * e.g. n_rows * n_in / 256 for a matrix whose rows hold a multiple of 256
 * values) in place into the ORC_Q8_0_X8 layout. Apply once per matrix; the
 * matrix is then used with type ORC_Q8_0_X8 only. */
int orc_q8_0_regroup(void* d_w, int64_t n_blocks8, orc_stream_t stream);
/* Dequantize n_el contiguous elements to fp32, bit-exact with the reference
 * codecs: F32/F16/BF16/Q4_0/Q8_0/Q4_K/Q6_K (core/gguf_parser.cpp:1002-1154,
 * dequantize_into :420-441); also ORC_Q8_0_X8 (n_el a multiple of 256 from
 * the start of a regrouped row), with the values of the Q8_0 blocks it holds. */
int orc_dequant(int type, const void* d_w, int64_t n_el, float* d_y, orc_stream_t stream);
/* Embedding gather: y[t][:] = dequant(row ids[t] of an [n_in, n_rows] table);
 * ids outside [0, n_rows) read row 0 (model.cpp:352-358, 549-558 +
 * dequantize_row gguf_parser.cpp:443-482). ids is a device array. */
int orc_embed(int type, const void* d_table, int n_in, int n_rows, const int32_t* d_ids, int n_tok, float* d_y,
              int ldy, orc_stream_t stream);

/* ── quantized GEMV / GEMM ──────────────────────────────────────────────── */
/* Y[t][j] = dot(X[t], dequant(W[j])) for t < n_tok, j < n_out, fp32
 * accumulation. n_tok = 1 is the decode GEMV (gemv_q / gemv_q_range,
 * core/gguf_parser.cpp:868-911); n_tok > 1 is the verify / prefill GEMM
 * (gemm_q, core/gguf_parser.cpp:919-997). The per-(token,row) reduction order
 * does not depend on n_tok, so the verify pass is bit-identical to n_tok
 * separate GEMVs. Supported types: Q4_0, Q8_0, Q4_K, Q6_K, and the dense
 * F32, F16 and BF16 (n_in a multiple of 32), which the reference runs through
 * its dequantize + ops::matmul fallback (core/model.cpp:370-381): fp32 FMA
 * on the exactly widened values, one kernel family at every token count. */
int orc_gemm(int type, const void* d_w, int n_tok, int n_out, int n_in, const float* d_x, int ldx, float* d_y,
             int ldy, orc_stream_t stream);
static inline int orc_gemv(int type, const void* d_w, int n_out, int n_in, const float* d_x, float* d_y,
                           orc_stream_t stream) {
    return orc_gemm(type, d_w, 1, n_out, n_in, d_x, n_in, d_y, n_out, stream);
}

/* Fused multi-output GEMM: up to 3 weight matrices of one type sharing X and
 * n_in (e.g. Q|K|V, or gate|up), with an optional RMSNorm prologue applied to
 * each X row (ops::rmsnorm, core/ops.cpp:149-195, eps as given) and one of the
 * epilogues below. Replaces the projection sequences of Model::forward
 * (model.cpp:366-388, 449-473) and forward_prefill (model.cpp:565-581,
 * 629-643). */
#define ORC_EPI_STORE 0  /* y = W·x (+ bias)                          */
#define ORC_EPI_ACCUM 1  /* y += W·x   (residual add, model.cpp:444,473) */
#define ORC_EPI_SWIGLU 2 /* seg0 = gate, seg1 = up: y0 = silu(g) * u   */
typedef struct {
    const void* d_w;    /* weight rows */
    int n_out;          /* rows */
    float* d_y;         /* output column base; element (t, j) at d_y[t*ldy + j] */
    const float* d_bias;/* optional per-row bias (Qwen2 QKV bias, model.cpp:384-388) */
} orc_seg;
int orc_gemm_fused(int type, const orc_seg* segs, int n_segs, int n_tok, int n_in, const float* d_x, int ldx, int ldy,
                   const float* d_norm_w, float eps, int epilogue, orc_stream_t stream);

/* orc_gemm_fused over Q4_K and Q6_K segments of different types in one
 * launch on the matrix cores (the Q|K|V projections of a Q4_K_M layer, whose
 * attn_v is Q6_K: core/model.cpp:366-388). types[i] is segment i's type;
 * every segment has a positive multiple of 16 rows, fewer than 65536; store
 * or accumulate epilogue. Each segment's rows equal orc_gemm_fused on that
 * segment alone, bit for bit. No reference counterpart (the reference runs
 * one gemv_q per tensor). */
int orc_gemm_fused_mixed(const int* types, const orc_seg* segs, int n_segs, int n_tok, int n_in, const float* d_x,
                         int ldx, int ldy, const float* d_norm_w, float eps, int epilogue, orc_stream_t stream);

/* Live kernel timing (no reference counterpart; the reference times whole
 * loops with std::chrono, bench_engine.cpp:225-244). While enabled, every
 * GEMM launch made outside stream capture carries a start and a stop HIP
 * event (hipExtLaunchKernelGGL: both take the timestamps of the kernel's own
 * dispatch on its stream) and its algorithmic HBM bytes (weight blocks + x +
 * y) are noted; so does every attention launch of orc_attn_fused_at with
 * host positions (families ORC_PROF_ATTN_WG / _MT / _SPLIT / _MERGE, and
 * orc_attn_prefill: ORC_PROF_ATTN_PF; bytes = the K
 * and V rows its tokens read, counted once, + QKV rows in + rows out; the
 * merge is noted with 0 bytes). Once the work has run, orc_prof_accumulate
 * adds every launch's elapsed time to its record; orc_prof_read sums the
 * records of one kernel family (type = a GGML type id, 256 for mixed
 * Q4_K + Q6_K launches, or an attention family; type < 0: all families;
 * n_tok 0: all token counts). orc_prof_enable:
 * 1 = on and clear all records, 2 = on keeping them, 0 = off (accumulate is
 * then a no-op); returns the previous state. */
#define ORC_PROF_ATTN_WG 300
#define ORC_PROF_ATTN_SPLIT 301
#define ORC_PROF_ATTN_MERGE 302
#define ORC_PROF_ATTN_MT 303
#define ORC_PROF_ATTN_PF 304
int orc_prof_enable(int on);
int orc_prof_accumulate(void);
int orc_prof_read(int type, int n_tok, int64_t* launches, double* total_ms, double* total_bytes);

/* ── free functions on float arrays (namespace ops, core/ops.hpp:42-92) ──── */
/* Device arrays; fp32; reductions in a fixed order of the device, so results
 * match the reference's AVX2 loops to fp32 summation order. */
#define ORC_VEC_MUL 0  /* out = a * b  (ops::mul, ops.cpp:339-354)  */
#define ORC_VEC_ADD 1  /* out = a + b  (ops::add, ops.cpp:359-374)  */
#define ORC_VEC_COPY 2 /* out = a      (ops::copy, ops.cpp:379-381) */
int orc_vec_binary(int op, float* d_out, const float* d_a, const float* d_b, int n, orc_stream_t stream);
/* x = x / (1 + exp(-x)) in place (ops::silu, ops.cpp:308-334). */
int orc_vec_silu(float* d_x, int n, orc_stream_t stream);
/* Row-wise softmax in place of n_rows rows of n, ld floats apart
 * (ops::softmax, ops.cpp:386-435). */
int orc_softmax(float* d_x, int n, int n_rows, int ld, orc_stream_t stream);
/* *d_out = sum a[i] b[i] (ops::dot, ops.cpp:102-143). */
int orc_dot(const float* d_a, const float* d_b, int n, float* d_out, orc_stream_t stream);
/* out (m x n) = A (m x k) x B^T with B n x k when b_trans (ops::matmul,
 * ops.cpp:207-289), else A x B with B k x n (ops::matmul_nn, ops.cpp:294-303). */
int orc_matmul_f32(float* d_out, const float* d_a, const float* d_b, int m, int n, int k, int b_trans,
                   orc_stream_t stream);
/* Rotate-half RoPE of one position (ops::rope, ops.cpp:440-485) in place on
 * n_heads q heads and n_kv_heads k heads of head_dim values; d_cs holds the
 * position's head_dim/2 (cos, sin) pairs, computed on the host as the
 * reference does. An odd head_dim rotates the pairs (i, i + head_dim/2) and
 * leaves each head's last value as it is, as the reference does. */
int orc_rope_pos(float* d_q, float* d_k, int n_heads, int n_kv_heads, int head_dim, const float* d_cs,
                 orc_stream_t stream);

/* ── elementwise / attention ─────────────────────────────────────────────── */
/* out[t] = rmsnorm(x[t]) for n_rows rows of n (ops::rmsnorm, ops.cpp:149-195);
 * any n >= 1 (pointers 16-byte aligned when n is a multiple of 4). */
int orc_rmsnorm(float* d_out, const float* d_x, const float* d_w, int n, int n_rows, float eps, orc_stream_t stream);
/* QK-norm (Qwen3; core/model.cpp:390-399, 584-593): ops::rmsnorm over each
 * head of head_dim values, in place, on the q heads (weights d_qw) and k heads
 * (weights d_kw; head_dim floats each, shared by the heads) of n_tok QKV rows
 * [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)] with row stride ldqkv, before
 * RoPE; eps is the model's attention.layer_norm_rms_epsilon, as the reference
 * passes cfg.rms_eps there. 1 <= head_dim <= 128. */
int orc_qk_norm(float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim, const float* d_qw,
                const float* d_kw, float eps, orc_stream_t stream);
/* RoPE (rotate-half pairs (i, i+hd/2), theta = pos / base^(2i/hd),
 * ops::rope ops.cpp:440-485) on the q and k columns of n_tok QKV rows laid out
 * [q (n_heads*hd) | k (n_kv*hd) | v (n_kv*hd)] with row stride ldqkv, then
 * store k and v of token t at KV position start_pos + t (model.cpp:401-408,
 * 595-602). The cos/sin table d_rope is [max_pos][hd/2] pairs of floats built
 * on the host with the reference's float powf/cosf/sinf, so angles are
 * bit-identical. KV cache layout: [n_kv][ctx][hd] fp32 per layer. */
int orc_rope_kv_store(float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim, int start_pos,
                      const float* d_rope, float* d_kcache, float* d_vcache, int ctx, orc_stream_t stream);
/* As orc_rope_kv_store with the first position read on the device:
 * start_pos = *d_pos + pos_off (d_pos null: start_pos = pos_off). A graph
 * captured with a device position replays at whatever position the device
 * holds; tokens whose position falls outside [0, ctx) are skipped. No
 * reference counterpart (the reference passes pos by value,
 * core/model.cpp:340); used for captured decode / verify rounds. */
int orc_rope_kv_store_at(float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim,
                         const int32_t* d_pos, int pos_off, const float* d_rope, float* d_kcache, float* d_vcache,
                         int ctx, orc_stream_t stream);
/* Causal GQA attention for n_tok query tokens at positions start_pos..,
 * each attending to KV positions [0, start_pos + t] (model.cpp:410-435,
 * 604-626). q rows have stride ldq, output rows stride ldo. Scale
 * 1/sqrt(head_dim), softmax with max subtraction. Split over KV chunks with
 * an online-softmax merge; d_work needs orc_attn_workspace() bytes. */
size_t orc_attn_workspace(int n_tok, int n_heads, int head_dim, int max_pos);
int orc_attn_gqa(const float* d_q, int ldq, int n_tok, int n_heads, int n_kv, int head_dim, int start_pos,
                 const float* d_kcache, const float* d_vcache, int ctx, float* d_out, int ldo, void* d_work,
                 orc_stream_t stream);
/* As orc_attn_gqa with start_pos = *d_pos + pos_off read on the device (d_pos
 * null: start_pos = pos_off). With a device position the grid covers the whole
 * context, so the launch is valid for any position a replayed graph reaches;
 * d_work must hold orc_attn_workspace(n_tok, n_heads, head_dim, ctx) bytes. */
int orc_attn_gqa_at(const float* d_q, int ldq, int n_tok, int n_heads, int n_kv, int head_dim, const int32_t* d_pos,
                    int pos_off, const float* d_kcache, const float* d_vcache, int ctx, float* d_out, int ldo,
                    void* d_work, orc_stream_t stream);

/* RoPE + KV store + causal GQA attention in one launch (the attention block
 * of Model::forward / forward_prefill, core/model.cpp:401-435, 595-626):
 * for n_tok QKV rows (layout as orc_rope_kv_store, left unmodified) at
 * positions start_pos.. (start_pos = *d_pos + pos_off, or pos_off when d_pos
 * is null), rotates q and k, stores k and v of every token in the cache and
 * writes each token's attention output (rows of ldo floats). Results equal
 * orc_rope_kv_store followed by orc_attn_gqa up to fp32 rounding; a token's
 * result does not depend on n_tok. At most 8 query heads per kv head and 16
 * tokens per call; head_dim 64 or 128; 16-byte aligned rows.
 * A token attending to at most orc_attn_wg_limit() (512) positions is
 * computed by one workgroup per query head; a longer one's positions are
 * split over up to 256 chunks (64 positions each up to 16384, one workgroup
 * per chunk and kv head for all tokens of the call, on the matrix cores in
 * fp32; wider chunks above) whose partial
 * results a second launch merges: d_work holds orc_attn_fused_workspace(n_heads, n_kv,
 * head_dim) bytes, 16-byte aligned; calls that share a workspace must not
 * overlap. With device positions, every token position p of the call (or of
 * a captured graph replaying it at later device positions) must satisfy
 * pos_floor <= p < pos_limit (0 <= pos_floor < pos_limit <= ctx): the call
 * launches only the kernels such positions need (a token outside the range
 * may be left unwritten) and sizes their grids by pos_limit. Host-position
 * calls take pos_floor = 0, pos_limit = ctx. */
size_t orc_attn_fused_workspace(int n_heads, int n_kv, int head_dim);
/* Prefill form of orc_attn_fused_at (host positions pos_off.., any n_tok, no
 * workspace): RoPE on q and k, K / V of every token stored in the cache,
 * causal attention of each token over positions 0..its own, written to
 * d_out (rows of ldo floats); the same layouts, limits (head_dim 64 / 128,
 * at most 8 query heads per kv head) and alignment. One workgroup per
 * (16-token block, kv head) walks the key chunks with an online softmax:
 * within fp32 rounding of orc_attn_fused_at's results, not equal to them
 * bit for bit (core/model.cpp:595-626 is the prefill counterpart). */
int orc_attn_prefill(const float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim, int pos_off,
                     const float* d_rope, float* d_kc, float* d_vc, int ctx, float* d_out, int ldo,
                     orc_stream_t stream);
int orc_attn_wg_limit(void);
int orc_attn_fused_at(const float* d_qkv, int ldqkv, int n_tok, int n_heads, int n_kv, int head_dim,
                      const int32_t* d_pos, int pos_off, const float* d_rope, float* d_kcache, float* d_vcache,
                      int ctx, int pos_floor, int pos_limit, float* d_out, int ldo, void* d_work,
                      orc_stream_t stream);

/* ── argmax, sampling, acceptance ────────────────────────────────────────── */
/* out[r] = first index of the maximum of row r (ops::argmax ops.cpp:490-497,
 * bench_engine.cpp:82-88). d_work needs orc_argmax_workspace() bytes. */
size_t orc_argmax_workspace(int n_rows, int n);
int orc_argmax(const float* d_x, int n_rows, int n, int ld, int32_t* d_out, void* d_work, orc_stream_t stream);
/* orc_argmax without a workspace argument, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No reference counterpart. The partials go to a library-owned
 * 32 KiB device array, one per GPU, set up by orc_init; at most 16 rows per
 * call (ORC_E_INVALID beyond). Results equal orc_argmax's. It allocates and
 * clears nothing. Every call on one GPU shares that array: calls that overlap
 * on one GPU (different streams or threads without ordering) race. */
int orc_argmax_noalloc(const float* d_x, int n_rows, int n, int ld, int32_t* d_out, orc_stream_t stream);

/* Greedy acceptance of one batched verify round (bench_engine.cpp:337-355):
 * given the verify logits argmax ids tgt[0..n_draft] and the draft ids
 * d_draft[0..n_draft-1], writes out[0] = a (number accepted), out[1] = the
 * next token (first mismatch, or the bonus tgt[n_draft] when all match). */
int orc_spec_accept_greedy(const int32_t* d_tgt_ids, const int32_t* d_draft_ids, int n_draft, int32_t* d_out,
                           orc_stream_t stream);
/* Device-resident round state for captured spec rounds: as
 * orc_spec_accept_greedy, and also out[2 .. 2+a] = the emitted ids
 * tgt[0..a], *d_pos += a + 1 and *d_next = the next input token (d_out holds
 * n_draft + 3 ints). The position advance is bench_engine.cpp:352-355. */
int orc_spec_accept_greedy_at(const int32_t* d_tgt_ids, const int32_t* d_draft_ids, int n_draft, int32_t* d_out,
                              int32_t* d_pos, int32_t* d_next, orc_stream_t stream);
/* ── device sampler (core/sampler.cpp:7-105) ─────────────────────────────── */
/* Sampler state in device memory: mt19937 seeded with (uint32_t)seed as
 * std::mt19937 is (the reference passes a 64-bit seed that the engine
 * truncates, sampler.cpp:7-8), the parameters of SamplerParams
 * (sampler.hpp:16-22) and the history, initialised with n_hist recorded ids.
 * top_k 0 = all tokens, for vocabularies of at most 16384 tokens when
 * T > 0 (T <= 0 is the argmax and sorts nothing): with such a state,
 * orc_sample / orc_spec_accept_engine / orc_transform_probs on a larger
 * vocabulary return ORC_E_UNSUPPORTED. 0 <= repeat_last < 4096 (ORC_E_INVALID
 * beyond): the penalty over the last repeat_last entries is the reference's
 * at every such value; from 2048 up the history a full buffer keeps is its
 * last repeat_last entries (the reference keeps up to 2 * repeat_last). */
size_t orc_sampler_state_bytes(void);
int orc_sampler_init(void* d_state, float temperature, float top_p, int top_k, float repeat_penalty, int repeat_last,
                     uint64_t seed, const int32_t* d_hist, int n_hist, orc_stream_t stream);
/* Sampler::sample (sampler.cpp:91-97) on one row of n_vocab logits: penalty,
 * temperature, softmax, top-k, top-p, draw, record. Like the reference it
 * rewrites the row in place (it ends up holding the probabilities). */
int orc_sample(void* d_state, float* d_logits, int n_vocab, int32_t* d_out, orc_stream_t stream);
/* Sampler::record (sampler.cpp:99-105) of n device ids, in order. */
int orc_sampler_record(void* d_state, const int32_t* d_tok, int n, orc_stream_t stream);
/* The last min(cap, size) history entries into d_out, their count into *d_n. */
int orc_sampler_history(const void* d_state, int32_t* d_out, int cap, int32_t* d_n, orc_stream_t stream);
/* Sampler::set_params (sampler.hpp:37): new parameters; generator state and
 * history unchanged (limits as orc_sampler_init). */
int orc_sampler_set_params(void* d_state, float temperature, float top_p, int top_k, float repeat_penalty,
                           int repeat_last, orc_stream_t stream);
/* Sampler::reset (sampler.hpp:34): the history is cleared, the generator
 * keeps its state. */
int orc_sampler_clear_history(void* d_state, orc_stream_t stream);
/* Engine-style stochastic verify (core/engine.cpp:183-232) over the k+1 rows
 * of one batched verify pass (row i = target logits at the i-th verify
 * position, rows ld floats apart; rows are rewritten by sampling): for each
 * draft id, sample (recording it) and record it again as the Engine does,
 * stop at the first mismatch; if all k match, sample the bonus row the same
 * way. At most max_emit ids are emitted (or *d_budget, which is then
 * decremented). d_out: [0] emitted, [1] accepted, [2] rows sampled (the
 * reference's target forwards), [3] 1 if all drafts matched (the caller then
 * refills the draft's KV), [4..] the emitted ids (k+5 ints). With d_pos and
 * d_next the round state advances: *d_pos += emitted, *d_next = last id.
 * Up to 16 proposals, vocabularies up to 196608, T > 0 and
 * 1 <= top_k <= 128: every row's kept set is computed up front (row i's
 * penalty window is the history plus proposals 0 .. i-1 twice each, the only
 * case in which it is sampled) into the state's scratch, then drawn from in
 * row order; calls on one state must not overlap. */
int orc_spec_accept_engine(void* d_state, float* d_logits, int ld, int n_vocab, const int32_t* d_draft, int n_draft,
                           int max_emit, int32_t* d_budget, int32_t* d_out, int32_t* d_pos, int32_t* d_next,
                           orc_stream_t stream);

/* ── speculative sampling, min(1, p/q) with residual resampling ──────────────
 * No reference counterpart: the reference's Engine accepts a proposal when
 * the target's own sample equals it (core/engine.cpp:183-232), which the
 * functions above reproduce. These give the exact-distribution rule. */
/* The sampler's transform of `rows` rows of logits written out as
 * distributions: penalty over the history plus the pending proposals
 * d_extra[0 .. extra_base + r) for row r, temperature, softmax, top-k, top-p,
 * kept set renormalised into d_p (zeros elsewhere); T <= 0 puts all mass on
 * the argmax. The logits rows are rewritten (sampler.cpp:15-85 does the same
 * steps on one row). Nothing is recorded and no random number is drawn.
 * Up to 17 rows of up to 196608 logits, T > 0 and 1 <= top_k <= 128 run split
 * over many workgroups, with per-slice partial results kept in the state's
 * scratch area: calls on one state must not overlap. */
int orc_transform_probs(const void* d_state, float* d_logits, int ld, int n_vocab, int rows, const int32_t* d_extra,
                        int extra_base, float* d_p, int ldp, orc_stream_t stream);
/* One draw from the distribution d_p (one mt19937 uniform u; first index
 * where the running sum of p reaches u * sum(p)); the id goes to d_out[0] and,
 * if given, d_out2[0]. Not recorded. */
int orc_draw(void* d_state, const float* d_p, int n_vocab, int32_t* d_out, int32_t* d_out2, orc_stream_t stream);
/* orc_transform_probs of one row (pending proposals d_extra[0 .. n_extra))
 * followed by orc_draw from it, in one call: the draft step of a speculative
 * sampling round (the draft's q and its proposal). The draw reads the kept set
 * instead of the whole row; same uniform, same sums in index order. Like
 * orc_transform_probs it uses the state's scratch: calls on one state must not
 * overlap. */
int orc_transform_draw(void* d_state, float* d_logits, int n_vocab, const int32_t* d_extra, int n_extra, float* d_p,
                       int32_t* d_out, int32_t* d_out2, orc_stream_t stream);
/* The acceptance test of proposal x with explicit uniforms: accept when
 * q[x] > 0 and u_acc * q[x] < p[x]; otherwise draw from norm(max(0, p - q))
 * with u_res (argmax of p if that is empty). d_out = [id, accepted]. */
int orc_accept_resample(const float* d_p, const float* d_q, int n_vocab, int32_t x, float u_acc, float u_res,
                        int32_t* d_out, orc_stream_t stream);
/* One round's acceptance chain: proposal i (drawn from row i of d_q) is
 * accepted with probability min(1, p_i[x_i] / q_i[x_i]); the first rejection
 * emits a residual draw and ends the round; when all k are accepted a bonus
 * id is drawn from p_k. Uniforms come from the state's mt19937 (acceptance,
 * then the residual or bonus draw); each emitted id is recorded once.
 * d_out layout, budget and round state as orc_spec_accept_engine. Rows of up
 * to 196608 entries keep the draw's partial sums in the state's scratch:
 * calls on one state must not overlap. */
int orc_spec_accept_stochastic(void* d_state, const float* d_p, int ldp, const float* d_q, int ldq, int n_vocab,
                               const int32_t* d_x, int k, int max_emit, int32_t* d_budget, int32_t* d_out,
                               int32_t* d_pos, int32_t* d_next, orc_stream_t stream);

/* Tail of a captured greedy decode step (bench_engine.cpp:233-240 keeps the
 * chain on the host): d_tok[1] (the step's argmax) is appended at
 * d_hist[*d_count] and copied to d_tok[0] (the next input); *d_pos and
 * *d_count advance by one. The caller sizes d_hist for every step it replays. */
int orc_decode_advance(int32_t* d_tok, int32_t* d_hist, int32_t* d_pos, int32_t* d_count, orc_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif

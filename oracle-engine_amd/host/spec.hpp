// Decode loops on the device: greedy decode with the reference harness
// protocol (benchmark/bench_engine.cpp:221-243) and speculative greedy
// decode with one batched (k+1)-token verify per round
// (benchmark/bench_engine.cpp:300-356). Token ids are produced and consumed
// on the device; per round only the verify argmax ids and the accepted count
// cross to the host.
#pragma once
#include "model.hpp"

#include <cstdint>
#include <string>
#include <vector>

struct SpecStats {
    long accepted = 0, proposed = 0, passes = 0, rounds = 0;
};

// SamplerParams (core/sampler.hpp:16-22) plus the seed.
struct SamplerConfig {
    float temperature = 0.8f, top_p = 0.95f, repeat_penalty = 1.1f;
    int top_k = 40, repeat_last = 64;
    uint64_t seed = 42;
};

// Device scratch reused across calls (no allocation in the decode loops).
// With graphs on (the default), one greedy step and one speculative round
// are each captured once per (models, k) and replayed: positions and the
// next input token live on the device, so a captured graph is valid for every
// position, and the host only launches graphs and reads the round's ids.
class DecodeSession {
public:
    explicit DecodeSession(int max_tokens = 4096, int max_k = 16);
    ~DecodeSession();
    DecodeSession(const DecodeSession&) = delete;
    DecodeSession& operator=(const DecodeSession&) = delete;

    // Also drops captured graphs: the next loop captures them again (e.g.
    // after kernel timing was switched on, to include its event nodes).
    void set_graphs(bool on) {
        graphs_ = on;
        for (int i = 0; i < kBands; ++i) {
            drop(greedy_g_[i]);
            drop(spec_g_[i]);
            drop(eng_g_[i]);
            drop(smp_g_[i]);
        }
    }
    bool graphs() const { return graphs_; }
    // Message of the last error a loop reported ("" if none): a bad argument,
    // or a session whose device set-up failed (every loop then returns that
    // set-up's code).
    const char* error() const { return err_.c_str(); }
    bool usable() const { return init_rc_ == ORC_OK; }
    void clear_error() { err_.clear(); }

    // Batched prefill of prompt[0 .. n_prompt-2] into the model's KV cache.
    // ORC_E_INVALID when the prompt does not leave its last token a position
    // inside the context (n_prompt > ctx_len) or the pass failed.
    int prefill(Model& m, const int32_t* prompt, int n_prompt);
    // n_gen greedy tokens after a prefilled prompt; returns tokens written or <0.
    int greedy(Model& m, const int32_t* prompt, int n_prompt, int n_gen, int32_t* out);
    // Speculative greedy with draft length k after both models are prefilled.
    // The draft's context bounds the proposals and the target's the verify
    // width (bench_engine.cpp:313-323), so models of different context
    // lengths end a run as the reference harness does.
    int spec_greedy(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, int n_gen, int k, int32_t* out,
                    SpecStats* st);
    // The Engine's stochastic speculative loop (core/engine.cpp:100-240):
    // resets and prefills both models with prompt[0 .. n_prompt-2] (recorded
    // in the sampler history), greedy draft proposals, target samples with the
    // device sampler at every verify position, accept while equal.
    // stats: accepted, proposed, target forwards of the reference loop.
    // The draft's context may not exceed the target's (ORC_E_INVALID).
    int spec_engine(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                    const SamplerConfig& sc, int32_t* out, SpecStats* st);

    // Speculative sampling with the exact-distribution rule (no reference
    // counterpart): same reset / prefill / recorded prompt as spec_engine; the
    // draft proposes x_i ~ q_i (its logits through the sampler transform, with
    // pending proposals in the penalty window), the target scores the round in
    // one batch, proposal i is accepted with min(1, p_i/q_i), a rejection
    // emits a residual draw, a fully accepted round a bonus draw from p_k.
    // stats: accepted, proposed, target passes (one per round).
    int spec_sampled(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, int n_gen, int k,
                     const SamplerConfig& sc, int32_t* out, SpecStats* st);

private:
    int max_tokens_, max_k_;
    bool graphs_ = true;
    std::string err_;
    // set by the constructor when orc_init or a device allocation failed
    int init_rc_ = ORC_OK;
    std::string init_err_;
    int unusable() {
        err_ = init_err_;
        return init_rc_;
    }
    int invalid(const std::string& m) {
        err_ = m;
        return ORC_E_INVALID;
    }
    int32_t* d_hist_ = nullptr;  // greedy token chain
    int32_t* d_vin_ = nullptr;   // [next, d0 .. d_{k-1}]
    int32_t* d_tgt_ = nullptr;   // verify argmax ids
    int32_t* d_acc_ = nullptr;   // accepted count, next token, emitted ids
    int32_t* d_pos_ = nullptr;   // device position (+ step count for greedy)
    int32_t* d_tok_ = nullptr;   // greedy step input / output
    struct Captured {
        uint64_t a = 0, b = 0;  // model uids
        int k = -1;
        int floor = 0, lim = 0;  // floor <= every position the graph's passes reach < lim
        orc_graph_t g = nullptr, fill = nullptr;
    };
    // One graph per position band of a loop (the attention kernels a replay
    // needs depend on which side of orc_attn_wg_limit() its positions lie).
    static constexpr int kBands = 3;
    struct Band {
        int idx, floor, lim;
    };
    static Band band_of(int p_lo, int p_hi, int run_lim, int ctx);
    // the slot of band b, emptied when it holds another capture
    Captured& slot(Captured (&set)[kBands], const Band& b, uint64_t a, uint64_t bb, int k);
    Captured greedy_g_[kBands], spec_g_[kBands], eng_g_[kBands], smp_g_[kBands];
    float* d_p_ = nullptr;  // target distributions, k+1 rows
    float* d_q_ = nullptr;  // draft distributions, k rows
    size_t pq_cap_ = 0;     // floats in each of d_p_ / d_q_
    void* d_samp_ = nullptr;      // device sampler state
    int32_t* d_eout_ = nullptr;   // Engine-style acceptance output (k+5 ints)
    int32_t* d_budget_ = nullptr; // tokens still to emit
    void drop(Captured& c);
    int begin_sampled(Model& tgt, Model& dft, const int32_t* prompt, int n_prompt, const SamplerConfig& sc,
                      std::vector<int32_t>& ids);
    int sampled_round(Model& tgt, Model& dft, int k, int V);
    int greedy_graphed(Model& m, int pos, int32_t first, int n_gen, int32_t* out);
    int spec_rounds(Model& tgt, Model& dft, int pos, int32_t next, int n_gen, int k, int32_t* out, SpecStats& S);
};

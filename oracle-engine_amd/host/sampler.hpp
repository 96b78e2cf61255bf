// Sampler — the reference's token sampler (core/sampler.hpp:16-48) with its
// state in device memory: the mt19937 generator, the parameters and the
// history live in one orc_sampler state, and sample() runs the device
// sampler (orc_sample: penalty, temperature, softmax, top-k, top-p, draw,
// record) on a copy of the host logits, then writes the rewritten row back
// (the reference's sample leaves the probabilities in the caller's array).
// The device loops take the same state through device_state().
#pragma once
#include <cstdint>
#include <string>

struct SamplerParams {  // core/sampler.hpp:16-22
    float temperature = 0.7f;
    float top_p = 0.9f;
    int top_k = 40;
    float repeat_pen = 1.1f;
    int repeat_last = 64;
};

class Sampler {
public:
    // core/sampler.hpp:26; the seed is truncated to 32 bits as std::mt19937's
    // constructor does with the reference's 64-bit seed. The device history
    // holds 4096 ids: repeat_last must be below 4096 (the reference takes any
    // value); a larger one, or a failed device set-up, is reported here
    // through error() (and stderr), and sample() then returns -1.
    explicit Sampler(const SamplerParams& p = {}, uint64_t seed = 42);
    ~Sampler();
    Sampler(const Sampler&) = delete;
    Sampler& operator=(const Sampler&) = delete;
    Sampler(Sampler&& o) noexcept;
    Sampler& operator=(Sampler&& o) noexcept;

    // core/sampler.hpp:29-30: next token from n_vocab logits (rewritten in
    // place), recorded in the history. -1 if the device call failed (error()).
    int32_t sample(float* logits, int n_vocab);
    // core/sampler.hpp:32
    void record(int32_t token_id);
    // core/sampler.hpp:34: history cleared, generator kept
    void reset();
    // core/sampler.hpp:37: parameters replaced, generator and history kept
    void set_params(const SamplerParams& p);

    const SamplerParams& params() const { return p_; }
    void* device_state() const { return d_state_; }
    const std::string& error() const { return err_; }

private:
    SamplerParams p_;
    void* d_state_ = nullptr;
    float* d_logits_ = nullptr;
    int32_t* d_id_ = nullptr;
    int cap_ = 0;
    std::string err_;

    bool fail(const char* what);
    void release();
};

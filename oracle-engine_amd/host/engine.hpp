// Engine — the reference's chat front end (core/engine.hpp:10-76) over the
// device path: load a model (+ tokenizer from its GGUF), optionally a draft,
// and generate a reply to a conversation with streaming.
//
// generate keeps the reference's behaviour (core/engine.cpp:83-243): the
// Llama-3 / ChatML prompt template, the tokenized prompt with BOS, the
// "prompt too long" refusal (ctx - 4), a fresh KV cache, the batched prefill
// of all but the last prompt id (recorded in the sampler history), SamplerParams
// {temperature, top_p, top_k 40, repeat_penalty, repeat_last_n}, the EOS id
// (<|im_end|> for qwen*, else <|eot_id|>, each falling back to the other), and
// on_token called with each emitted piece in order. Without a draft every step
// runs on the device (forward, sampler, next id) and only the id crosses to
// the host for the EOS test and the piece. With a draft the speculative loop
// runs on the device in one call (DecodeSession::spec_engine: greedy draft
// proposals, target samples at every verify position) and the emitted ids are
// then cut at the first EOS and streamed: the same pieces, delivered after
// the loop. The seed is the steady clock's, as the reference's, unless
// set_seed fixes it (no reference counterpart; for reproducible runs).
#pragma once
#include "model.hpp"
#include "spec.hpp"
#include "tokenizer.hpp"

#include <cstdint>
#include <functional>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

static constexpr const char* ORACLE_DEFAULT_MODEL = "models/qwen2.5-7b-instruct-q4km.gguf";  // core/engine.hpp:11-12
static constexpr const char* ORACLE_DEFAULT_DRAFT = "models/llama-3.2-3b-q4k.gguf";         // core/engine.hpp:15-16

struct Message {  // core/engine.hpp:20-23
    std::string role;  // "system" | "user" | "assistant"
    std::string content;
};
using ChatMessage = Message;

struct GenParams {  // core/engine.hpp:26-33
    int n_predict = 256;
    float temperature = 0.7f;
    float top_p = 0.9f;
    float repeat_penalty = 1.15f;
    int repeat_last_n = 64;
    int n_gpu_layers = 0;  // ignored: every layer runs on the GPU
};

class Engine {
public:
    Engine() = default;
    ~Engine();

    bool load(const std::string& model_path, const GenParams& params = {});
    std::string generate(const std::vector<Message>& messages, const GenParams& params = {},
                         std::function<void(const std::string&)> on_token = nullptr);
    std::vector<float> embed(const std::string& text);
    bool load_draft(const std::string& draft_path);
    bool has_draft() const { return draft_loaded_; }

    bool is_loaded() const { return model_.is_loaded(); }
    std::string model_path() const { return model_path_; }
    Tokenizer& tokenizer() { return tok_; }

    // Fixed sampler seed for the following generate calls (the reference
    // seeds from the clock on every call).
    void set_seed(uint64_t seed) {
        seed_ = seed;
        fixed_seed_ = true;
    }
    // Why the last call failed or stopped early ("" if it did not).
    const std::string& last_error() const { return err_; }

private:
    std::string model_path_;
    Model model_;
    Tokenizer tok_;
    std::mutex mtx_;
    Model draft_model_;
    Tokenizer draft_tok_;
    bool draft_loaded_ = false;
    static constexpr int SPEC_N = 4;  // draft proposals per round (core/engine.hpp:72)
    std::unique_ptr<DecodeSession> sess_;
    void* d_samp_ = nullptr;  // device sampler state
    int32_t* d_ids_ = nullptr;
    size_t ids_cap_ = 0;
    bool fixed_seed_ = false;
    uint64_t seed_ = 0;
    std::string err_;

    std::string format_prompt(const std::vector<Message>& messages) const;
    bool ensure_ids(size_t n);
};

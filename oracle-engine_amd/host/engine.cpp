// Engine on the device path (see engine.hpp).
#include "engine.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>

Engine::~Engine() {
    if (d_samp_) orc_free(d_samp_);
    if (d_ids_) orc_free(d_ids_);
}

bool Engine::load(const std::string& path, const GenParams&) {  // core/engine.cpp:8-27
    if (!model_.load(path)) {
        err_ = std::string("model load failed: ") + model_.last_error();
        return false;
    }
    if (!tok_.load(model_.gguf())) {
        err_ = "the GGUF has no tokenizer";
        return false;
    }
    model_path_ = path;
    model_.warmup();
    return true;
}

bool Engine::load_draft(const std::string& path) {  // core/engine.cpp:29-44
    if (!draft_model_.load(path)) {
        err_ = std::string("draft load failed: ") + draft_model_.last_error();
        return false;
    }
    if (!draft_tok_.load(draft_model_.gguf())) {
        err_ = "the draft GGUF has no tokenizer";
        return false;
    }
    draft_model_.warmup();
    draft_loaded_ = true;
    return true;
}

std::vector<float> Engine::embed(const std::string& text) {  // core/engine.cpp:46-53
    std::lock_guard<std::mutex> lk(mtx_);
    if (!model_.is_loaded()) return {};
    auto ids = tok_.encode(text, true);
    if (ids.empty()) return {};
    if (ids.size() > 512) ids.resize(512);
    return model_.embed_tokens(ids);
}

std::string Engine::format_prompt(const std::vector<Message>& msgs) const {  // core/engine.cpp:55-81
    const std::string arch = model_.gguf().meta_str("general.architecture", "llama");
    const bool qwen = arch.compare(0, 4, "qwen") == 0;
    const bool has_system = std::any_of(msgs.begin(), msgs.end(), [](const Message& m) { return m.role == "system"; });
    const std::string sys_default = "Tu es un assistant utile.";
    std::string p;
    if (qwen) {  // ChatML
        if (!has_system) p += "<|im_start|>system\n" + sys_default + "<|im_end|>\n";
        for (const auto& m : msgs) p += "<|im_start|>" + m.role + "\n" + m.content + "<|im_end|>\n";
        p += "<|im_start|>assistant\n";
    } else {  // Llama 3 instruct
        p += "<|begin_of_text|>";
        if (!has_system) p += "<|start_header_id|>system<|end_header_id|>\n\n" + sys_default + "<|eot_id|>";
        for (const auto& m : msgs)
            p += "<|start_header_id|>" + m.role + "<|end_header_id|>\n\n" + m.content + "<|eot_id|>";
        p += "<|start_header_id|>assistant<|end_header_id|>\n\n";
    }
    return p;
}

bool Engine::ensure_ids(size_t n) {
    if (n <= ids_cap_) return true;
    if (d_ids_) orc_free(d_ids_);
    d_ids_ = nullptr;
    ids_cap_ = 0;
    if (orc_malloc((void**)&d_ids_, n * 4) != ORC_OK) return false;
    ids_cap_ = n;
    return true;
}

std::string Engine::generate(const std::vector<Message>& messages, const GenParams& gp,
                             std::function<void(const std::string&)> on_token) {  // core/engine.cpp:83-243
    std::lock_guard<std::mutex> lk(mtx_);
    err_.clear();
    if (!model_.is_loaded()) return "";
    const std::vector<int32_t> ids = tok_.encode(format_prompt(messages), true);
    const int max_ctx = (int)model_.cfg.ctx_len;
    if ((int)ids.size() >= max_ctx - 4) {
        err_ = "prompt too long for the context";
        return "";
    }
    SamplerConfig sc;
    sc.temperature = gp.temperature;
    sc.top_p = gp.top_p;
    sc.top_k = 40;  // core/engine.cpp:106
    sc.repeat_penalty = gp.repeat_penalty;
    sc.repeat_last = gp.repeat_last_n;
    sc.seed = fixed_seed_ ? seed_ : (uint64_t)std::chrono::steady_clock::now().time_since_epoch().count();
    const std::string arch = model_.gguf().meta_str("general.architecture", "llama");
    const bool qwen = arch.size() >= 4 && arch.compare(0, 4, "qwen") == 0;
    int32_t eos = tok_.special_id(qwen ? "<|im_end|>" : "<|eot_id|>");
    if (eos < 0) eos = tok_.special_id(qwen ? "<|eot_id|>" : "<|im_end|>");
    std::string resp;
    auto emit = [&](int32_t id) {
        const std::string piece = tok_.decode_one(id);
        resp += piece;
        if (on_token) on_token(piece);
    };
    const int n = (int)ids.size();

    if (draft_loaded_) {
        // the device loop resets and prefills both models and records the
        // prompt; then the ids up to the first EOS are streamed
        if (!sess_) sess_ = std::make_unique<DecodeSession>(std::max(4096, gp.n_predict + 64), 16);
        std::vector<int32_t> out((size_t)std::max(0, gp.n_predict) + SPEC_N + 2);
        SpecStats st;
        const int got = sess_->spec_engine(model_, draft_model_, ids.data(), n, std::max(0, gp.n_predict), SPEC_N,
                                           sc, out.data(), &st);
        if (got < 0) {
            err_ = std::string("speculative loop: ") + (sess_->error()[0] ? sess_->error() : orc_last_error());
            return resp;
        }
        for (int i = 0; i < got; ++i) {
            if (eos >= 0 && out[i] == eos) break;
            emit(out[i]);
        }
        return resp;
    }

    model_.reset();
    if (!d_samp_ && orc_malloc(&d_samp_, orc_sampler_state_bytes()) != ORC_OK) {
        err_ = orc_last_error();
        return "";
    }
    const int n_prefill = n - 1;
    if (!ensure_ids((size_t)std::max(n, 1)) || orc_memcpy_h2d(d_ids_, ids.data(), (size_t)n * 4, nullptr) ||
        orc_sampler_init(d_samp_, sc.temperature, sc.top_p, sc.top_k, sc.repeat_penalty, sc.repeat_last, sc.seed,
                         d_ids_, n_prefill, nullptr)) {
        err_ = orc_last_error();
        return "";
    }
    int pos = 0;
    if (n_prefill > 0) {
        model_.forward_prefill(ids.data(), n_prefill, 0);
        if (model_.last_error()[0]) {
            err_ = model_.last_error();
            return "";
        }
        pos = n_prefill;
    }
    // the step's input id lives in d_ids_[0]: the last prompt id, then each sampled id
    int32_t* d_tok = d_ids_;
    if (orc_memcpy_h2d(d_tok, &ids.back(), 4, nullptr)) {
        err_ = orc_last_error();
        return "";
    }
    for (int step = 0; step < gp.n_predict && pos < max_ctx - 1; ++step) {
        int32_t next = 0;
        if (model_.forward_dev(d_tok, 1, pos, true, nullptr) ||
            orc_sample(d_samp_, model_.d_logits(), (int)model_.cfg.n_vocab, d_tok, nullptr) ||
            orc_memcpy_d2h(&next, d_tok, 4, nullptr)) {
            err_ = model_.last_error()[0] ? model_.last_error() : orc_last_error();
            break;
        }
        ++pos;
        if (eos >= 0 && next == eos) break;
        emit(next);
    }
    return resp;
}

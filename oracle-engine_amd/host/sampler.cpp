// Sampler on a device state (see sampler.hpp).
#include "sampler.hpp"

#include "orc.h"

#include <cstdio>
#include <utility>

Sampler::Sampler(const SamplerParams& p, uint64_t seed) : p_(p) {  // sampler.cpp:7-8
    if (orc_init(0) != ORC_OK || orc_malloc(&d_state_, orc_sampler_state_bytes()) != ORC_OK ||
        orc_malloc((void**)&d_id_, 256) != ORC_OK) {
        fail("allocation");
        return;
    }
    if (orc_sampler_init(d_state_, p.temperature, p.top_p, p.top_k, p.repeat_pen, p.repeat_last, seed, nullptr, 0,
                         nullptr) != ORC_OK) {
        // e.g. repeat_last >= 4096: reported here (error()), and the sampler
        // is left without a state, so sample() returns -1 and record() does nothing
        fail("init");
        release();
    }
}

Sampler::~Sampler() { release(); }

void Sampler::release() {
    for (void* q : {d_state_, (void*)d_logits_, (void*)d_id_})
        if (q) orc_free(q);
    d_state_ = nullptr;
    d_logits_ = nullptr;
    d_id_ = nullptr;
    cap_ = 0;
}

Sampler::Sampler(Sampler&& o) noexcept { *this = std::move(o); }

Sampler& Sampler::operator=(Sampler&& o) noexcept {
    if (this != &o) {
        release();
        p_ = o.p_;
        d_state_ = std::exchange(o.d_state_, nullptr);
        d_logits_ = std::exchange(o.d_logits_, nullptr);
        d_id_ = std::exchange(o.d_id_, nullptr);
        cap_ = std::exchange(o.cap_, 0);
        err_ = std::move(o.err_);
    }
    return *this;
}

bool Sampler::fail(const char* what) {
    err_ = std::string("Sampler ") + what + ": " + orc_last_error();
    std::fprintf(stderr, "[Sampler] %s\n", err_.c_str());
    return false;
}

int32_t Sampler::sample(float* logits, int n_vocab) {  // sampler.cpp:91-97
    if (!d_state_ || n_vocab <= 0) return -1;
    if (n_vocab > cap_) {
        if (d_logits_) orc_free(d_logits_);
        d_logits_ = nullptr;
        cap_ = 0;
        if (orc_malloc((void**)&d_logits_, (size_t)n_vocab * 4) != ORC_OK) return fail("allocation"), -1;
        cap_ = n_vocab;
    }
    int32_t id = -1;
    if (orc_memcpy_h2d(d_logits_, logits, (size_t)n_vocab * 4, nullptr) != ORC_OK ||
        orc_sample(d_state_, d_logits_, n_vocab, d_id_, nullptr) != ORC_OK ||
        orc_memcpy_d2h(logits, d_logits_, (size_t)n_vocab * 4, nullptr) != ORC_OK ||
        orc_memcpy_d2h(&id, d_id_, 4, nullptr) != ORC_OK)
        return fail("sample"), -1;
    return id;
}

void Sampler::record(int32_t token_id) {  // sampler.cpp:99-105
    if (!d_state_) return;
    if (orc_memcpy_h2d(d_id_, &token_id, 4, nullptr) != ORC_OK ||
        orc_sampler_record(d_state_, d_id_, 1, nullptr) != ORC_OK ||
        orc_stream_sync(nullptr) != ORC_OK)
        fail("record");
}

void Sampler::reset() {
    if (d_state_ && (orc_sampler_clear_history(d_state_, nullptr) != ORC_OK || orc_stream_sync(nullptr) != ORC_OK))
        fail("reset");
}

void Sampler::set_params(const SamplerParams& p) {
    p_ = p;
    if (d_state_ && (orc_sampler_set_params(d_state_, p.temperature, p.top_p, p.top_k, p.repeat_pen, p.repeat_last,
                                            nullptr) != ORC_OK ||
                     orc_stream_sync(nullptr) != ORC_OK))
        fail("set_params");
}

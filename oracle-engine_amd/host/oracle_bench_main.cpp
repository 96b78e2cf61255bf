// oracle_bench — drop-in for the reference harness (benchmark/bench_engine.cpp)
// on the MI355X path. Same protocol: batched prefill of n_prompt-1 tokens
// (untimed), greedy generation of n_gen tokens timed over R runs with the
// first discarded, median reported, FNV-1a checksum of the generated ids; with
// --draft, speculative greedy decoding with a (k+1)-token batched verify and
// the "exact output" check (spec checksum == greedy checksum).
//
// The synthetic models carry no tokenizer, so the prompt is uniform random
// token ids from --seed (or raw int32 ids from --prompt-file) instead of the
// reference's tiled English prompt (bench_engine.cpp:194-201).
#include "model.hpp"
#include "spec.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <string>
#include <vector>

namespace {
struct Args {
    std::string model, draft, json, prompt_file;
    int n_prompt = 128, n_gen = 128, runs = 5, spec_n = 4, ctx = 0;
    uint64_t seed = 1234;
};

void usage(const char* exe) {
    std::fprintf(stderr,
                 "usage: %s -m <model.gguf> [-p N] [-g N] [-r N] [--draft <gguf>] [--spec-n K] [--ctx N]\n"
                 "          [--seed S | --prompt-file ids.bin] [--json out.json]\n",
                 exe);
}

bool parse(int argc, char** argv, Args& a) {
    for (int i = 1; i < argc; ++i) {
        std::string k = argv[i];
        auto nx = [&]() -> const char* { return i + 1 < argc ? argv[++i] : nullptr; };
        const char* v = nullptr;
        if (k == "-h" || k == "--help") return false;
        if (!(v = nx())) { std::fprintf(stderr, "missing value after %s\n", k.c_str()); return false; }
        if (k == "-m") a.model = v;
        else if (k == "-p") a.n_prompt = std::atoi(v);
        else if (k == "-g") a.n_gen = std::atoi(v);
        else if (k == "-r") a.runs = std::atoi(v);
        else if (k == "-t") {}  // thread count: meaningless on the GPU path, accepted for compatibility
        else if (k == "--draft") a.draft = v;
        else if (k == "--spec-n") a.spec_n = std::atoi(v);
        else if (k == "--ctx") a.ctx = std::atoi(v);
        else if (k == "--seed") a.seed = std::strtoull(v, nullptr, 10);
        else if (k == "--prompt-file") a.prompt_file = v;
        else if (k == "--json") a.json = v;
        else { std::fprintf(stderr, "unknown option %s\n", k.c_str()); return false; }
    }
    if (a.model.empty()) return false;
    a.n_prompt = std::max(a.n_prompt, 2);
    a.n_gen = std::max(a.n_gen, 1);
    a.runs = std::max(a.runs, 1);
    a.spec_n = std::min(std::max(a.spec_n, 1), 16);
    return true;
}

double median(std::vector<double> v) {
    std::sort(v.begin(), v.end());
    const size_t n = v.size();
    return n == 0 ? 0.0 : (n & 1) ? v[n / 2] : 0.5 * (v[n / 2 - 1] + v[n / 2]);
}

uint64_t fnv(const std::vector<int32_t>& t) {
    uint64_t h = 1469598103934665603ULL;
    for (int32_t x : t) h = (h ^ (uint64_t)(uint32_t)x) * 1099511628211ULL;
    return h;
}
}  // namespace

int main(int argc, char** argv) {
    Args a;
    if (!parse(argc, argv, a)) { usage(argv[0]); return 2; }
    const int ctx = a.ctx > 0 ? a.ctx : std::max(512, a.n_prompt + a.n_gen + a.spec_n + 2);
    Model model;
    if (!model.load(a.model, ctx)) { std::fprintf(stderr, "error: cannot load %s\n", a.model.c_str()); return 1; }
    const ModelConfig& c = model.cfg;
    std::vector<int32_t> prompt;
    if (!a.prompt_file.empty()) {
        FILE* f = std::fopen(a.prompt_file.c_str(), "rb");
        if (!f) { std::fprintf(stderr, "error: cannot read %s\n", a.prompt_file.c_str()); return 1; }
        int32_t v;
        while (std::fread(&v, 4, 1, f) == 1) prompt.push_back(v);
        std::fclose(f);
        a.n_prompt = (int)prompt.size();
    } else {
        std::mt19937_64 rng(a.seed);
        std::uniform_int_distribution<int32_t> u(0, (int32_t)c.n_vocab - 1);
        for (int i = 0; i < a.n_prompt; ++i) prompt.push_back(u(rng));
    }
    char dev[256] = {0};
    int n_cu = 0;
    size_t hbm = 0;
    orc_device_info(dev, sizeof dev, &n_cu, &hbm);
    std::printf("ORACLE on %s, %d CUs, %.0f GB HBM\n", dev, n_cu, hbm / 1e9);
    std::printf("model   : %s\nconfig  : %u layers, %u/%u q/kv heads, embed=%u, ffn=%u, vocab=%u, ctx=%u\n",
                a.model.c_str(), c.n_layers, c.n_heads, c.n_kv_heads, c.embed_dim, c.ffn_hidden, c.n_vocab, c.ctx_len);
    std::printf("prefill : %d tokens | generation: %d tokens | runs: %d (1 discarded)\n", a.n_prompt - 1, a.n_gen,
                a.runs);
    model.warmup();
    DecodeSession sess(std::max(4096, a.n_gen + 8), 16);
    std::vector<double> pf, gen;
    std::vector<int32_t> toks(a.n_gen);
    uint64_t csum = 0;
    for (int r = 0; r < a.runs; ++r) {
        model.reset();
        auto t0 = std::chrono::steady_clock::now();
        sess.prefill(model, prompt.data(), a.n_prompt);
        auto t1 = std::chrono::steady_clock::now();
        int n = sess.greedy(model, prompt.data(), a.n_prompt, a.n_gen, toks.data());
        auto t2 = std::chrono::steady_clock::now();
        if (n != a.n_gen) { std::fprintf(stderr, "error: generation failed: %s\n", orc_last_error()); return 1; }
        const double dp = std::chrono::duration<double>(t1 - t0).count();
        const double dg = std::chrono::duration<double>(t2 - t1).count();
        const bool warm = r == 0 && a.runs > 1;
        std::printf("  run %d/%d%s: prefill %.1f tok/s | gen %.1f tok/s (%.4f s)\n", r + 1, a.runs,
                    warm ? " [warmup]" : "", (a.n_prompt - 1) / dp, a.n_gen / dg, dg);
        if (!warm) {
            pf.push_back((a.n_prompt - 1) / dp);
            gen.push_back(a.n_gen / dg);
            csum = fnv(toks);
        }
    }
    const double g_med = median(gen);
    std::printf("RESULTS (median of %zu runs)\n  prefill    : %.1f tok/s\n  generation : %.1f tok/s\n"
                "  checksum   : %016llx\n",
                gen.size(), median(pf), g_med, (unsigned long long)csum);
    double spec_tps = 0, acc_rate = 0;
    uint64_t spec_csum = 0;
    bool exact = false;
    SpecStats spec_st;  // counts of the measured speculative run
    int spec_n_tok = 0;
    if (!a.draft.empty()) {
        Model draft;
        if (!draft.load(a.draft, ctx)) { std::fprintf(stderr, "error: cannot load draft\n"); return 1; }
        if (draft.cfg.n_vocab != c.n_vocab) { std::fprintf(stderr, "error: draft vocab differs\n"); return 1; }
        draft.warmup();
        SpecStats st;
        std::vector<int32_t> st_toks(a.n_gen + a.spec_n + 2);
        for (int r = 0; r < 2; ++r) {  // run 0 warmup, run 1 measured (bench_engine.cpp:300)
            model.reset();
            draft.reset();
            sess.prefill(model, prompt.data(), a.n_prompt);
            sess.prefill(draft, prompt.data(), a.n_prompt);
            st = SpecStats{};
            auto t0 = std::chrono::steady_clock::now();
            int n = sess.spec_greedy(model, draft, prompt.data(), a.n_prompt, a.n_gen, a.spec_n, st_toks.data(), &st);
            const double dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            if (n < 0) { std::fprintf(stderr, "error: spec decode failed: %s\n", orc_last_error()); return 1; }
            st_toks.resize(n);
            spec_tps = n / dt;
        }
        spec_csum = fnv(st_toks);
        exact = spec_csum == csum;
        spec_st = st;
        spec_n_tok = (int)st_toks.size();
        acc_rate = st.proposed ? 100.0 * st.accepted / st.proposed : 0.0;
        std::printf("speculative (k=%d): %.1f tok/s (x%.2f vs greedy)\n  acceptance : %.1f%% (%ld/%ld)\n"
                    "  passes/tok : %.2f\n  exact      : %s (spec %016llx vs greedy %016llx)\n",
                    a.spec_n, spec_tps, g_med > 0 ? spec_tps / g_med : 0.0, acc_rate, st.accepted, st.proposed,
                    st_toks.empty() ? 0.0 : (double)st.passes / st_toks.size(), exact ? "YES" : "NO (BUG)",
                    (unsigned long long)spec_csum, (unsigned long long)csum);
    }
    if (!a.json.empty()) {
        FILE* f = std::fopen(a.json.c_str(), "w");
        if (f) {
            std::fprintf(f,
                         "{\"engine\": \"ORACLE-mi355x\", \"model\": \"%s\", \"prompt_tokens\": %d, \"gen_tokens\": %d, "
                         "\"generation_tok_s\": %.3f, \"prefill_tok_s\": %.3f, \"gen_checksum\": \"%016llx\", "
                         "\"spec_tok_s\": %.3f, \"acceptance_pct\": %.3f, \"spec_exact\": %s, "
                         "\"spec_checksum\": \"%016llx\", \"accepted\": %ld, \"proposed\": %ld, \"passes\": %ld, "
                         "\"spec_tokens\": %d}\n",
                         a.model.c_str(), a.n_prompt - 1, a.n_gen, g_med, median(pf), (unsigned long long)csum, spec_tps,
                         acc_rate, exact ? "true" : "false", (unsigned long long)spec_csum, spec_st.accepted,
                         spec_st.proposed, spec_st.passes, spec_n_tok);
            std::fclose(f);
        }
    }
    return 0;
}

// ref_driver — runs the REFERENCE implementation (compiled from the sources
// under /root/reference by oracle/Makefile) on given inputs and writes its
// outputs as raw little-endian files. It is test infrastructure only: it
// produces the golden vectors under tests/golden/ and the reference CPU
// baseline timed by bench.py. It calls only the reference's public API
// (GGUFParser, Model, Sampler, ops); the decode / spec loops below restate the
// reference harness protocol (benchmark/bench_engine.cpp:221-263, 300-363) and
// the Engine's stochastic spec loop (core/engine.cpp:150-240) with a fixed seed.
#include "core/engine.hpp"
#include "core/gguf_parser.hpp"
#include "core/model.hpp"
#include "core/tokenizer.hpp"
#include "core/ops.hpp"
#include "core/sampler.hpp"

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

template <typename T>
static std::vector<T> read_bin(const char* path) {
    std::vector<T> v;
    FILE* f = std::fopen(path, "rb");
    if (!f) { std::fprintf(stderr, "cannot open %s\n", path); std::exit(3); }
    std::fseek(f, 0, SEEK_END);
    long n = std::ftell(f);
    std::fseek(f, 0, SEEK_SET);
    v.resize((size_t)n / sizeof(T));
    if (n && std::fread(v.data(), sizeof(T), v.size(), f) != v.size()) std::exit(3);
    std::fclose(f);
    return v;
}
template <typename T>
static void write_bin(const char* path, const T* p, size_t n) {
    FILE* f = std::fopen(path, "wb");
    if (!f || (n && std::fwrite(p, sizeof(T), n, f) != n)) { std::fprintf(stderr, "cannot write %s\n", path); std::exit(3); }
    std::fclose(f);
}

static int32_t argmax_first(const float* v, int n) {
    int32_t best = 0;
    float bv = v[0];
    for (int i = 1; i < n; i++)
        if (v[i] > bv) { bv = v[i]; best = i; }
    return best;
}

static uint64_t fnv_step(uint64_t h, int32_t tok) { return (h ^ (uint64_t)(uint32_t)tok) * 1099511628211ULL; }

static bool load_model(Model& m, const char* path) {
    if (!m.load(path)) { std::fprintf(stderr, "model load failed: %s\n", path); return false; }
    return true;
}

// Greedy decode after a batched prefill of n-1 prompt tokens (bench protocol).
static std::vector<int32_t> greedy(Model& m, const std::vector<int32_t>& prompt, int n_gen,
                                   std::vector<float>* logits_out, int n_logit_steps) {
    m.reset();
    const int np = (int)prompt.size() - 1;
    m.forward_prefill(prompt.data(), np, 0);
    int32_t cur = prompt[np];
    int pos = np;
    std::vector<int32_t> out;
    const int V = (int)m.cfg.n_vocab;
    for (int s = 0; s < n_gen; s++) {
        const float* lg = m.forward(cur, pos++);
        if (logits_out && s < n_logit_steps) logits_out->insert(logits_out->end(), lg, lg + V);
        cur = argmax_first(lg, V);
        out.push_back(cur);
    }
    return out;
}

struct SpecStats { long acc = 0, prop = 0, passes = 0; };

// Speculative greedy decode with one batched (k+1)-token verify per round.
static std::vector<int32_t> spec_greedy(Model& tgt, Model& dft, const std::vector<int32_t>& prompt, int n_gen,
                                        int k, SpecStats& st, bool prefill = true) {
    const int np = (int)prompt.size() - 1;
    if (prefill) {
        tgt.reset(); dft.reset();
        tgt.forward_prefill(prompt.data(), np, 0);
        dft.forward_prefill(prompt.data(), np, 0);
    }
    const int V = (int)tgt.cfg.n_vocab;
    const int max_ctx = (int)tgt.cfg.ctx_len;
    std::vector<float> blog((size_t)(k + 1) * V);
    std::vector<int32_t> out;
    int pos = np;
    int32_t next = prompt[np];
    while ((int)out.size() < n_gen && pos < max_ctx - 1) {
        int32_t dtok[64];
        int ndt = 0;
        int dp = pos;
        int32_t dt = next;
        for (int i = 0; i < k && dp < (int)dft.cfg.ctx_len - 1; i++) {
            const float* dl = dft.forward(dt, dp++);
            dtok[ndt++] = dt = argmax_first(dl, (int)dft.cfg.n_vocab);
        }
        if (ndt == 0) break;
        st.prop += ndt;
        int nver = ndt + 1;
        if (pos + nver > max_ctx) nver = max_ctx - pos;
        int32_t vin[65];
        vin[0] = next;
        for (int i = 0; i < nver - 1; i++) vin[i + 1] = dtok[i];
        tgt.forward_batch(vin, nver, pos, blog.data());
        st.passes++;
        int a = 0;
        bool brk = false;
        for (int i = 0; i < ndt && i < nver; i++) {
            int32_t mt = argmax_first(blog.data() + (size_t)i * V, V);
            out.push_back(mt);
            if (mt != dtok[i]) { next = mt; a = i; brk = true; break; }
            st.acc++; a = i + 1; next = dtok[i];
            if ((int)out.size() >= n_gen) { brk = true; break; }
        }
        pos += a + 1;
        if (brk) continue;
        if ((int)out.size() < n_gen && ndt < nver && pos < max_ctx - 1) {
            next = argmax_first(blog.data() + (size_t)ndt * V, V);
            out.push_back(next);
            dft.forward(dtok[ndt - 1], pos - 1, false);
        }
    }
    return out;
}

// Engine-style speculative sampling: greedy draft proposals, one sequential
// target forward + Sampler::sample per proposal, accept iff the sampled token
// equals the proposal, every verified token recorded twice, bonus token when
// all are accepted. Prompt tokens except the last are recorded first.
static std::vector<int32_t> spec_engine(Model& tgt, Model& dft, const std::vector<int32_t>& ids, int n_predict,
                                        int k, const SamplerParams& sp, uint64_t seed, SpecStats& st) {
    tgt.reset(); dft.reset();
    Sampler sampler(sp, seed);
    const int max_ctx = (int)tgt.cfg.ctx_len;
    const int V = (int)tgt.cfg.n_vocab;
    std::vector<float> lb(V);
    int pos = 0;
    const int n_prefill = (int)ids.size() - 1;
    if (n_prefill > 0) {
        tgt.forward_prefill(ids.data(), n_prefill, 0);
        for (int i = 0; i < n_prefill; i++) sampler.record(ids[i]);
        pos = n_prefill;
        dft.forward_prefill(ids.data(), n_prefill, 0);
    }
    int32_t next = ids.back();
    std::vector<int32_t> out;
    for (int step = 0; step < n_predict && pos < max_ctx - 1;) {
        std::vector<int32_t> dts;
        int dp = pos;
        int32_t dt = next;
        for (int i = 0; i < k && dp < (int)dft.cfg.ctx_len - 1; i++) {
            const float* dl = dft.forward(dt, dp++);
            dts.push_back(dt = argmax_first(dl, (int)dft.cfg.n_vocab));
        }
        if (dts.empty()) break;
        st.prop += (long)dts.size();
        bool done = false;
        int accepted = 0;
        int32_t verify = next;
        for (size_t i = 0; i < dts.size(); i++) {
            if (pos >= max_ctx - 1) { done = true; break; }
            const float* lg = tgt.forward(verify, pos++);
            st.passes++;
            std::memcpy(lb.data(), lg, V * sizeof(float));
            int32_t mt = sampler.sample(lb.data(), V);
            sampler.record(mt);
            if (mt != dts[i]) { next = mt; out.push_back(next); step++; break; }
            next = dts[i];
            accepted++; st.acc++;
            out.push_back(next);
            step++;
            if (step >= n_predict) { done = true; break; }
            verify = next;
        }
        if (done) break;
        if (accepted == (int)dts.size() && pos < max_ctx - 1) {
            const float* lg = tgt.forward(next, pos++);
            st.passes++;
            std::memcpy(lb.data(), lg, V * sizeof(float));
            next = sampler.sample(lb.data(), V);
            sampler.record(next);
            out.push_back(next);
            step++;
            dft.forward(dts.back(), pos - 1, false);
        }
    }
    return out;
}

static int usage() {
    std::fprintf(stderr,
        "ref_driver cfg <model>\n"
        "ref_driver dqhook <q4_0|q4_k|q6_k> <in.bin> <n_el> <out.bin>\n"
        "ref_driver dqrow <model> <tensor> <row0> <nrows> <out.bin>\n"
        "ref_driver gemv <model> <tensor> <x.bin> <out.bin>\n"
        "ref_driver gemm <model> <tensor> <X.bin> <ntok> <out.bin>\n"
        "ref_driver greedy <model> <prompt.bin> <n_gen> <tokens.bin> [<logits.bin> <n_steps>]\n"
        "ref_driver batch <model> <tokens.bin> <n_prefill> <n_batch> <logits.bin>\n"
        "ref_driver spec <target> <draft> <prompt.bin> <n_gen> <k> <tokens.bin> [<target_ctx> <draft_ctx>]\n"
        "ref_driver espec <target> <draft> <prompt.bin> <n_gen> <k> <temp> <top_p> <top_k> <pen> <last> <seed> <tokens.bin>\n"
        "ref_driver sample <logits.bin> <temp> <top_p> <top_k> <pen> <last> <seed> <history.bin> <n_draws> <out.bin>\n"
        "ref_driver op <rmsnorm|softmax|silu|rope|argmax|dot> ...\n"
        "ref_driver bench <model> <draft|-> <prompt.bin> <n_gen> <k> <threads>\n"
        "ref_driver embed <model> <tokens.bin> <out.bin>\n"
        "ref_driver orkv <model> <prompt.bin> <state.orkv> <logits.bin>\n"
        "ref_driver tokenize <model> <text.bin> <add_bos> <ids.bin>\n"
        "ref_driver detok <model> <ids.bin> <pieces.bin>\n"
        "ref_driver engine <model> <draft|-> <n_predict> <temp> <messages.bin> <pieces.bin>\n");
    return 2;
}

int main(int argc, char** argv) {
    if (argc < 2) return usage();
    const std::string cmd = argv[1];
    if (cmd == "cfg" && argc == 3) {
        Model m;
        if (!load_model(m, argv[2])) return 1;
        const auto& c = m.cfg;
        std::printf("{\"n_vocab\": %u, \"n_layers\": %u, \"n_heads\": %u, \"n_kv_heads\": %u, \"embed_dim\": %u, "
                    "\"ffn_hidden\": %u, \"head_dim\": %u, \"ctx_len\": %u, \"rope_freq\": %.9g, \"rms_eps\": %.9g, "
                    "\"qk_norm\": %d}\n",
                    c.n_vocab, c.n_layers, c.n_heads, c.n_kv_heads, c.embed_dim, c.ffn_hidden, c.head_dim, c.ctx_len,
                    (double)c.rope_freq, (double)c.rms_eps, (int)c.qk_norm);
        return 0;
    }
    if (cmd == "dqhook" && argc == 6) {
        auto in = read_bin<uint8_t>(argv[3]);
        uint64_t n = std::strtoull(argv[4], nullptr, 10);
        std::vector<float> out(n);
        std::string t = argv[2];
        if (t == "q4_0") GGUFParser::test_dq_q4_0(in.data(), n, out.data());
        else if (t == "q4_k") GGUFParser::test_dq_q4_k(in.data(), n, out.data());
        else if (t == "q6_k") GGUFParser::test_dq_q6_k(in.data(), n, out.data());
        else return usage();
        write_bin(argv[5], out.data(), n);
        return 0;
    }
    if (cmd == "dqrow" && argc == 7) {
        GGUFParser g;
        if (!g.load(argv[2])) return 1;
        const auto& ti = g.tensor_info(argv[3]);
        const int64_t cols = (int64_t)ti.shape[0];
        const int64_t r0 = std::atoll(argv[4]), nr = std::atoll(argv[5]);
        std::vector<float> out((size_t)(cols * nr));
        for (int64_t r = 0; r < nr; r++) g.dequantize_row(argv[3], r0 + r, out.data() + r * cols);
        write_bin(argv[6], out.data(), out.size());
        return 0;
    }
    if ((cmd == "gemv" && argc == 6) || (cmd == "gemm" && argc == 7)) {
        GGUFParser g;
        if (!g.load(argv[2])) return 1;
        const auto& ti = g.tensor_info(argv[3]);
        const int n_in = (int)ti.shape[0], n_out = (int)ti.shape[1];
        auto x = read_bin<float>(argv[4]);
        if (cmd == "gemv") {
            std::vector<float> y(n_out);
            if (!g.gemv_q(argv[3], y.data(), x.data(), n_out, n_in)) return 1;
            write_bin(argv[5], y.data(), y.size());
        } else {
            const int nt = std::atoi(argv[5]);
            std::vector<float> y((size_t)nt * n_out);
            if (!g.gemm_q(argv[3], y.data(), x.data(), nt, n_out, n_in)) return 1;
            write_bin(argv[6], y.data(), y.size());
        }
        return 0;
    }
    if (cmd == "greedy" && (argc == 6 || argc == 8)) {
        Model m;
        if (!load_model(m, argv[2])) return 1;
        auto prompt = read_bin<int32_t>(argv[3]);
        std::vector<float> lg;
        int steps = argc == 8 ? std::atoi(argv[7]) : 0;
        auto toks = greedy(m, prompt, std::atoi(argv[4]), argc == 8 ? &lg : nullptr, steps);
        write_bin(argv[5], toks.data(), toks.size());
        if (argc == 8) write_bin(argv[6], lg.data(), lg.size());
        return 0;
    }
    if (cmd == "batch" && argc == 7) {
        Model m;
        if (!load_model(m, argv[2])) return 1;
        auto toks = read_bin<int32_t>(argv[3]);
        const int npf = std::atoi(argv[4]), nb = std::atoi(argv[5]);
        m.reset();
        if (npf > 0) m.forward_prefill(toks.data(), npf, 0);
        std::vector<float> lg((size_t)nb * m.cfg.n_vocab);
        m.forward_batch(toks.data() + npf, nb, npf, lg.data());
        write_bin(argv[6], lg.data(), lg.size());
        return 0;
    }
    if (cmd == "spec" && (argc == 8 || argc == 10)) {
        Model t, d;
        if (!load_model(t, argv[2]) || !load_model(d, argv[3])) return 1;
        if (argc == 10) {
            // contexts below the reference's own 512 positions (core/model.cpp:64;
            // its per-head scratch is sized for 512, so only smaller values are
            // safe); spec_greedy's reset() re-sizes the KV caches for them
            const int tc = std::atoi(argv[8]), dc = std::atoi(argv[9]);
            if (tc < 2 || tc > 512 || dc < 2 || dc > 512) return usage();
            t.cfg.ctx_len = (uint32_t)tc;
            d.cfg.ctx_len = (uint32_t)dc;
        }
        auto prompt = read_bin<int32_t>(argv[4]);
        SpecStats st;
        auto toks = spec_greedy(t, d, prompt, std::atoi(argv[5]), std::atoi(argv[6]), st);
        write_bin(argv[7], toks.data(), toks.size());
        std::fprintf(stderr, "{\"accepted\": %ld, \"proposed\": %ld, \"passes\": %ld}\n", st.acc, st.prop, st.passes);
        return 0;
    }
    if (cmd == "espec" && argc == 14) {
        Model t, d;
        if (!load_model(t, argv[2]) || !load_model(d, argv[3])) return 1;
        auto prompt = read_bin<int32_t>(argv[4]);
        SamplerParams sp;
        sp.temperature = (float)std::atof(argv[7]);
        sp.top_p = (float)std::atof(argv[8]);
        sp.top_k = std::atoi(argv[9]);
        sp.repeat_pen = (float)std::atof(argv[10]);
        sp.repeat_last = std::atoi(argv[11]);
        SpecStats st;
        auto toks = spec_engine(t, d, prompt, std::atoi(argv[5]), std::atoi(argv[6]), sp,
                                std::strtoull(argv[12], nullptr, 10), st);
        write_bin(argv[13], toks.data(), toks.size());
        std::fprintf(stderr, "{\"accepted\": %ld, \"proposed\": %ld, \"passes\": %ld}\n", st.acc, st.prop, st.passes);
        return 0;
    }
    if (cmd == "sample" && argc == 12) {
        auto logits = read_bin<float>(argv[2]);
        SamplerParams sp;
        sp.temperature = (float)std::atof(argv[3]);
        sp.top_p = (float)std::atof(argv[4]);
        sp.top_k = std::atoi(argv[5]);
        sp.repeat_pen = (float)std::atof(argv[6]);
        sp.repeat_last = std::atoi(argv[7]);
        Sampler s(sp, std::strtoull(argv[8], nullptr, 10));
        auto hist = read_bin<int32_t>(argv[9]);
        for (int32_t h : hist) s.record(h);
        const int nd = std::atoi(argv[10]);
        std::vector<int32_t> out;
        for (int i = 0; i < nd; i++) {
            std::vector<float> lb(logits);
            out.push_back(s.sample(lb.data(), (int)lb.size()));
        }
        write_bin(argv[11], out.data(), out.size());
        return 0;
    }
    if (cmd == "op" && argc >= 3) {
        const std::string op = argv[2];
        if (op == "rmsnorm" && argc == 7) {  // x w eps out
            auto x = read_bin<float>(argv[3]);
            auto w = read_bin<float>(argv[4]);
            std::vector<float> o(x.size());
            ops::rmsnorm(o.data(), x.data(), w.data(), (int)x.size(), (float)std::atof(argv[5]));
            write_bin(argv[6], o.data(), o.size());
            return 0;
        }
        if ((op == "softmax" || op == "silu") && argc == 5) {
            auto x = read_bin<float>(argv[3]);
            if (op == "softmax") ops::softmax(x.data(), (int)x.size());
            else ops::silu(x.data(), (int)x.size());
            write_bin(argv[4], x.data(), x.size());
            return 0;
        }
        if (op == "rope" && argc == 12) {  // q k H KVH hd pos base outq outk
            auto q = read_bin<float>(argv[3]);
            auto k = read_bin<float>(argv[4]);
            ops::rope(q.data(), k.data(), std::atoi(argv[5]), std::atoi(argv[6]), std::atoi(argv[7]),
                      std::atoi(argv[8]), (float)std::atof(argv[9]));
            write_bin(argv[10], q.data(), q.size());
            write_bin(argv[11], k.data(), k.size());
            return 0;
        }
        if (op == "argmax" && argc == 4) {
            auto x = read_bin<float>(argv[3]);
            std::printf("%d\n", ops::argmax(x.data(), (int)x.size()));
            return 0;
        }
        if (op == "dot" && argc == 5) {
            auto a = read_bin<float>(argv[3]);
            auto b = read_bin<float>(argv[4]);
            std::printf("%.9g\n", (double)ops::dot(a.data(), b.data(), (int)a.size()));
            return 0;
        }
        return usage();
    }
    if (cmd == "embed" && argc == 5) {  // Model::embed_tokens (core/model.cpp:248-270)
        Model m;
        if (!load_model(m, argv[2])) return 1;
        auto toks = read_bin<int32_t>(argv[3]);
        auto e = m.embed_tokens(toks);
        write_bin(argv[4], e.data(), e.size());
        return 0;
    }
    if (cmd == "orkv" && argc == 6) {
        // prefill all but the last prompt id, save_state; then a second Model
        // loads the file and decodes the last id: its logits
        Model m;
        if (!load_model(m, argv[2])) return 1;
        auto prompt = read_bin<int32_t>(argv[3]);
        const int n = (int)prompt.size() - 1;
        m.reset();
        m.forward_prefill(prompt.data(), n, 0);
        if (!m.save_state(argv[4], n)) return 1;
        Model m2;
        if (!load_model(m2, argv[2])) return 1;
        int pos = -1;
        if (!m2.load_state(argv[4], pos) || pos != n) return 1;
        const float* lg = m2.forward(prompt.back(), pos);
        write_bin(argv[5], lg, m2.cfg.n_vocab);
        return 0;
    }
    // pieces.bin: each piece as a uint32 byte length, then its bytes
    auto write_pieces = [](const char* path, const std::vector<std::string>& ps) {
        std::vector<uint8_t> out;
        for (const auto& p : ps) {
            const uint32_t n = (uint32_t)p.size();
            out.insert(out.end(), (const uint8_t*)&n, (const uint8_t*)&n + 4);
            out.insert(out.end(), p.begin(), p.end());
        }
        write_bin(path, out.data(), out.size());
    };
    if (cmd == "tokenize" && argc == 6) {  // Tokenizer::encode (core/tokenizer.cpp:252-273)
        GGUFParser g;
        if (!g.load(argv[2])) return 1;
        Tokenizer t;
        if (!t.load(g)) return 1;
        auto txt = read_bin<char>(argv[3]);
        auto ids = t.encode(std::string(txt.begin(), txt.end()), std::atoi(argv[4]) != 0);
        write_bin(argv[5], ids.data(), ids.size());
        return 0;
    }
    if (cmd == "detok" && argc == 5) {  // Tokenizer::decode_one of each id (core/tokenizer.cpp:278-296)
        GGUFParser g;
        if (!g.load(argv[2])) return 1;
        Tokenizer t;
        if (!t.load(g)) return 1;
        auto ids = read_bin<int32_t>(argv[3]);
        std::vector<std::string> ps;
        for (int32_t id : ids) ps.push_back(t.decode_one(id));
        write_pieces(argv[4], ps);
        return 0;
    }
    if (cmd == "engine" && argc == 8) {
        // Engine::generate (core/engine.cpp:83-243) as the reference runs it;
        // messages.bin: role, NUL, content, NUL, ... ; the on_token pieces
        Engine e;
        GenParams gp;
        gp.n_predict = std::atoi(argv[4]);
        gp.temperature = (float)std::atof(argv[5]);
        if (!e.load(argv[2], gp)) return 1;
        if (std::strcmp(argv[3], "-") != 0 && !e.load_draft(argv[3])) return 1;
        auto raw = read_bin<char>(argv[6]);
        std::vector<std::string> f;
        std::string cur;
        for (char c : raw) {
            if (c == 0) { f.push_back(cur); cur.clear(); }
            else cur += c;
        }
        std::vector<Message> msgs;
        for (size_t i = 0; i + 1 < f.size(); i += 2) msgs.push_back({f[i], f[i + 1]});
        std::vector<std::string> ps;
        const std::string resp = e.generate(msgs, gp, [&](const std::string& p) { ps.push_back(p); });
        std::string joined;
        for (const auto& p : ps) joined += p;
        if (joined != resp) { std::fprintf(stderr, "response differs from the streamed pieces\n"); return 1; }
        write_pieces(argv[7], ps);
        return 0;
    }
    if (cmd == "bench" && argc == 8) {
#ifdef _OPENMP
        if (std::atoi(argv[7]) > 0) omp_set_num_threads(std::atoi(argv[7]));
        const int threads = omp_get_max_threads();
#else
        const int threads = 1;
#endif
        Model t;
        if (!load_model(t, argv[2])) return 1;
        auto prompt = read_bin<int32_t>(argv[4]);
        const int n_gen = std::atoi(argv[5]), k = std::atoi(argv[6]);
        const bool spec = std::strcmp(argv[3], "-") != 0;
        Model d;
        if (spec && !load_model(d, argv[3])) return 1;
        // Untimed prefill, then the timed generation, as the reference harness does.
        double dt = 0;
        std::vector<int32_t> toks;
        SpecStats st;
        if (spec) {
            t.reset(); d.reset();
            t.forward_prefill(prompt.data(), (int)prompt.size() - 1, 0);
            d.forward_prefill(prompt.data(), (int)prompt.size() - 1, 0);
            auto g0 = std::chrono::steady_clock::now();
            toks = spec_greedy(t, d, prompt, n_gen, k, st, /*prefill=*/false);
            dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - g0).count();
        } else {
            t.reset();
            t.forward_prefill(prompt.data(), (int)prompt.size() - 1, 0);
            int32_t cur = prompt.back();
            int pos = (int)prompt.size() - 1;
            auto g0 = std::chrono::steady_clock::now();
            for (int s = 0; s < n_gen; s++) {
                const float* lg = t.forward(cur, pos++);
                toks.push_back(cur = argmax_first(lg, (int)t.cfg.n_vocab));
            }
            dt = std::chrono::duration<double>(std::chrono::steady_clock::now() - g0).count();
        }
        uint64_t h = 1469598103934665603ULL;
        for (int32_t x : toks) h = fnv_step(h, x);
        std::fprintf(stderr, "REF_BENCH {\"tok_s\": %.6f, \"tokens\": %zu, \"seconds\": %.6f, \"threads\": %d, "
                             "\"accepted\": %ld, \"proposed\": %ld, \"checksum\": \"%016llx\"}\n",
                     toks.size() / dt, toks.size(), dt, threads, st.acc, st.prop, (unsigned long long)h);
        return 0;
    }
    return usage();
}

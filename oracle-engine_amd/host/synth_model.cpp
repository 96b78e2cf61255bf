#include "synth_model.hpp"
#include "gguf_writer.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <map>

namespace orc {

static inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static uint64_t tensor_key(uint64_t seed, const std::string& name) {
    uint64_t h = 0xCBF29CE484222325ull ^ mix64(seed);
    for (unsigned char c : name) h = (h ^ c) * 0x100000001B3ull;
    return mix64(h);
}

static inline float normal_at(uint64_t key, uint64_t i, float sigma) {
    uint64_t r = mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
    double u1 = ((double)(r >> 32) + 0.5) * (1.0 / 4294967296.0);
    double u2 = ((double)(r & 0xFFFFFFFFull) + 0.5) * (1.0 / 4294967296.0);
    double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
    return (float)(sigma * z);
}

float synth_weight(uint64_t seed, const std::string& tensor, uint64_t i) {
    return normal_at(tensor_key(seed, tensor), i, 0.02f);
}

static SynthSpec tiny(const std::string& name) {
    SynthSpec s;
    s.name = name;
    s.n_layers = 2; s.d_model = 512; s.n_heads = 8; s.n_kv_heads = 2; s.head_dim = 64;
    s.ffn = 1024; s.vocab = 2048; s.seed = 7;
    return s;
}

bool synth_preset(const std::string& name, SynthSpec& s) {
    using T = GGMLType;
    if (name == "c1") {  // Llama-3.2-1B shape, all Q8_0, tied
        s = SynthSpec{}; s.name = name; s.arch = "llama";
        s.n_layers = 16; s.d_model = 2048; s.n_heads = 32; s.n_kv_heads = 8; s.head_dim = 64;
        s.ffn = 8192; s.vocab = 128256; s.rope_theta = 500000.f; s.tied = true; s.seed = 101;
        s.t_default = s.t_attn_v = s.t_ffn_down = s.t_embd = T::Q8_0;
        return true;
    }
    if (name == "c2" || name == "c3d") {  // Llama-3.2-3B shape, Q4_K_M mix, tied (head = token_embd Q6_K)
        s = SynthSpec{}; s.name = name; s.arch = "llama";
        s.n_layers = 28; s.d_model = 3072; s.n_heads = 24; s.n_kv_heads = 8; s.head_dim = 128;
        s.ffn = 8192; s.vocab = 128256; s.rope_theta = 500000.f; s.tied = true; s.seed = 202;
        s.t_default = T::Q4_K; s.t_attn_v = T::Q6_K; s.t_ffn_down = T::Q6_K; s.t_embd = T::Q6_K;
        if (name == "c3d") {  // draft: the target's float layers 0..7 and head, all Q8_0
            s.n_layers = 8; s.tied = false; s.head_from_embd = true;
            s.t_default = s.t_attn_v = s.t_ffn_down = s.t_embd = s.t_output = T::Q8_0;
        }
        return true;
    }
    if (name == "c4" || name == "c5") {  // Qwen2.5-7B shape, QKV bias, untied
        s = SynthSpec{}; s.name = name; s.arch = "qwen2";
        s.n_layers = 28; s.d_model = 3584; s.n_heads = 28; s.n_kv_heads = 4; s.head_dim = 128;
        s.ffn = 18944; s.vocab = 152064; s.rope_theta = 1000000.f; s.rms_eps = 1e-6f;
        s.tied = false; s.qkv_bias = true; s.seed = 404;
        if (name == "c4") {
            s.t_default = T::Q4_K; s.t_attn_v = T::Q6_K; s.t_ffn_down = T::Q6_K;
            s.t_embd = T::Q4_K; s.t_output = T::Q6_K;
        } else {
            s.t_default = s.t_attn_v = s.t_ffn_down = s.t_embd = s.t_output = T::Q6_K;
        }
        return true;
    }
    if (name == "c4d") {  // Qwen2.5-0.5B shape draft, Q8_0, tied
        s = SynthSpec{}; s.name = name; s.arch = "qwen2";
        s.n_layers = 24; s.d_model = 896; s.n_heads = 14; s.n_kv_heads = 2; s.head_dim = 64;
        s.ffn = 4864; s.vocab = 152064; s.rope_theta = 1000000.f; s.rms_eps = 1e-6f;
        s.tied = true; s.qkv_bias = true; s.seed = 505;
        s.t_default = s.t_attn_v = s.t_ffn_down = s.t_embd = T::Q8_0;
        return true;
    }
    // Small models for parity tests (the reference runs them in seconds).
    if (name == "t-q8") { s = tiny(name); return true; }
    if (name == "t-q40") {
        s = tiny(name); s.t_default = s.t_attn_v = s.t_ffn_down = s.t_embd = T::Q4_0; return true;
    }
    if (name == "t-q4k" || name == "t-q4k-d") {  // Q4_K_M-style mix; -d: 1-layer Q8_0 draft of it
        s = tiny("t-q4k");
        s.t_default = T::Q4_K; s.t_attn_v = T::Q6_K; s.t_ffn_down = T::Q6_K; s.t_embd = T::Q6_K;
        if (name == "t-q4k-d") {
            s.name = name; s.n_layers = 1; s.tied = false; s.head_from_embd = true;
            s.t_default = s.t_attn_v = s.t_ffn_down = s.t_embd = s.t_output = T::Q8_0;
        }
        return true;
    }
    if (name == "t-q6k") {
        s = tiny(name); s.tied = false;
        s.t_default = s.t_attn_v = s.t_ffn_down = s.t_embd = s.t_output = T::Q6_K; return true;
    }
    if (name == "t-qwen") {  // qwen2 arch: biases, untied Q4_K embedding + Q6_K head
        s = tiny(name); s.arch = "qwen2"; s.qkv_bias = true; s.tied = false; s.rope_theta = 1000000.f;
        s.n_heads = 8; s.n_kv_heads = 4; s.rms_eps = 1e-6f;
        s.t_default = T::Q4_K; s.t_attn_v = T::Q6_K; s.t_ffn_down = T::Q6_K;
        s.t_embd = T::Q4_K; s.t_output = T::Q6_K; return true;
    }
    if (name == "t-q8-a64") {  // t-q8's tensors in a file that declares general.alignment = 64
        s = tiny("t-q8"); s.alignment = 64; return true;
    }
    if (name == "t-dense") {  // dense weights: F16 embedding, BF16 head, an all-F32 layer, a raw-F32 norm
        s = tiny(name); s.tied = false; s.seed = 11;
        s.t_embd = T::F16; s.t_output = T::BF16; s.f32_layer = 0; s.raw_norm_layer = 1;
        return true;
    }
    if (name == "t-qwen3") {  // qwen3 arch: per-head QK-norm, head_dim 128 (q width 1024 > d_model 512), no bias
        s = tiny(name); s.arch = "qwen3"; s.qk_norm = true; s.tied = false; s.rope_theta = 1000000.f;
        s.head_dim = 128; s.n_heads = 8; s.n_kv_heads = 2; s.rms_eps = 1e-6f; s.seed = 13;
        s.t_default = T::Q4_K; s.t_attn_v = T::Q6_K; s.t_ffn_down = T::Q6_K;
        s.t_embd = T::Q4_K; s.t_output = T::Q6_K; return true;
    }
    if (name == "t-qwen-d") {  // independent 1-layer Q8_0 draft for t-qwen (stochastic spec tests)
        s = tiny(name); s.arch = "qwen2"; s.qkv_bias = true; s.tied = true; s.rope_theta = 1000000.f;
        s.n_layers = 1; s.d_model = 256; s.n_heads = 4; s.n_kv_heads = 2; s.ffn = 512; s.seed = 9;
        s.rms_eps = 1e-6f; return true;
    }
    return false;
}

std::vector<std::string> synth_preset_names() {
    return {"c1", "c2", "c3d", "c4", "c4d", "c5", "t-q8", "t-q40", "t-q4k", "t-q4k-d", "t-q6k", "t-qwen",
            "t-qwen-d", "t-dense", "t-q8-a64", "t-qwen3"};
}

// ── tokenizer stub ──────────────────────────────────────────────────────────

static std::string utf8_of(uint32_t cp) {
    std::string o;
    if (cp < 0x80) {
        o += (char)cp;
    } else if (cp < 0x800) {
        o += (char)(0xC0 | (cp >> 6));
        o += (char)(0x80 | (cp & 0x3F));
    } else {
        o += (char)(0xE0 | (cp >> 12));
        o += (char)(0x80 | ((cp >> 6) & 0x3F));
        o += (char)(0x80 | (cp & 0x3F));
    }
    return o;
}

// GPT-2's byte -> symbol map (OpenAI's published bytes_to_unicode): printable
// Latin-1 bytes map to themselves, the other 68 bytes to U+0100 upwards in
// byte order.
static std::vector<std::string> byte_symbols() {
    std::vector<std::string> sym(256);
    int next = 256;
    for (int b = 0; b < 256; ++b) {
        const bool keep = (b >= 33 && b <= 126) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
        sym[b] = utf8_of(keep ? (uint32_t)b : (uint32_t)next++);
    }
    return sym;
}

// Text the stub's merges are learned from (spaces attach to the next word,
// as the reference's pre-tokenizer splits).
static const char* kStubCorpus =
    "the quick brown fox jumps over the lazy dog and then the dog sleeps in the sun while the fox runs "
    "into the green forest where the trees are tall and the river is cold there is a small house near "
    "the river and the people who live there are kind they speak to the animals and the animals answer "
    "in their own language the system is an assistant that helps the user the user asks a question and "
    "the assistant gives an answer with care and patience every answer is short and true";

VocabStub make_vocab_stub(const SynthSpec& s) {
    VocabStub v;
    const int V = s.vocab;
    const std::vector<std::string> sym = byte_symbols();
    v.tokens.assign(V, std::string());
    v.types.assign(V, 1);
    for (int b = 0; b < 256 && b < V; ++b) v.tokens[b] = sym[b];
    // words of the corpus as symbol sequences
    std::vector<std::vector<std::string>> words;
    {
        std::string cur;
        auto flush = [&] {
            if (cur.empty()) return;
            std::vector<std::string> w;
            for (unsigned char c : cur) w.push_back(sym[c]);
            words.push_back(w);
            cur.clear();
        };
        for (const char* p = kStubCorpus; *p; ++p) {
            if (*p == ' ') flush();
            cur += *p;
        }
        flush();
    }
    // greedy pair merges: the most frequent adjacent pair, ties by the smaller key
    const int n_merge = std::max(0, std::min(300, V - 256 - 32));
    int next_id = 256;
    for (int m = 0; m < n_merge; ++m) {
        std::map<std::string, int> cnt;
        for (const auto& w : words)
            for (size_t i = 0; i + 1 < w.size(); ++i) ++cnt[w[i] + " " + w[i + 1]];
        std::string best;
        int bc = 0;
        for (const auto& kv : cnt)
            if (kv.second > bc) {
                bc = kv.second;
                best = kv.first;
            }
        if (bc < 2) break;
        const size_t sp = best.find(' ');
        const std::string a = best.substr(0, sp), b = best.substr(sp + 1);
        v.merges.push_back(best);
        v.tokens[next_id++] = a + b;
        for (auto& w : words) {
            std::vector<std::string> o;
            for (size_t i = 0; i < w.size(); ++i) {
                if (i + 1 < w.size() && w[i] == a && w[i + 1] == b) {
                    o.push_back(a + b);
                    ++i;
                } else {
                    o.push_back(w[i]);
                }
            }
            w.swap(o);
        }
    }
    for (int i = next_id; i < V; ++i) v.tokens[i] = "<unused" + std::to_string(i) + ">";
    // chat special tokens (control type 3) at the architecture's usual ids,
    // or near the end of a small vocabulary
    std::vector<std::pair<std::string, int>> sp;
    const bool qwen = s.arch.rfind("qwen", 0) == 0;
    if (qwen) {
        const int base = V >= 151646 ? 151643 : V - 16;
        sp = {{"<|endoftext|>", base}, {"<|im_start|>", base + 1}, {"<|im_end|>", base + 2}};
    } else {
        const int base = V >= 128256 ? 128000 : V - 16;
        sp = {{"<|begin_of_text|>", base}, {"<|end_of_text|>", base + 1}, {"<|start_header_id|>", base + 6},
              {"<|end_header_id|>", base + 7}, {"<|eot_id|>", base + 9}};
    }
    const std::string eot_name = qwen ? "<|im_end|>" : "<|eot_id|>";
    for (auto& t : sp) {
        if (t.first == eot_name && s.eot_id >= 0 && s.eot_id < V) t.second = s.eot_id;
        v.tokens[t.second] = t.first;
        v.types[t.second] = 3;
    }
    v.bos = sp[0].second;
    for (const auto& t : sp)
        if (t.first == eot_name) v.eos = t.second;
    return v;
}

bool synth_write(const SynthSpec& s, const std::string& path, bool verbose) {
    GGUFWriter w;
    w.alignment = s.alignment;
    const std::string a = s.arch;
    w.add_str("general.architecture", a);
    w.add_str("general.name", "orc-synthetic-" + s.name);
    w.add_u32(a + ".block_count", (uint32_t)s.n_layers);
    w.add_u32(a + ".context_length", 131072);
    w.add_u32(a + ".embedding_length", (uint32_t)s.d_model);
    w.add_u32(a + ".feed_forward_length", (uint32_t)s.ffn);
    w.add_u32(a + ".attention.head_count", (uint32_t)s.n_heads);
    w.add_u32(a + ".attention.head_count_kv", (uint32_t)s.n_kv_heads);
    w.add_u32(a + ".attention.key_length", (uint32_t)s.head_dim);
    w.add_u32(a + ".attention.value_length", (uint32_t)s.head_dim);
    w.add_f32(a + ".rope.freq_base", s.rope_theta);
    w.add_f32(a + ".attention.layer_norm_rms_epsilon", s.rms_eps);
    w.add_u32(a + ".vocab_size", (uint32_t)s.vocab);
    if (s.vocab_stub) {
        const VocabStub v = make_vocab_stub(s);
        w.add_str("tokenizer.ggml.model", "gpt2");
        w.add_str_array("tokenizer.ggml.tokens", v.tokens);
        w.add_i32_array("tokenizer.ggml.token_type", v.types);
        w.add_str_array("tokenizer.ggml.merges", v.merges);
        w.add_u32("tokenizer.ggml.bos_token_id", (uint32_t)v.bos);
        w.add_u32("tokenizer.ggml.eos_token_id", (uint32_t)v.eos);
    }

    const uint64_t seed = s.seed;
    const int D = s.d_model, NQ = s.n_heads * s.head_dim, NKV = s.n_kv_heads * s.head_dim, FF = s.ffn;

    // A quantized matrix [n_in, n_out] whose floats come from stream `src`.
    auto matrix = [&](const std::string& name, const std::string& src, int n_in, int n_out, GGMLType t) {
        w.add_tensor(name, {(uint64_t)n_in, (uint64_t)n_out}, t,
                     [seed, src, n_in, t](int64_t r0, int64_t r1, uint8_t* dst) {
                         const uint64_t key = tensor_key(seed, src);
                         const uint64_t rb = row_bytes(t, n_in);
#pragma omp parallel for schedule(dynamic, 16)
                         for (int64_t r = r0; r < r1; ++r) {
                             std::vector<float> row(n_in);
                             for (int i = 0; i < n_in; ++i) row[i] = normal_at(key, (uint64_t)r * n_in + i, 0.02f);
                             quantize_any(t, row.data(), n_in, dst + (r - r0) * rb);
                         }
                     });
    };
    auto ones = [&](const std::string& name, int n) {
        w.add_tensor(name, {(uint64_t)n}, GGMLType::F32, [n](int64_t, int64_t, uint8_t* dst) {
            for (int i = 0; i < n; ++i) { float one = 1.f; std::memcpy(dst + 4 * i, &one, 4); }
        });
    };
    auto bias = [&](const std::string& name, int n) {
        w.add_tensor(name, {(uint64_t)n}, GGMLType::F32, [seed, name, n](int64_t, int64_t, uint8_t* dst) {
            const uint64_t key = tensor_key(seed, name);
            for (int i = 0; i < n; ++i) { float v = normal_at(key, (uint64_t)i, 0.02f); std::memcpy(dst + 4 * i, &v, 4); }
        });
    };

    // per-head QK-norm weights (Qwen3): head_dim F32 values 1 + N(0, 0.1^2),
    // so the norm's weights matter
    auto head_norm = [&](const std::string& name, int n) {
        w.add_tensor(name, {(uint64_t)n}, GGMLType::F32, [seed, name, n](int64_t, int64_t, uint8_t* dst) {
            const uint64_t key = tensor_key(seed, name);
            for (int i = 0; i < n; ++i) { float v = 1.f + normal_at(key, (uint64_t)i, 0.1f); std::memcpy(dst + 4 * i, &v, 4); }
        });
    };

    // norm weights 1 + N(0, 0.1^2) stored as F32 bytes under a declared F16
    // type of 2n values (the same byte count)
    auto raw_norm = [&](const std::string& name, int n) {
        w.add_tensor(name, {(uint64_t)(2 * n)}, GGMLType::F16, [seed, name, n](int64_t, int64_t, uint8_t* dst) {
            const uint64_t key = tensor_key(seed, name);
            for (int i = 0; i < n; ++i) { float v = 1.f + normal_at(key, (uint64_t)i, 0.1f); std::memcpy(dst + 4 * i, &v, 4); }
        });
    };

    matrix("token_embd.weight", "token_embd.weight", D, s.vocab, s.t_embd);
    for (int l = 0; l < s.n_layers; ++l) {
        const std::string b = "blk." + std::to_string(l) + ".";
        const bool f32 = l == s.f32_layer;
        const GGMLType td = f32 ? GGMLType::F32 : s.t_default, tv = f32 ? GGMLType::F32 : s.t_attn_v,
                       tdn = f32 ? GGMLType::F32 : s.t_ffn_down;
        if (l == s.raw_norm_layer) raw_norm(b + "attn_norm.weight", D);
        else ones(b + "attn_norm.weight", D);
        matrix(b + "attn_q.weight", b + "attn_q.weight", D, NQ, td);
        matrix(b + "attn_k.weight", b + "attn_k.weight", D, NKV, td);
        matrix(b + "attn_v.weight", b + "attn_v.weight", D, NKV, tv);
        if (s.qkv_bias) {
            bias(b + "attn_q.bias", NQ);
            bias(b + "attn_k.bias", NKV);
            bias(b + "attn_v.bias", NKV);
        }
        if (s.qk_norm) {
            head_norm(b + "attn_q_norm.weight", s.head_dim);
            head_norm(b + "attn_k_norm.weight", s.head_dim);
        }
        matrix(b + "attn_output.weight", b + "attn_output.weight", NQ, D, td);
        ones(b + "ffn_norm.weight", D);
        matrix(b + "ffn_gate.weight", b + "ffn_gate.weight", D, FF, td);
        matrix(b + "ffn_up.weight", b + "ffn_up.weight", D, FF, td);
        matrix(b + "ffn_down.weight", b + "ffn_down.weight", FF, D, tdn);
    }
    ones("output_norm.weight", D);
    if (!s.tied)
        matrix("output.weight", s.head_from_embd ? "token_embd.weight" : "output.weight", D, s.vocab, s.t_output);
    return w.write(path, verbose);
}

}  // namespace orc

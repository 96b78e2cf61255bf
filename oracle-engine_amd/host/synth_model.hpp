// Synthetic random-init Llama/Qwen2/Qwen3-shaped GGUF models.
//
// Every linear weight is i.i.d. N(0, 0.02^2) drawn from a counter-based
// generator keyed by (seed, tensor name, element index), so any tensor can be
// regenerated independently and in parallel, and a draft model can reuse the
// exact float weights of its target's layers. Norm weights are 1.0, Qwen2
// QKV biases are N(0, 0.02^2) and Qwen3 QK-norm weights 1 + N(0, 0.1^2), in F32. The tensor names and metadata keys are
// the ones the reference reads (core/model.cpp:48-80, 99-154).
#pragma once
#include "gguf_types.hpp"
#include <cstdint>
#include <string>
#include <vector>

namespace orc {

struct SynthSpec {
    std::string name;
    std::string arch = "llama";     // "llama", "qwen2" or "qwen3"
    int n_layers = 2, d_model = 512, n_heads = 8, n_kv_heads = 2, head_dim = 64;
    int ffn = 1024, vocab = 2048;
    float rope_theta = 500000.f, rms_eps = 1e-5f;
    bool tied = true;               // no output.weight: the LM head is token_embd
    bool qkv_bias = false;
    bool qk_norm = false;           // Qwen3 per-head attn_q_norm / attn_k_norm (head_dim F32 each)
    GGMLType t_default = GGMLType::Q8_0;   // attn_q/k/output, ffn_gate/up
    GGMLType t_attn_v = GGMLType::Q8_0;
    GGMLType t_ffn_down = GGMLType::Q8_0;
    GGMLType t_embd = GGMLType::Q8_0;
    GGMLType t_output = GGMLType::Q8_0;    // only when !tied
    uint64_t seed = 1;
    // Layer whose seven matrices are all F32 (-1: none), and layer whose
    // attn_norm is declared F16 with twice the values while its bytes are
    // the F32 norm weights (1 + N(0, 0.1^2)), which the reference reads as
    // raw F32 whatever the declared type (core/model.cpp:317-320); -1: none.
    int f32_layer = -1, raw_norm_layer = -1;
    // general.alignment of the file (32: not declared, the reference's only value)
    uint32_t alignment = 32;
    // When true, output.weight holds the same float weights as token_embd
    // (a draft that owns a re-quantized copy of its target's tied head).
    bool head_from_embd = false;
    // Tokenizer metadata stub (tokenizer.ggml.*): a byte-level BPE vocabulary
    // the reference's Tokenizer (core/tokenizer.cpp:41-78) loads: the 256
    // byte symbols, merges learned from a fixed text, the architecture's chat
    // special tokens, the rest filler. Off by default (the file then equals
    // the one the reference fixtures were made from).
    bool vocab_stub = false;
    // With the stub: the id of the end-of-turn token (<|eot_id|>, qwen2:
    // <|im_end|>) instead of its usual place; -1 keeps it.
    int eot_id = -1;
};

// The stub's tokens, types, merges, bos / eos ids for a spec (exposed for tests).
struct VocabStub {
    std::vector<std::string> tokens, merges;
    std::vector<int32_t> types;
    int32_t bos = 0, eos = 0;
};
VocabStub make_vocab_stub(const SynthSpec& s);

// Named presets: the five benchmark configurations (c1..c5, c3d/c4d drafts)
// and small test models (t-*). Returns false for an unknown name.
bool synth_preset(const std::string& name, SynthSpec& out);
std::vector<std::string> synth_preset_names();

// The float value of element `i` of tensor `tensor` under `seed` (N(0, 0.02^2)).
float synth_weight(uint64_t seed, const std::string& tensor, uint64_t i);

// Writes the model; returns false on failure.
bool synth_write(const SynthSpec& s, const std::string& path, bool verbose);

}  // namespace orc

// Tokenizer — the reference's byte-level BPE tokenizer (core/tokenizer.hpp:17-79),
// loaded from the GGUF metadata (tokenizer.ggml.tokens / token_type / merges /
// bos_token_id / eos_token_id). It stays on the host: it runs once per
// prompt and once per generated id. Its rules follow the reference exactly,
// since the ids it yields must be the reference's:
//  * bytes map to symbols with GPT-2's published bytes_to_unicode table;
//  * pre-tokenization splits only at spaces, tabs and line breaks: a space or
//    tab starts the next word, a line break is a word of its own;
//  * a word that is a control token (type >= 3) as a whole encodes to its id,
//    any other word is merged by the lowest merge rank first (the leftmost
//    pair on equal ranks), and a piece missing from the vocabulary falls back
//    to <0xXX> byte tokens, or id 0;
//  * decode_one: <0xXX> tokens give their byte, control tokens nothing, the
//    rest their symbols mapped back to bytes.
#pragma once
#include "gguf_parser.hpp"

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

class Tokenizer {
public:
    bool load(const GGUFParser& gguf);
    bool is_loaded() const { return !tokens_.empty(); }

    std::vector<int32_t> encode(const std::string& text, bool add_bos = true) const;
    std::string decode(const std::vector<int32_t>& ids) const;
    std::string decode_one(int32_t id) const;
    // the id of a token by its exact text, -1 if absent
    int32_t special_id(const std::string& name) const;

    int32_t bos_id() const { return bos_id_; }
    int32_t eos_id() const { return eos_id_; }
    uint32_t vocab_size() const { return (uint32_t)tokens_.size(); }

private:
    std::vector<std::string> tokens_;
    std::vector<int32_t> types_;
    std::unordered_map<std::string, int32_t> id_of_;
    std::unordered_map<std::string, int> rank_;  // "left right" -> merge rank
    int32_t bos_id_ = 128000, eos_id_ = 128009;   // core/tokenizer.hpp:66-67 defaults
    std::string sym_[256];                        // byte -> symbol (UTF-8)
    uint8_t byte_of_[512] = {};                   // symbol code point (< 512) -> byte

    std::vector<std::string> words(const std::string& text) const;
    void merge_word(const std::string& word, std::vector<int32_t>& out) const;
    std::string to_bytes(const std::string& symbols) const;
};

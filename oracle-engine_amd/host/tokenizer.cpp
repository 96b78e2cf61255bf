// Byte-level BPE tokenizer (see tokenizer.hpp for the rules it keeps).
#include "tokenizer.hpp"

#include <climits>
#include <cstdio>

namespace {

// Length of the UTF-8 sequence a lead byte starts (1 for ASCII and for the
// continuation bytes the reference also steps over one at a time).
int seq_len(unsigned char c) { return c < 0x80 ? 1 : c < 0xE0 ? 2 : c < 0xF0 ? 3 : 4; }

// Code point of the sequence at p (len bytes, as seq_len says).
uint32_t code_point(const unsigned char* p, int len) {
    switch (len) {
        case 1: return p[0];
        case 2: return ((p[0] & 0x1Fu) << 6) | (p[1] & 0x3Fu);
        case 3: return ((p[0] & 0x0Fu) << 12) | ((p[1] & 0x3Fu) << 6) | (p[2] & 0x3Fu);
        default: return ((p[0] & 0x07u) << 18) | ((p[1] & 0x3Fu) << 12) | ((p[2] & 0x3Fu) << 6) | (p[3] & 0x3Fu);
    }
}

std::string utf8(uint32_t cp) {
    std::string o;
    if (cp < 0x80) {
        o += (char)cp;
    } else if (cp < 0x800) {
        o += (char)(0xC0 | (cp >> 6));
        o += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        o += (char)(0xE0 | (cp >> 12));
        o += (char)(0x80 | ((cp >> 6) & 0x3F));
        o += (char)(0x80 | (cp & 0x3F));
    } else {
        o += (char)(0xF0 | (cp >> 18));
        o += (char)(0x80 | ((cp >> 12) & 0x3F));
        o += (char)(0x80 | ((cp >> 6) & 0x3F));
        o += (char)(0x80 | (cp & 0x3F));
    }
    return o;
}

}  // namespace

bool Tokenizer::load(const GGUFParser& g) {  // core/tokenizer.cpp:41-78
    // GPT-2 bytes_to_unicode: printable Latin-1 bytes keep their value, the
    // rest take U+0100, U+0101, ... in byte order
    int next = 256;
    for (int b = 0; b < 256; ++b) {
        const bool keep = (b >= 33 && b <= 126) || (b >= 0xA1 && b <= 0xAC) || (b >= 0xAE && b <= 0xFF);
        const uint32_t cp = keep ? (uint32_t)b : (uint32_t)next++;
        sym_[b] = utf8(cp);
        byte_of_[cp] = (uint8_t)b;
    }
    tokens_ = g.meta_arr_str("tokenizer.ggml.tokens");
    if (tokens_.empty()) {
        std::fprintf(stderr, "[Tokenizer] tokenizer.ggml.tokens missing from the GGUF\n");
        return false;
    }
    const MetaValue& ty = g.meta("tokenizer.ggml.token_type");
    types_ = ty.kind == MetaValue::ARR_I32 ? ty.arr_i32 : std::vector<int32_t>();
    id_of_.clear();
    id_of_.reserve(tokens_.size());
    for (int32_t i = 0; i < (int32_t)tokens_.size(); ++i) id_of_[tokens_[i]] = i;  // a later duplicate wins
    rank_.clear();
    const auto& mg = g.meta_arr_str("tokenizer.ggml.merges");
    rank_.reserve(mg.size());
    for (int i = 0; i < (int)mg.size(); ++i) rank_[mg[i]] = i;
    bos_id_ = (int32_t)g.meta_u32("tokenizer.ggml.bos_token_id", 1);
    eos_id_ = (int32_t)g.meta_u32("tokenizer.ggml.eos_token_id", 2);
    return true;
}

// core/tokenizer.cpp:214-247
std::vector<std::string> Tokenizer::words(const std::string& text) const {
    std::vector<std::string> out;
    std::string w;
    size_t i = 0;
    while (i < text.size()) {
        const unsigned char c = (unsigned char)text[i];
        if (c == ' ' || c == '\t' || c == '\n' || c == '\r') {
            if (!w.empty()) out.push_back(w);
            w.assign(1, (char)c);
            ++i;
            if (c == '\n' || c == '\r') {  // a line break stands alone
                out.push_back(w);
                w.clear();
            }
            continue;
        }
        const size_t n = std::min<size_t>(seq_len(c), text.size() - i);
        w.append(text, i, n);
        i += n;
    }
    if (!w.empty()) out.push_back(w);
    return out;
}

// core/tokenizer.cpp:162-206: merge the word's symbols, lowest rank first
void Tokenizer::merge_word(const std::string& word, std::vector<int32_t>& out) const {
    std::string gs;  // the word's bytes as symbols
    for (unsigned char b : word) gs += sym_[b];
    std::vector<std::string> parts;
    for (size_t i = 0; i < gs.size();) {
        const int n = std::min<int>(seq_len((unsigned char)gs[i]), (int)(gs.size() - i));
        const uint32_t cp = code_point((const unsigned char*)gs.data() + i, n);
        parts.push_back(utf8(cp));
        i += n;
    }
    while (parts.size() > 1) {
        int best = INT_MAX, at = -1;
        for (size_t i = 0; i + 1 < parts.size(); ++i) {
            auto it = rank_.find(parts[i] + " " + parts[i + 1]);
            if (it != rank_.end() && it->second < best) {
                best = it->second;
                at = (int)i;
            }
        }
        if (at < 0) break;
        parts[at] += parts[at + 1];
        parts.erase(parts.begin() + at + 1);
    }
    for (const std::string& p : parts) {
        auto it = id_of_.find(p);
        if (it != id_of_.end()) {
            out.push_back(it->second);
            continue;
        }
        for (unsigned char b : to_bytes(p)) {  // byte fallback
            char name[8];
            std::snprintf(name, sizeof name, "<0x%02X>", b);
            auto jt = id_of_.find(name);
            out.push_back(jt != id_of_.end() ? jt->second : 0);
        }
    }
}

// symbols back to bytes (core/tokenizer.cpp:140-155): code points below 512
// through the byte table, others as their UTF-8
std::string Tokenizer::to_bytes(const std::string& s) const {
    std::string out;
    for (size_t i = 0; i < s.size();) {
        const int n = seq_len((unsigned char)s[i]);
        const uint32_t cp = code_point((const unsigned char*)s.data() + i, n);
        if (cp < 512) out += (char)byte_of_[cp];
        else out += utf8(cp);
        i += n;
    }
    return out;
}

std::vector<int32_t> Tokenizer::encode(const std::string& text, bool add_bos) const {  // core/tokenizer.cpp:252-273
    std::vector<int32_t> ids;
    if (add_bos) ids.push_back(bos_id_);
    for (const std::string& w : words(text)) {
        auto it = id_of_.find(w);
        if (it != id_of_.end() && it->second < (int32_t)types_.size() && types_[it->second] >= 3) {
            ids.push_back(it->second);
            continue;
        }
        merge_word(w, ids);
    }
    return ids;
}

std::string Tokenizer::decode_one(int32_t id) const {  // core/tokenizer.cpp:278-296
    if (id < 0 || id >= (int32_t)tokens_.size()) return "";
    const std::string& t = tokens_[id];
    if (t.size() == 6 && t[0] == '<' && t[1] == '0' && t[2] == 'x') {
        unsigned int b = 0;
        if (std::sscanf(t.c_str() + 3, "%02x>", &b) == 1) return std::string(1, (char)b);
    }
    if (id < (int32_t)types_.size() && types_[id] >= 3) return "";
    return to_bytes(t);
}

std::string Tokenizer::decode(const std::vector<int32_t>& ids) const {
    std::string out;
    for (int32_t id : ids) out += decode_one(id);
    return out;
}

int32_t Tokenizer::special_id(const std::string& name) const {
    auto it = id_of_.find(name);
    return it != id_of_.end() ? it->second : -1;
}

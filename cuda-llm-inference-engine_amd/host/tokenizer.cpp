// tokenizer.cpp — GPT-2 byte-level BPE tokenizer (include/ie_bpe_tokenizer.h)
// and its C ABI (include/ie_tokenizer.h).  Host code: prompts are tokenized
// once per request, next to a decode step that runs on the GPU.
//
// Behaviour follows the reference's BPETokenizer (src/tokenizer.cpp):
//   * symbols: every byte is one printable character, GPT-2's published
//     byte-to-unicode table (tokenizer.cpp:11-48);
//   * vocab.json: token string -> id; ids in [0, 50257) also fill the id ->
//     token table, which has 50257 entries whatever the file holds
//     (tokenizer.cpp:61-116);
//   * merges.txt: one "a b" pair per line in rank order, blank lines and lines
//     starting with '#' skipped, the split at the first space, a repeated pair
//     keeping its later rank (tokenizer.cpp:118-131);
//   * encode: the text split at whitespace, every word after the first
//     prefixed with the space byte's symbol, its symbols merged greedily by
//     lowest rank, the leftmost pair first among equal ranks and one pair per
//     pass, then each piece looked up and dropped when absent
//     (tokenizer.cpp:134-189);
//   * decode: each character of the id's token mapped back to its byte,
//     characters outside the table copied as they are, ids outside the table
//     giving nothing (tokenizer.cpp:191-217).
// vocab.json is parsed as JSON (the reference scans for quotes, which ends a
// key early when it closes on an escaped backslash, and writes each half of a
// surrogate pair as its own character); on every other file both give the
// same tables.
#include "ie_bpe_tokenizer.h"
#include "ie_tokenizer.h"

#include <algorithm>
#include <climits>
#include <cstring>
#include <fstream>
#include <functional>
#include <sstream>
#include <stdexcept>

#include "../csrc/ie_internal.h"

namespace {

constexpr int kTableIds = 50257;  // the reference's fixed id -> token table

void put_utf8(std::string& s, unsigned cp) {
    if (cp < 0x80) {
        s += (char)cp;
    } else if (cp < 0x800) {
        s += (char)(0xC0 | (cp >> 6));
        s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
        s += (char)(0xE0 | (cp >> 12));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    } else {
        s += (char)(0xF0 | (cp >> 18));
        s += (char)(0x80 | ((cp >> 12) & 0x3F));
        s += (char)(0x80 | ((cp >> 6) & 0x3F));
        s += (char)(0x80 | (cp & 0x3F));
    }
}

// Bytes of one character starting at lead byte c, as the reference counts
// them (a stray continuation byte counts as one).
int char_len(unsigned char c) { return c >= 0xF0 ? 4 : c >= 0xE0 ? 3 : c >= 0xC0 ? 2 : 1; }

bool is_space(char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\v' || c == '\f' || c == '\r'; }

std::string read_file(const std::string& path) {
    std::ifstream f(path, std::ios::binary);
    if (!f) throw std::runtime_error("cannot open " + path);
    std::ostringstream ss;
    ss << f.rdbuf();
    return ss.str();
}

// A JSON object of string keys and non-negative integer values.
class VocabReader {
public:
    explicit VocabReader(const std::string& s) : s_(s) {}

    template <typename F>
    void each(F&& f) {
        ws();
        expect('{');
        ws();
        if (peek() == '}') return;
        for (;;) {
            ws();
            std::string key = str();
            ws();
            expect(':');
            ws();
            f(key, id());
            ws();
            const char c = get();
            if (c == '}') return;
            if (c != ',') fail("',' or '}'");
        }
    }

private:
    const std::string& s_;
    size_t i_ = 0;

    [[noreturn]] void fail(const char* what) const {
        throw std::runtime_error("vocab.json: expected " + std::string(what) + " at byte " + std::to_string(i_));
    }
    char peek() const { return i_ < s_.size() ? s_[i_] : '\0'; }
    char get() {
        if (i_ >= s_.size()) fail("more input");
        return s_[i_++];
    }
    void expect(char c) {
        if (get() != c) fail(std::string(1, c).c_str());
    }
    void ws() {
        while (i_ < s_.size() && (s_[i_] == ' ' || s_[i_] == '\t' || s_[i_] == '\n' || s_[i_] == '\r')) ++i_;
    }
    unsigned hex4() {
        unsigned v = 0;
        for (int k = 0; k < 4; ++k) {
            const char c = get();
            v <<= 4;
            if (c >= '0' && c <= '9') v |= (unsigned)(c - '0');
            else if (c >= 'a' && c <= 'f') v |= (unsigned)(c - 'a' + 10);
            else if (c >= 'A' && c <= 'F') v |= (unsigned)(c - 'A' + 10);
            else fail("a hex digit");
        }
        return v;
    }
    std::string str() {
        expect('"');
        std::string out;
        for (;;) {
            const char c = get();
            if (c == '"') return out;
            if (c != '\\') {
                out += c;
                continue;
            }
            const char e = get();
            switch (e) {
                case '"': out += '"'; break;
                case '\\': out += '\\'; break;
                case '/': out += '/'; break;
                case 'b': out += '\b'; break;
                case 'f': out += '\f'; break;
                case 'n': out += '\n'; break;
                case 'r': out += '\r'; break;
                case 't': out += '\t'; break;
                case 'u': {
                    unsigned cp = hex4();
                    // A high surrogate followed by an escaped low one is one
                    // code point; a lone half is kept as its own character.
                    if (cp >= 0xD800 && cp < 0xDC00 && i_ + 5 < s_.size() && s_[i_] == '\\' && s_[i_ + 1] == 'u') {
                        const size_t at = i_;
                        i_ += 2;
                        const unsigned lo = hex4();
                        if (lo >= 0xDC00 && lo < 0xE000)
                            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                        else
                            i_ = at;
                    }
                    put_utf8(out, cp);
                    break;
                }
                default: fail("an escape character");
            }
        }
    }
    int id() {
        const size_t start = i_;
        long long v = 0;
        while (peek() >= '0' && peek() <= '9') {
            v = v * 10 + (get() - '0');
            if (v > INT_MAX) fail("an id below 2^31");
        }
        if (i_ == start) fail("a non-negative integer id");
        return (int)v;
    }
};

}  // namespace

size_t BPETokenizer::PairHash::operator()(const std::pair<std::string, std::string>& p) const {
    const size_t h = std::hash<std::string>()(p.first);
    return h ^ (std::hash<std::string>()(p.second) + 0x9E3779B97F4A7C15ull + (h << 6) + (h >> 2));
}

BPETokenizer::BPETokenizer(const std::string& model_dir) {
    // GPT-2's byte -> character table: the printable Latin-1 bytes stand for
    // themselves, the other 68 take code points 256, 257, ... in byte order.
    int next = 256;
    for (int b = 0; b < 256; ++b) {
        const bool printable = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
        std::string sym;
        put_utf8(sym, printable ? (unsigned)b : (unsigned)next++);
        byte_sym_[b] = sym;
        sym_byte_[sym] = (unsigned char)b;
    }

    id_to_token_.assign(kTableIds, std::string());
    const std::string vocab = read_file(model_dir + "/vocab.json");
    VocabReader(vocab).each([&](const std::string& tok, int id) {
        token_to_id_[tok] = id;
        if (id < kTableIds) id_to_token_[id] = tok;
    });

    const std::string merges = read_file(model_dir + "/merges.txt");
    int rank = 0;
    size_t p = 0;
    while (p < merges.size()) {
        size_t e = merges.find('\n', p);
        if (e == std::string::npos) e = merges.size();
        const std::string line = merges.substr(p, e - p);
        p = e + 1;
        if (line.empty() || line[0] == '#') continue;
        const size_t sp = line.find(' ');
        if (sp == std::string::npos) continue;
        rank_[{line.substr(0, sp), line.substr(sp + 1)}] = rank++;
    }
}

std::vector<std::string> BPETokenizer::merge(std::vector<std::string> syms) const {
    while (syms.size() > 1) {
        int best = INT_MAX;
        size_t at = 0;
        for (size_t j = 0; j + 1 < syms.size(); ++j) {
            const auto it = rank_.find({syms[j], syms[j + 1]});
            if (it != rank_.end() && it->second < best) {
                best = it->second;
                at = j;
            }
        }
        if (best == INT_MAX) break;
        syms[at] += syms[at + 1];
        syms.erase(syms.begin() + (long)at + 1);
    }
    return syms;
}

std::vector<int> BPETokenizer::encode(const std::string& text) const {
    std::vector<int> ids;
    bool first = true;
    size_t i = 0;
    while (i < text.size()) {
        while (i < text.size() && is_space(text[i])) ++i;
        if (i == text.size()) break;
        std::vector<std::string> syms;
        if (!first) syms.push_back(byte_sym_[0x20]);
        first = false;
        for (; i < text.size() && !is_space(text[i]); ++i) syms.push_back(byte_sym_[(unsigned char)text[i]]);
        for (const std::string& piece : merge(std::move(syms))) {
            const auto it = token_to_id_.find(piece);
            if (it != token_to_id_.end()) ids.push_back(it->second);
        }
    }
    return ids;
}

std::string BPETokenizer::decode(int token_id) const {
    if (token_id < 0 || token_id >= (int)id_to_token_.size()) return std::string();
    const std::string& tok = id_to_token_[token_id];
    std::string out;
    for (size_t i = 0; i < tok.size();) {
        const std::string ch = tok.substr(i, (size_t)char_len((unsigned char)tok[i]));
        const auto it = sym_byte_.find(ch);
        if (it != sym_byte_.end())
            out += (char)it->second;
        else
            out += ch;
        i += ch.size();
    }
    return out;
}

std::string BPETokenizer::decode(const std::vector<int>& token_ids) const {
    std::string out;
    for (int id : token_ids) out += decode(id);
    return out;
}

// ------------------------------------------------------------------ C ABI
struct ie_tokenizer {
    BPETokenizer tok;
};

namespace {
template <typename F>
int tk_guarded(const char* fn, F&& f) {
    try {
        f();
        return IE_OK;
    } catch (const std::exception& ex) {
        return ie::fail(IE_ERR_INVALID, "%s: %s", fn, ex.what());
    }
}
}  // namespace

extern "C" int ie_tokenizer_create(ie_tokenizer** out, const char* model_dir) {
    if (!out || !model_dir) return ie::fail(IE_ERR_INVALID, "ie_tokenizer_create: null argument");
    *out = nullptr;
    return tk_guarded("ie_tokenizer_create", [&] { *out = new ie_tokenizer{BPETokenizer(model_dir)}; });
}

extern "C" int ie_tokenizer_destroy(ie_tokenizer* t) {
    delete t;
    return IE_OK;
}

extern "C" int ie_tokenizer_encode(const ie_tokenizer* t, const char* text, size_t len, int* ids, size_t cap,
                                   size_t* n_ids) {
    if (!t || !n_ids || (!text && len) || (!ids && cap))
        return ie::fail(IE_ERR_INVALID, "ie_tokenizer_encode: null argument");
    return tk_guarded("ie_tokenizer_encode", [&] {
        const std::vector<int> v = t->tok.encode(std::string(text ? text : "", len));
        *n_ids = v.size();
        if (cap) std::memcpy(ids, v.data(), std::min(cap, v.size()) * sizeof(int));
    });
}

extern "C" int ie_tokenizer_decode(const ie_tokenizer* t, const int* ids, size_t n, char* out, size_t cap,
                                   size_t* n_bytes) {
    if (!t || !n_bytes || (!ids && n) || (!out && cap))
        return ie::fail(IE_ERR_INVALID, "ie_tokenizer_decode: null argument");
    return tk_guarded("ie_tokenizer_decode", [&] {
        const std::string s = t->tok.decode(std::vector<int>(ids, ids + n));
        *n_bytes = s.size();
        if (cap) std::memcpy(out, s.data(), std::min(cap, s.size()));
    });
}

extern "C" int ie_tokenizer_vocab_size(const ie_tokenizer* t) { return t ? t->tok.vocab_size() : -1; }

extern "C" int ie_tokenizer_eos_token(const ie_tokenizer* t) { return t ? t->tok.eos_token() : -1; }

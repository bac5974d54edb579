// tokenizer_sanitize.cpp — the tokenizer's C ABI (host/tokenizer.cpp) driven
// over seeded random text, random ids, undersized output buffers and
// malformed vocabulary files.  Built by tests/test_tokenizer_sanitize.py
// with g++'s AddressSanitizer and UndefinedBehaviorSanitizer, so an
// out-of-bounds access, a use after free, a leak or undefined arithmetic
// in the parser, the merge loop or the C ABI's copies ends the run with a
// report.  It also checks the results the C ABI promises:
//   * encode/decode with cap 0 size the output, and a short buffer receives
//     the prefix of the full result with the full count;
//   * with every byte in the vocabulary, decode(encode(t)) is t's words
//     joined by single spaces;
//   * every strict prefix of a valid vocab.json is rejected, and any
//     mutation of it is either accepted or rejected with IE_ERR_INVALID.
// Usage: tokenizer_sanitize <model_dir with vocab.json + merges.txt> <scratch_dir>
#include "ie_tokenizer.h"

#include <climits>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <string>
#include <vector>

// The library's failure sink (defined in csrc/capi.cpp, which is not part
// of this host-only build): keeps the message for the checks below.
namespace ie {
static char g_msg[512];
int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(g_msg, sizeof g_msg, fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace ie

namespace {

uint64_t g_state = 0x9E3779B97F4A7C15ull;
uint32_t next_u32() {  // xorshift64*
    g_state ^= g_state >> 12;
    g_state ^= g_state << 25;
    g_state ^= g_state >> 27;
    return (uint32_t)((g_state * 0x2545F4914F6CDD1Dull) >> 32);
}
uint32_t below(uint32_t n) { return next_u32() % n; }

int g_failures = 0;
#define CHECK(cond, ...)                              \
    do {                                              \
        if (!(cond)) {                                \
            std::fprintf(stderr, "FAIL %s:%d: ", __FILE__, __LINE__); \
            std::fprintf(stderr, __VA_ARGS__);        \
            std::fprintf(stderr, "\n");               \
            if (++g_failures > 20) return 1;          \
        }                                             \
    } while (0)

bool is_space(char c) { return c == ' ' || c == '\t' || c == '\n' || c == '\v' || c == '\f' || c == '\r'; }

std::string random_text() {
    static const char kSpace[] = " \t\n\v\f\r";
    static const char kPunct[] = ",.!?'\"\\/:;-_()[]{}";
    std::string t;
    const uint32_t n = below(8) == 0 ? below(2000) : below(120);
    for (uint32_t i = 0; i < n; ++i) {
        const uint32_t k = below(100);
        if (k < 45) t += (char)('a' + below(16));
        else if (k < 62) t += kSpace[below(6)];
        else if (k < 75) t += (char)(0x80 + below(128));
        else if (k < 85) t += kPunct[below(sizeof kPunct - 1)];
        else if (k < 88) t += '\0';
        else t += (char)(32 + below(95));
    }
    return t;
}

std::string words_joined(const std::string& t) {
    std::string out;
    size_t i = 0;
    while (i < t.size()) {
        while (i < t.size() && is_space(t[i])) ++i;
        if (i == t.size()) break;
        if (!out.empty()) out += ' ';
        while (i < t.size() && !is_space(t[i])) out += t[i++];
    }
    return out;
}

void write_file(const std::string& path, const std::string& s) {
    std::ofstream f(path, std::ios::binary | std::ios::trunc);
    f.write(s.data(), (std::streamsize)s.size());
}

// create over dir; returns the status and destroys the handle on success.
int try_create(const std::string& dir) {
    ie_tokenizer* t = nullptr;
    const int st = ie_tokenizer_create(&t, dir.c_str());
    if (st == IE_OK) ie_tokenizer_destroy(t);
    return st;
}

int fuzz_trained(const std::string& dir) {
    ie_tokenizer* tok = nullptr;
    CHECK(ie_tokenizer_create(&tok, dir.c_str()) == IE_OK, "create: %s", ie::g_msg);
    if (!tok) return 1;
    CHECK(ie_tokenizer_vocab_size(tok) == 50257 && ie_tokenizer_eos_token(tok) == 50256, "table sizes");
    size_t total_ids = 0;
    for (int it = 0; it < 20000; ++it) {
        const std::string text = random_text();
        size_t n = 0;
        CHECK(ie_tokenizer_encode(tok, text.data(), text.size(), nullptr, 0, &n) == IE_OK, "encode sizing");
        std::vector<int> ids(n + 1, -7);
        size_t n2 = 0;
        CHECK(ie_tokenizer_encode(tok, text.data(), text.size(), ids.data(), n, &n2) == IE_OK && n2 == n,
              "encode count %zu vs %zu", n2, n);
        CHECK(ids[n] == -7, "encode wrote past cap");
        if (n > 1) {
            std::vector<int> part(n / 2 + 1, -7);
            size_t n3 = 0;
            CHECK(ie_tokenizer_encode(tok, text.data(), text.size(), part.data(), n / 2, &n3) == IE_OK && n3 == n,
                  "short encode count");
            CHECK(std::memcmp(part.data(), ids.data(), n / 2 * sizeof(int)) == 0 && part[n / 2] == -7,
                  "short encode prefix");
        }
        total_ids += n;

        size_t nb = 0;
        CHECK(ie_tokenizer_decode(tok, ids.data(), n, nullptr, 0, &nb) == IE_OK, "decode sizing");
        std::string back(nb + 1, '\x5A');
        size_t nb2 = 0;
        CHECK(ie_tokenizer_decode(tok, ids.data(), n, &back[0], nb, &nb2) == IE_OK && nb2 == nb, "decode count");
        CHECK(back[nb] == '\x5A', "decode wrote past cap");
        back.resize(nb);
        CHECK(back == words_joined(text), "round trip of a %zu-byte text", text.size());
        if (nb > 1) {
            std::string part(nb / 2 + 1, '\x5A');
            size_t nb3 = 0;
            CHECK(ie_tokenizer_decode(tok, ids.data(), n, &part[0], nb / 2, &nb3) == IE_OK && nb3 == nb,
                  "short decode count");
            CHECK(part.compare(0, nb / 2, back, 0, nb / 2) == 0 && part[nb / 2] == '\x5A', "short decode prefix");
        }

        // arbitrary ids, including negative and past the table
        std::vector<int> junk(below(64));
        for (int& v : junk) {
            const uint32_t k = below(10);
            v = k == 0 ? INT_MIN : k == 1 ? INT_MAX : k == 2 ? -(int)below(100) : (int)below(70000);
        }
        size_t nj = 0;
        CHECK(ie_tokenizer_decode(tok, junk.data(), junk.size(), nullptr, 0, &nj) == IE_OK, "junk decode");
        std::string jb(nj, '\0');
        CHECK(ie_tokenizer_decode(tok, junk.data(), junk.size(), nj ? &jb[0] : nullptr, nj, &nj) == IE_OK,
              "junk decode copy");
    }
    CHECK(total_ids > 100000, "the texts produced only %zu ids", total_ids);
    ie_tokenizer_destroy(tok);
    return 0;
}

int fuzz_files(const std::string& dir) {
    // A valid vocabulary with every escape form the reader handles: \uXXXX,
    // a surrogate pair, a lone high surrogate before another escape, and
    // the short escapes.
    const std::string valid =
        "{\"a\": 0, \"\\u00e9t\\u00c9\": 1, \"\\ud83d\\ude00\": 2, \"\\ud800\\n\": 3, "
        "\"q\\\"\\\\\\/\\b\\f\\r\\t\": 4, \"\\ud800\": 50256, \"big\": 2147483647}";
    const std::string vocab = dir + "/vocab.json", merges = dir + "/merges.txt";
    write_file(merges, "#version: 0.2\na b\n\nnospace\n# c d\n\xc4\xa0 a\nlast pair");
    write_file(vocab, valid);
    CHECK(try_create(dir) == IE_OK, "valid vocabulary rejected: %s", ie::g_msg);
    for (size_t cut = 0; cut < valid.size(); ++cut) {
        write_file(vocab, valid.substr(0, cut));
        CHECK(try_create(dir) == IE_ERR_INVALID, "prefix of %zu bytes accepted", cut);
    }
    for (int it = 0; it < 4000; ++it) {
        std::string m = valid;
        for (uint32_t e = 0, ne = 1 + below(4); e < ne; ++e) {
            const size_t at = below((uint32_t)m.size());
            switch (below(3)) {
                case 0: m[at] = (char)below(256); break;
                case 1: m.erase(at, 1 + below(3)); break;
                default: m.insert(at, 1, "\\u\"{}:,0123456789dD8e"[below(21)]); break;
            }
            if (m.empty()) break;
        }
        write_file(vocab, m);
        const int st = try_create(dir);
        CHECK(st == IE_OK || st == IE_ERR_INVALID, "mutation gave status %d", st);
    }
    for (const char* bad : {"", "{", "{\"", "{\"a\"", "{\"a\":", "{\"a\": 2147483648}", "{\"\\u12\": 1}",
                            "{\"a\": 1}}x", "[]", "{\"a\": 1,}", "\xff\xfe{}"}) {
        write_file(vocab, bad);
        const int st = try_create(dir);
        CHECK(st == IE_ERR_INVALID || std::strcmp(bad, "{\"a\": 1}}x") == 0, "accepted '%s'", bad);
    }
    // merges.txt of random bytes: always accepted, never read out of bounds
    write_file(vocab, valid);
    for (int it = 0; it < 300; ++it) {
        std::string m(below(400), '\0');
        for (char& c : m) c = below(4) == 0 ? '\n' : below(4) == 0 ? ' ' : (char)below(256);
        write_file(merges, m);
        CHECK(try_create(dir) == IE_OK, "merges.txt rejected: %s", ie::g_msg);
    }
    return 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 3) {
        std::fprintf(stderr, "usage: %s <model_dir> <scratch_dir>\n", argv[0]);
        return 2;
    }
    if (fuzz_trained(argv[1]) || fuzz_files(argv[2]) || g_failures) return 1;
    std::printf("tokenizer_sanitize: ok\n");
    return 0;
}

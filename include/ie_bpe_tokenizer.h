/*
 * ie_bpe_tokenizer.h — GPT-2 byte-level BPE tokenizer (C++; C ABI in
 * ie_tokenizer.h).  Same class name, methods and results as the reference's
 * BPETokenizer (include/tokenizer.h:7-25), except that a missing or malformed
 * file throws std::runtime_error instead of exiting the process, and
 * vocab.json is read as JSON: keys ending in an escaped backslash and
 * surrogate-pair escapes are decoded as JSON defines them.
 */
#ifndef IE_BPE_TOKENIZER_H
#define IE_BPE_TOKENIZER_H

#include <array>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

class BPETokenizer {
public:
    explicit BPETokenizer(const std::string& model_dir);

    std::vector<int> encode(const std::string& text) const;
    std::string decode(int token_id) const;
    std::string decode(const std::vector<int>& token_ids) const;

    int vocab_size() const { return (int)id_to_token_.size(); }
    int eos_token() const { return 50256; }

private:
    struct PairHash {
        size_t operator()(const std::pair<std::string, std::string>& p) const;
    };
    std::unordered_map<std::string, int> token_to_id_;
    std::vector<std::string> id_to_token_;
    std::unordered_map<std::pair<std::string, std::string>, int, PairHash> rank_;
    std::array<std::string, 256> byte_sym_;          // byte -> its one-character symbol (UTF-8)
    std::unordered_map<std::string, unsigned char> sym_byte_;  // and back

    std::vector<std::string> merge(std::vector<std::string> syms) const;
};

#endif /* IE_BPE_TOKENIZER_H */

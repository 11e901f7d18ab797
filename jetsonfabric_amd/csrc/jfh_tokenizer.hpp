// Byte-level BPE tokenizer of a Qwen2 GGUF vocabulary, the tokenizer the
// reference serves native packages with (LlamaCppTokenizer,
// runtime/adapters/llama_cpp_tokenizer.{hpp,cpp}, which loads llama.cpp's
// llama_vocab from the package's preserved metadata.gguf). llama.cpp is not
// vendored in the reference, so this restates the published algorithm of
// its BPE vocabulary for the "gpt2" tokenizer model with the "qwen2"
// pre-tokenizer:
//   tokenize(text)  = llama_vocab::tokenize(text, add_special = true,
//                     parse_special = true): control / user-defined tokens
//                     split out of the text first (longest text first), the
//                     rest pre-tokenized by the Qwen2 regex, each piece's
//                     bytes mapped to GPT-2 byte characters and merged by
//                     merge rank (lowest first, leftmost on ties); BOS / EOS
//                     added when the metadata asks for them;
//   token_piece(id) = token_to_piece(id, lstrip 0, special = true);
//   is_end_token    = id == -1 or an end-of-generation id (EOS, EOT, EOM,
//                     FIM pad / repo / separator and the end texts llama.cpp
//                     recognises).
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <string_view>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "jfh_runtime.hpp"

namespace jfh::runtime::tokenization {

class BpeTokenizer final : public Tokenizer {
public:
    // GGUF token types (tokenizer.ggml.token_type).
    enum TokenType : int32_t { kNormal = 1, kUnknown = 2, kControl = 3, kUserDefined = 4, kUnused = 5, kByte = 6 };

    // From GGUF metadata bytes (a package's metadata.gguf or a GGUF file's
    // header). Throws jfh::Error(FormatError) when the metadata holds no
    // byte-level BPE vocabulary.
    static std::shared_ptr<const BpeTokenizer> from_gguf(const uint8_t* data, size_t size);
    // A package directory (its metadata.gguf) or a GGUF file.
    static std::shared_ptr<const BpeTokenizer> open(const std::string& path);

    std::vector<std::int32_t> tokenize(std::string_view text) const override;
    std::string token_piece(std::int32_t token) const override;
    bool is_end_token(std::int32_t token) const override;

    std::vector<std::int32_t> encode(std::string_view text, bool add_special, bool parse_special) const;
    std::vector<std::int32_t> end_tokens() const;
    size_t vocab_size() const { return tokens_.size(); }

    // Pre-tokenizer pieces of text without special tokens, as byte ranges.
    std::vector<std::string> pre_tokenize(std::string_view text) const;

private:
    BpeTokenizer() = default;
    void bpe(const std::string& piece, std::vector<std::int32_t>& out) const;
    int32_t rank(const std::string& left, const std::string& right) const;

    std::vector<std::string> tokens_;
    std::vector<int32_t> types_;
    std::unordered_map<std::string, int32_t> text_to_id_;
    std::unordered_map<std::string, int32_t> merge_rank_;  // "left right" -> rank
    std::vector<int32_t> specials_;                        // control / user-defined / unknown, longest text first
    std::unordered_set<int32_t> end_;
    int32_t bos_ = -1, eos_ = -1;
    bool add_bos_ = false, add_eos_ = false;
};

}  // namespace jfh::runtime::tokenization

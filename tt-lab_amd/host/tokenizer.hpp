// ttlab::Tokenizer -- gpt-oss text <-> token ids, from a GGUF file's tokenizer.ggml.*
// metadata, with the behaviour of the reference's Tokenizer (tokenizer.h:15-34,
// tokenizer.cpp:273-406):
//
//  - only the byte-level BPE with the "gpt-4o" pre-tokenizer (tokenizer.ggml.model
//    "gpt2", tokenizer.ggml.pre "gpt-4o") is accepted;
//  - tokens whose tokenizer.ggml.token_type is not 1 (normal) are special: encode()
//    matches them anywhere in the text, the earliest first and the longest of those
//    starting there, and encodes the text between them as ordinary text;
//  - ordinary text is cut into pieces by the gpt-4o pattern as the reference
//    approximates it (libc wide-character classes for letters, digits and space under
//    the process's LC_CTYPE locale, which the constructor sets from the environment as
//    the reference does; ASCII-only case boundaries; contractions 's 't 're 've 'm 'll
//    'd of up to two ASCII letters after the apostrophe); each piece's bytes, as GPT-2's
//    printable byte characters, are merged pair by pair in merge-rank order (the lowest
//    rank first, the leftmost pair on equal ranks) and looked up in the vocabulary;
//  - decode_to() writes a token's bytes: a special token's text (or nothing), an
//    ordinary token's printable characters mapped back to bytes.
// Errors are std::runtime_error with the reference's messages.  Host code only.
#pragma once

#include "gguf.hpp"

#include <array>
#include <cstddef>
#include <cstdint>
#include <string>
#include <string_view>
#include <unordered_map>
#include <vector>

namespace ttlab {

class Tokenizer {
  public:
    explicit Tokenizer(const GgufFile &file);

    std::vector<int32_t> encode(std::string_view text) const;
    // Bytes of `token` into output[0, capacity); returns how many were written.
    size_t decode_to(int32_t token, char *output, size_t capacity, bool render_special = true) const;
    size_t vocabulary_size() const {
        return vocabulary_.size();
    }

  private:
    void encode_text(std::string_view text, std::vector<int32_t> &output) const;
    void encode_piece(std::string_view piece, std::vector<int32_t> &output) const;

    std::vector<std::string_view> vocabulary_;  // id -> printable-byte text (views into the file)
    std::vector<int32_t> kinds_;                // id -> tokenizer.ggml.token_type
    std::unordered_map<std::string_view, int32_t> ids_;    // text -> the first id holding it
    std::unordered_map<std::string, int32_t> merge_rank_;  // "left right" -> the first rank
    struct Special {
        std::string_view text;
        int32_t id;
    };
    std::vector<Special> specials_;
    std::array<int16_t, 512> byte_of_char_{};  // printable character -> byte, -1 if none
};

// The cuts of the gpt-4o pre-tokenizer (as the reference approximates its pattern,
// tokenizer.cpp:112-237) over `text`: views into it, in order, covering it.
std::vector<std::string_view> pretokenize(std::string_view text);

// The Harmony chat template of one user turn (tokenizer.cpp:404-406).
std::string harmony_prompt(std::string_view user_prompt);

}  // namespace ttlab

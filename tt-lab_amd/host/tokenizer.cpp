// gpt-oss tokenizer (see tokenizer.hpp).
//
// Design: the text is decoded once into code points, each tagged with its libc
// classes; a scanner then walks them and cuts pieces, one method per alternative of
// the gpt-4o pattern in the order the reference tries them (tokenizer.cpp:112-237).
// BPE works on one piece at a time as a list of cut positions in the piece's
// printable-byte text: merging a pair removes the cut between them, so no symbol is
// copied until the final vocabulary lookups.  Special tokens are searched for
// directly in the text; the reference's sorted candidate scan picks the same one (the
// earliest, then the longest).
#include "tokenizer.hpp"

#include <clocale>
#include <cstring>
#include <cwctype>
#include <limits>
#include <stdexcept>

namespace ttlab {
namespace {

constexpr uint32_t kReplacement = 0xfffd;
constexpr int32_t kNormalToken = 1;  // tokenizer.ggml.token_type of an ordinary token

[[noreturn]] void fail(const char *message) {
    throw std::runtime_error(message);
}

// The UTF-8 encoding of code point `cp` (< 2^21).
void put_utf8(std::string &out, uint32_t cp) {
    const int n = cp < 0x80 ? 1 : cp < 0x800 ? 2 : cp < 0x10000 ? 3 : 4;
    if (n == 1) {
        out.push_back(char(cp));
        return;
    }
    static constexpr uint8_t lead[5] = {0, 0, 0xc0, 0xe0, 0xf0};
    char bytes[4];
    for (int k = n - 1; k > 0; --k) {
        bytes[k] = char(0x80 | (cp & 0x3f));
        cp >>= 6;
    }
    bytes[0] = char(lead[n] | cp);
    out.append(bytes, size_t(n));
}

// The code point at text[at], advancing `at` past it.  Malformed input reads as the
// reference reads it (tokenizer.cpp:40-70): a stray continuation byte or a lead byte
// of 0xF8 and above is U+FFFD and takes one byte; a sequence cut off by the end of the
// text is U+FFFD and takes the rest; a sequence broken by a byte that is not a
// continuation is U+FFFD and ends before that byte.
uint32_t take_utf8(std::string_view text, size_t &at) {
    const uint8_t b0 = uint8_t(text[at++]);
    if (b0 < 0x80) {
        return b0;
    }
    int more;
    uint32_t cp;
    if (b0 >= 0xc0 && b0 < 0xe0) {
        more = 1, cp = b0 & 0x1fu;
    } else if (b0 >= 0xe0 && b0 < 0xf0) {
        more = 2, cp = b0 & 0x0fu;
    } else if (b0 >= 0xf0 && b0 < 0xf8) {
        more = 3, cp = b0 & 0x07u;
    } else {
        return kReplacement;
    }
    if (text.size() - at < size_t(more)) {
        at = text.size();
        return kReplacement;
    }
    for (; more > 0; --more) {
        const uint8_t b = uint8_t(text[at]);
        if ((b & 0xc0) != 0x80) {
            return kReplacement;
        }
        ++at;
        cp = (cp << 6) | (b & 0x3fu);
    }
    return cp;
}

// GPT-2's byte-level alphabet: the bytes '!'..'~', 0xA1..0xAC and 0xAE..0xFF stand for
// the code points of the same value; the other 68 bytes, in increasing order, for
// U+0100, U+0101, ...
struct ByteAlphabet {
    std::array<uint16_t, 256> char_of;
    ByteAlphabet() {
        uint16_t spare = 256;
        for (uint32_t b = 0; b < 256; ++b) {
            const bool printable = (b >= 0x21 && b <= 0x7e) || (b >= 0xa1 && b <= 0xac) || b >= 0xae;
            char_of[b] = printable ? uint16_t(b) : spare++;
        }
    }
};

const ByteAlphabet &alphabet() {
    static const ByteAlphabet table;
    return table;
}

bool ascii_upper(uint32_t c) {
    return c - 'A' < 26u;
}
bool ascii_lower(uint32_t c) {
    return c - 'a' < 26u;
}

// The gpt-4o pre-tokenizer over one stretch of ordinary text.
class Scanner {
  public:
    explicit Scanner(std::string_view text) : text_(text) {
        for (size_t at = 0; at < text.size();) {
            Glyph g;
            g.begin = at;
            g.cp = take_utf8(text, at);
            g.end = at;
            g.classes = classify(g.cp);
            glyphs_.push_back(g);
        }
    }

    std::vector<std::string_view> cut() {
        const size_t n = glyphs_.size();
        size_t i = 0;
        while (i < n) {
            if (digit(i)) {
                i = digit_run(i);
            } else if (cp(i) == ' ' && i + 1 < n && other(i + 1)) {
                i = symbol_run(i, i + 1);  // one ordinary space may lead punctuation
            } else if (letter(i)) {
                i = word_run(i, i);
            } else if (!line_end(i) && !digit(i) && i + 1 < n && letter(i + 1)) {
                i = word_run(i, i + 1);  // one leading character that is not a line end
            } else if (line_end(i) || space(i)) {
                i = space_run(i);
            } else {
                i = symbol_run(i, i + 1);
            }
        }
        return std::move(pieces_);
    }

  private:
    enum : uint8_t { kSpace = 1, kLetter = 2, kDigit = 4 };
    struct Glyph {
        uint32_t cp;
        size_t begin, end;
        uint8_t classes;
    };

    // The libc wide-character classes under the current LC_CTYPE (the reference's
    // is_space / is_letter / is_number); none for values past wchar_t's range.
    static uint8_t classify(uint32_t c) {
        if (c > uint32_t(std::numeric_limits<wchar_t>::max())) {
            return 0;
        }
        const wint_t w = wint_t(c);
        return uint8_t((std::iswspace(w) ? kSpace : 0) | (std::iswalpha(w) ? kLetter : 0) |
                       (std::iswdigit(w) ? kDigit : 0));
    }

    uint32_t cp(size_t i) const {
        return glyphs_[i].cp;
    }
    bool space(size_t i) const {
        return glyphs_[i].classes & kSpace;
    }
    bool letter(size_t i) const {
        return glyphs_[i].classes & kLetter;
    }
    bool digit(size_t i) const {
        return glyphs_[i].classes & kDigit;
    }
    bool other(size_t i) const {
        return !(glyphs_[i].classes & (kSpace | kLetter | kDigit));
    }
    bool line_end(size_t i) const {
        return cp(i) == '\r' || cp(i) == '\n';
    }

    void emit(size_t first, size_t last) {
        pieces_.push_back(text_.substr(glyphs_[first].begin, glyphs_[last - 1].end - glyphs_[first].begin));
    }

    // \p{N}{1,3}
    size_t digit_run(size_t first) {
        size_t j = first + 1;
        while (j < glyphs_.size() && j - first < 3 && digit(j)) {
            ++j;
        }
        emit(first, j);
        return j;
    }

    // [^\s\p{L}\p{N}]+[\r\n/]* from glyph j, the piece starting at `first`
    size_t symbol_run(size_t first, size_t j) {
        const size_t n = glyphs_.size();
        while (j < n && other(j)) {
            ++j;
        }
        while (j < n && (line_end(j) || cp(j) == '/')) {
            ++j;
        }
        emit(first, j);
        return j;
    }

    // A case boundary before glyph `at` of the letter run ending at `end`: lower (or
    // non-ASCII) to ASCII upper, or the last capital of an acronym before lower case.
    bool case_break(size_t at, size_t end) const {
        const bool up_before = ascii_upper(cp(at - 1)), up_here = ascii_upper(cp(at));
        if (up_here && !up_before) {
            return true;
        }
        return up_before && up_here && at + 1 < end && ascii_lower(cp(at + 1));
    }

    // A contraction after the letter run ending at `end`: the apostrophe and at most
    // two ASCII letters, kept if they spell (in any case) s, t, re, ve, m, ll or d.
    size_t contraction_end(size_t end) const {
        const size_t n = glyphs_.size();
        if (!(end + 1 < n && cp(end) == '\'')) {
            return end;
        }
        std::string suffix;
        size_t j = end + 1;
        while (j < n && j < end + 3 && (ascii_upper(cp(j)) || ascii_lower(cp(j)))) {
            suffix.push_back(char(ascii_upper(cp(j)) ? cp(j) + ('a' - 'A') : cp(j)));
            ++j;
        }
        static constexpr const char *kSuffixes[] = {"s", "t", "re", "ve", "m", "ll", "d"};
        for (const char *s : kSuffixes) {
            if (suffix == s) {
                return j;
            }
        }
        return end;
    }

    // A run of letters from `first_letter` (its optional one-glyph prefix at `prefix`),
    // cut at case boundaries; the last part takes a contraction after it.
    size_t word_run(size_t prefix, size_t first_letter) {
        size_t end = first_letter + 1;
        while (end < glyphs_.size() && letter(end)) {
            ++end;
        }
        for (size_t part = first_letter; part < end;) {
            size_t stop = part + 1;
            while (stop < end && !case_break(stop, end)) {
                ++stop;
            }
            const size_t last = stop == end ? contraction_end(end) : stop;
            emit(part == first_letter ? prefix : part, last);
            if (last > end) {
                return last;
            }
            part = stop;
        }
        return end;
    }

    // A run of white space: whole if it holds a line end or ends the text, otherwise
    // without its last space (which then leads the next piece).
    size_t space_run(size_t first) {
        const size_t n = glyphs_.size();
        size_t j = first;
        bool newline = false;
        while (j < n && space(j)) {
            newline = newline || line_end(j);
            ++j;
        }
        if (j == first) {
            j = first + 1;  // a line end outside the space class (no C library has one)
        }
        if (!newline && j < n && j - first > 1) {
            --j;
        }
        emit(first, j);
        return j;
    }

    std::string_view text_;
    std::vector<Glyph> glyphs_;
    std::vector<std::string_view> pieces_;
};

const GgufEntry *array_of(const GgufFile &file, const char *key, GgufKind element) {
    const GgufEntry *e = file.find(key);
    return e && e->kind == GgufKind::array && e->element == element ? e : nullptr;
}

}  // namespace

std::vector<std::string_view> pretokenize(std::string_view text) {
    return Scanner(text).cut();
}

std::string harmony_prompt(std::string_view user_prompt) {
    std::string out = "<|start|>user<|message|>";
    out.append(user_prompt);
    out.append("<|end|><|start|>assistant");
    return out;
}

Tokenizer::Tokenizer(const GgufFile &file) {
    if (file.string("tokenizer.ggml.model") != "gpt2" || file.string("tokenizer.ggml.pre") != "gpt-4o") {
        fail("only the gpt-oss gpt-4o BPE tokenizer is supported");
    }
    const GgufEntry *tokens = array_of(file, "tokenizer.ggml.tokens", GgufKind::string);
    const GgufEntry *types = array_of(file, "tokenizer.ggml.token_type", GgufKind::i32);
    const GgufEntry *merges = array_of(file, "tokenizer.ggml.merges", GgufKind::string);
    if (!tokens || !types || !merges || tokens->count != types->count) {
        fail("invalid tokenizer metadata");
    }
    vocabulary_ = tokens->strings;
    kinds_.resize(vocabulary_.size());
    std::memcpy(kinds_.data(), types->raw, kinds_.size() * sizeof(int32_t));
    ids_.reserve(vocabulary_.size());
    for (size_t id = 0; id < vocabulary_.size(); ++id) {
        ids_.try_emplace(vocabulary_[id], int32_t(id));
    }
    for (size_t id = 0; id < vocabulary_.size(); ++id) {
        if (kinds_[id] != kNormalToken) {
            specials_.push_back({vocabulary_[id], ids_.at(vocabulary_[id])});
        }
    }
    merge_rank_.reserve(merges->strings.size());
    for (size_t rank = 0; rank < merges->strings.size(); ++rank) {
        merge_rank_.try_emplace(std::string(merges->strings[rank]), int32_t(rank));
    }
    byte_of_char_.fill(-1);
    for (uint32_t b = 0; b < 256; ++b) {
        byte_of_char_[alphabet().char_of[b]] = int16_t(b);
    }
    // the letter, digit and space classes follow the environment's locale, as the
    // reference's tokenizer sets it (a process-wide setting)
    std::setlocale(LC_CTYPE, "");
}

std::vector<int32_t> Tokenizer::encode(std::string_view text) const {
    std::vector<int32_t> out;
    for (size_t at = 0; at < text.size();) {
        size_t hit = text.size();
        const Special *next = nullptr;
        for (const Special &s : specials_) {
            const size_t pos = text.find(s.text, at);
            if (pos == std::string_view::npos) {
                continue;
            }
            if (!next || pos < hit || (pos == hit && s.text.size() > next->text.size())) {
                hit = pos;
                next = &s;
            }
        }
        if (hit > at) {
            encode_text(text.substr(at, hit - at), out);
        }
        if (!next || next->text.empty()) {
            break;
        }
        out.push_back(next->id);
        at = hit + next->text.size();
    }
    return out;
}

void Tokenizer::encode_text(std::string_view text, std::vector<int32_t> &output) const {
    for (const std::string_view piece : pretokenize(text)) {
        encode_piece(piece, output);
    }
}

void Tokenizer::encode_piece(std::string_view piece, std::vector<int32_t> &output) const {
    // the piece as printable characters; cuts[k] is where symbol k starts
    std::string chars;
    std::vector<size_t> cuts;
    cuts.reserve(piece.size() + 1);
    for (const char c : piece) {
        cuts.push_back(chars.size());
        put_utf8(chars, alphabet().char_of[uint8_t(c)]);
    }
    cuts.push_back(chars.size());
    const std::string_view all(chars);
    auto symbol = [&](size_t k) { return all.substr(cuts[k], cuts[k + 1] - cuts[k]); };
    std::string pair;
    while (cuts.size() > 2) {
        size_t best = 0;
        int32_t best_rank = std::numeric_limits<int32_t>::max();
        bool found = false;
        for (size_t k = 0; k + 2 < cuts.size(); ++k) {
            pair.assign(symbol(k));
            pair.push_back(' ');
            pair.append(symbol(k + 1));
            const auto it = merge_rank_.find(pair);
            if (it != merge_rank_.end() && it->second < best_rank) {
                best = k;
                best_rank = it->second;
                found = true;
            }
        }
        if (!found) {
            break;
        }
        cuts.erase(cuts.begin() + ptrdiff_t(best + 1));
    }
    for (size_t k = 0; k + 1 < cuts.size(); ++k) {
        const auto it = ids_.find(symbol(k));
        if (it == ids_.end()) {
            fail("tokenizer produced an unknown BPE piece");
        }
        output.push_back(it->second);
    }
}

size_t Tokenizer::decode_to(int32_t token, char *output, size_t capacity, bool render_special) const {
    if (token < 0 || size_t(token) >= vocabulary_.size()) {
        fail("token id is out of range");
    }
    const std::string_view text = vocabulary_[size_t(token)];
    if (kinds_[size_t(token)] != kNormalToken) {
        if (!render_special) {
            return 0;
        }
        if (text.size() > capacity) {
            fail("decoded token buffer is too small");
        }
        std::memcpy(output, text.data(), text.size());
        return text.size();
    }
    size_t written = 0;
    for (size_t at = 0; at < text.size();) {
        const uint32_t c = take_utf8(text, at);
        if (c >= byte_of_char_.size() || byte_of_char_[c] < 0) {
            fail("token contains an invalid byte encoding");
        }
        if (written == capacity) {
            fail("decoded token buffer is too small");
        }
        output[written++] = char(byte_of_char_[c]);
    }
    return written;
}

}  // namespace ttlab

"""CPU restatement of the reference's gpt-oss tokenizer (src/tokenizer.cpp), as the
tokenizer tests' oracle.  TEST INFRASTRUCTURE ONLY: only tests/ imports it, as the
checker of ttlab::Tokenizer (tt-lab_amd/host/tokenizer.cpp); nothing in the product
uses it.

The reference itself cannot be built here: its GgufFile (gguf.cpp:234) calls
tensor_bytes() from tensor.cpp, which neither g++ 11 (_Float16, tensor.cpp:164) nor
AMD clang 22 (x86-64-v4 multiversioning) compiles, and a stand-in for that function
is not an option.  So this restatement is pinned instead by known answers that a
plausible mistake fails (tests/test_tokenizer.py): cuts worked out from the gpt-4o
pattern's alternatives, the BPE's leftmost-merge-then-rescan rule on a table where
merging every occurrence at once gives another result, the earliest-then-longest
special token, GPT-2's byte characters, malformed UTF-8, and byte-exact round trips.

Letters, digits and white space are libc's iswalpha / iswdigit / iswspace under the
LC_CTYPE the environment selects (setlocale(LC_CTYPE, ""), as tokenizer.cpp:305
does), called through ctypes so the classes are the C library's own.
"""
import ctypes
import ctypes.util

_libc = ctypes.CDLL(ctypes.util.find_library("c"))
_libc.setlocale.restype = ctypes.c_char_p
_libc.setlocale.argtypes = [ctypes.c_int, ctypes.c_char_p]
for _name in ("iswspace", "iswalpha", "iswdigit"):
    getattr(_libc, _name).argtypes = [ctypes.c_uint32]
    getattr(_libc, _name).restype = ctypes.c_int
LC_CTYPE = 0  # glibc
WCHAR_MAX = 0x7FFFFFFF  # glibc's wchar_t is a signed 32-bit integer
REPLACEMENT = 0xFFFD


def set_locale_from_environment():
    """tokenizer.cpp:305: std::setlocale(LC_CTYPE, "")."""
    _libc.setlocale(LC_CTYPE, b"")


def next_utf8(data, offset):
    """tokenizer.cpp:40-70: (code point, next offset) of the sequence at `offset`."""
    first = data[offset]
    offset += 1
    if first < 0x80:
        return first, offset
    if first & 0xE0 == 0xC0:
        extra, value = 1, first & 0x1F
    elif first & 0xF0 == 0xE0:
        extra, value = 2, first & 0x0F
    elif first & 0xF8 == 0xF0:
        extra, value = 3, first & 0x07
    else:
        return REPLACEMENT, offset
    if offset + extra > len(data):
        return REPLACEMENT, len(data)
    for _ in range(extra):
        byte = data[offset]
        if byte & 0xC0 != 0x80:
            return REPLACEMENT, offset
        offset += 1
        value = (value << 6) | (byte & 0x3F)
    return value, offset


def is_space(c):  # tokenizer.cpp:80-82
    return c <= WCHAR_MAX and _libc.iswspace(c) != 0


def is_letter(c):  # tokenizer.cpp:84-86
    return c <= WCHAR_MAX and _libc.iswalpha(c) != 0


def is_number(c):  # tokenizer.cpp:88-90
    return c <= WCHAR_MAX and _libc.iswdigit(c) != 0


def ascii_upper(c):  # tokenizer.cpp:73-75
    return ord("A") <= c <= ord("Z")


def ascii_lower(c):  # tokenizer.cpp:76-78
    return ord("a") <= c <= ord("z")


def characters(data):
    """tokenizer.cpp:98-106: (code point, begin, end) of each character."""
    out, offset = [], 0
    while offset < len(data):
        begin = offset
        cp, offset = next_utf8(data, offset)
        out.append((cp, begin, offset))
    return out


def split_gpt4o(data):
    """tokenizer.cpp:108-237: the pieces (bytes) of ordinary text `data` (bytes)."""
    chars = characters(data)
    n = len(chars)
    words = []

    def cp(k):
        return chars[k][0]

    def emit(first, last):
        words.append(data[chars[first][1]:chars[last - 1][2]])

    def other(k):
        return not is_space(cp(k)) and not is_letter(cp(k)) and not is_number(cp(k))

    i = 0
    while i < n:
        c = cp(i)
        if is_number(c):  # :123-130
            first = i
            i += 1
            while i < n and i - first < 3 and is_number(cp(i)):
                i += 1
            emit(first, i)
            continue
        if c == 0x20 and i + 1 < n and other(i + 1):  # :132-146
            first = i
            i += 1
            while i < n and other(i):
                i += 1
            while i < n and cp(i) in (0x0D, 0x0A, 0x2F):
                i += 1
            emit(first, i)
            continue
        prefix = first_letter = i  # :148-153
        if c not in (0x0D, 0x0A) and not is_letter(c) and not is_number(c) and i + 1 < n and is_letter(cp(i + 1)):
            i += 1
            first_letter = i
        if is_letter(cp(i)):  # :154-205
            end = i + 1
            while end < n and is_letter(cp(end)):
                end += 1
            part = first_letter
            while part < end:
                stop = part + 1
                while stop < end:
                    prev, cur = cp(stop - 1), cp(stop)
                    lower_to_upper = not ascii_upper(prev) and ascii_upper(cur)
                    acronym = ascii_upper(prev) and ascii_upper(cur) and stop + 1 < end and ascii_lower(cp(stop + 1))
                    if lower_to_upper or acronym:
                        break
                    stop += 1
                output_first = prefix if part == first_letter else part
                output_end = stop
                if stop == end and end < n and cp(end) == 0x27 and end + 1 < n:  # :179-195
                    ce = end + 1
                    while ce < n and ce < end + 3 and (ascii_upper(cp(ce)) or ascii_lower(cp(ce))):
                        ce += 1
                    suffix = "".join(chr(cp(k)).lower() for k in range(end + 1, ce))
                    if suffix in ("s", "t", "re", "ve", "m", "ll", "d"):
                        output_end = ce
                emit(output_first, output_end)
                part = stop
                if output_end > end:
                    end = output_end
                    part = end
            i = end
            continue
        if c in (0x0D, 0x0A) or is_space(c):  # :207-224
            first = i
            newline = False
            while i < n and is_space(cp(i)):
                newline = newline or cp(i) in (0x0D, 0x0A)
                i += 1
            if not newline and i < n and i - first > 1:
                emit(first, i - 1)
                i -= 1
            else:
                emit(first, i)
            continue
        first = i  # :226-235
        i += 1
        while i < n and other(i):
            i += 1
        while i < n and cp(i) in (0x0D, 0x0A, 0x2F):
            i += 1
        emit(first, i)
    return words


def byte_codepoint(byte):
    """tokenizer.cpp:239-250: GPT-2's printable stand-in for a byte."""
    def printable(b):
        return 0x21 <= b <= 0x7E or 0xA1 <= b <= 0xAC or b >= 0xAE
    if printable(byte):
        return byte
    return 256 + sum(1 for b in range(byte) if not printable(b))


def byte_encode(data):
    """tokenizer.cpp:252-259."""
    return "".join(chr(byte_codepoint(b)) for b in data)


class Tokenizer:
    """tokenizer.cpp:273-401 over the metadata lists of tokenizer.ggml.tokens (str),
    tokenizer.ggml.token_type (int) and tokenizer.ggml.merges (str "left right")."""

    def __init__(self, tokens, types, merges, model="gpt2", pre="gpt-4o"):
        if model != "gpt2" or pre != "gpt-4o":  # :274-276
            raise ValueError("only the gpt-oss gpt-4o BPE tokenizer is supported")
        if len(tokens) != len(types):  # :280-285
            raise ValueError("invalid tokenizer metadata")
        self.tokens, self.types = list(tokens), list(types)
        self.ids = {}
        for i, t in enumerate(self.tokens):  # :288-297: the first id of a text wins
            self.ids.setdefault(t, i)
        self.specials = sorted((t for t, k in zip(self.tokens, self.types) if k != 1), key=len, reverse=True)
        self.ranks = {}
        for i, m in enumerate(merges):  # :299-302
            self.ranks.setdefault(m, i)
        self.byte_of = {byte_codepoint(b): b for b in range(256)}  # :303-311
        set_locale_from_environment()

    def encode(self, data):
        """:308-331 (bytes in, ids out)."""
        out, offset = [], 0
        while offset < len(data):
            special_at, special = len(data), b""
            for cand in self.specials:
                c = cand.encode()
                found = data.find(c, offset)
                if 0 <= found < special_at:
                    special_at, special = found, c
            if special_at > offset:
                for word in split_gpt4o(data[offset:special_at]):
                    out += self.encode_word(word)
            if not special:
                break
            out.append(self.ids[special.decode()])
            offset = special_at + len(special)
        return out

    def encode_word(self, word):
        """:346-368: the lowest-ranked adjacent pair merged, the leftmost on equal ranks,
        then the pairs looked at again."""
        symbols = list(byte_encode(word))
        while len(symbols) > 1:
            best, best_rank = None, None
            for i in range(len(symbols) - 1):
                r = self.ranks.get(symbols[i] + " " + symbols[i + 1])
                if r is not None and (best_rank is None or r < best_rank):
                    best, best_rank = i, r
            if best is None:
                break
            symbols[best:best + 2] = [symbols[best] + symbols[best + 1]]
        out = []
        for s in symbols:
            if s not in self.ids:
                raise ValueError("tokenizer produced an unknown BPE piece")
            out.append(self.ids[s])
        return out

    def decode(self, token, render_special=True, capacity=1024):
        """:370-401: the bytes of `token`."""
        if token < 0 or token >= len(self.tokens):
            raise ValueError("token id is out of range")
        text = self.tokens[token]
        if self.types[token] != 1:
            if not render_special:
                return b""
            raw = text.encode()
            if len(raw) > capacity:
                raise ValueError("decoded token buffer is too small")
            return raw
        out = bytearray()
        for ch in text:
            b = self.byte_of.get(ord(ch))
            if b is None:
                raise ValueError("token contains an invalid byte encoding")
            if len(out) == capacity:
                raise ValueError("decoded token buffer is too small")
            out.append(b)
        return bytes(out)


def harmony_prompt(user):
    """tokenizer.cpp:404-406 (bytes in and out)."""
    return b"<|start|>user<|message|>" + user + b"<|end|><|start|>assistant"

"""ttlab::Tokenizer (tt-lab_amd/host/tokenizer.{hpp,cpp}) against the oracle's restatement
of the reference's Tokenizer (oracle/tokenizer_oracle.py, tokenizer.cpp:40-406) on
synthetic GGUF vocabularies: token ids of encode(), bytes of decode_to() for every id,
the Harmony template and the error messages, equal in the UTF-8 and the C locale.  The
reference's own tokenizer cannot be built here (its GgufFile needs tensor.cpp, which
this image's compilers reject), so the oracle is pinned by known answers that a
plausible mistake fails, and both implementations are checked against them: cuts
worked out from the gpt-4o pattern as the reference approximates it
(tokenizer.cpp:112-237), the BPE's leftmost-merge-then-rescan rule (tokenizer.cpp:346-368)
on a merge table where merging every occurrence at once gives another result, the
earliest-then-longest special token (:308-331), GPT-2's byte characters (:239-250),
malformed UTF-8 (:40-70), and byte-exact round trips.  No GPU.

The vocabularies: the 256 byte tokens (GPT-2's printable byte characters), merges
learned by a small greedy BPE over raw sample text (pairs across letters, digits,
spaces, punctuation and line ends, so merges that a wrong cut would let through exist),
their merged tokens, and special tokens of type 3 (one the prefix of another).
"""
import os
import random
import sys

import pytest

import ttlab_amd
from gguf_writer import ARRAY, I32, STRING, write_gguf

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import tokenizer_oracle as T  # noqa: E402

SPECIALS = ["<|start|>", "<|end|>", "<|message|>", "<|channel|>", "<|return|>", "<|endoftext|>", "<|ab|>",
            "<|ab|>c"]


def byte_chars():
    """GPT-2's printable stand-in for each byte (the alphabet the vocabulary is written in)."""
    out, spare = [], 256
    for b in range(256):
        if 0x21 <= b <= 0x7e or 0xa1 <= b <= 0xac or b >= 0xae:
            out.append(chr(b))
        else:
            out.append(chr(spare))
            spare += 1
    return out


CORPUS = (
    "Hello world! I'm here, you're there; they'll go. We've done it, he'd say. DON'T SHOUT.\n"
    "The HTTPServer parses JSONData and XMLHttpRequest; iPhone users ABCdef.\n\n"
    "Numbers: 12345 678 9 3.14159 2,718 100% 007 x2 y10z\r\n"
    "Paths like /usr/local/bin and C:\\\\tmp\\\\x, URLs http://a.b/c?d=e&f=g#h.\n"
    "  indented   spaces\tand\ttabs \t mixed  \n   \n"
    "Quotes 'single' \"double\" `back` (parens) [brackets] {braces} <angles> ... --- *** !!!\n"
    "naïve café résumé Ünïcödé Ελληνικά русский язык 日本語テキスト 한국어 العربية עברית\n"
    "emoji 😀👍🏽 🚀 mixed with text\n"
    "def f(x): return x**2 + 3*x - 1  # code\n"
    "<|start|>user<|message|>What is 2+2?<|end|><|start|>assistant\n"
)


def train_merges(corpus, count):
    """Greedy BPE over the raw corpus (no pre-split): the most frequent adjacent pair,
    first seen first on ties, merged `count` times (pairs seen once too, so long merges
    across the pattern's cuts exist)."""
    alpha = byte_chars()
    seq = [alpha[b] for b in corpus.encode()]
    merges = []
    for _ in range(count):
        freq, first = {}, {}
        for i in range(len(seq) - 1):
            p = (seq[i], seq[i + 1])
            freq[p] = freq.get(p, 0) + 1
            first.setdefault(p, i)
        if not freq:
            break
        best = max(freq, key=lambda p: (freq[p], -first[p]))
        merges.append(best)
        out, i = [], 0
        while i < len(seq):
            if i + 1 < len(seq) and (seq[i], seq[i + 1]) == best:
                out.append(seq[i] + seq[i + 1])
                i += 2
            else:
                out.append(seq[i])
                i += 1
        seq = out
    return merges


def write_tokenizer(path, merges, model="gpt2", pre="gpt-4o", drop=(), extra_tokens=(), extra_merges=()):
    tokens = list(byte_chars())
    types = [1] * len(tokens)
    seen = set(tokens)
    for a, b in merges:
        t = a + b
        if t not in seen:
            seen.add(t)
            tokens.append(t)
            types.append(1)
    for t, kind in extra_tokens:
        tokens.append(t)
        types.append(kind)
    for s in SPECIALS:
        tokens.append(s)
        types.append(3)
    md = [("general.architecture", STRING, "gpt-oss"),
          ("tokenizer.ggml.model", STRING, model),
          ("tokenizer.ggml.pre", STRING, pre),
          ("tokenizer.ggml.tokens", ARRAY, (STRING, tokens)),
          ("tokenizer.ggml.token_type", ARRAY, (I32, types)),
          ("tokenizer.ggml.merges", ARRAY, (STRING, [f"{a} {b}" for a, b in merges] + list(extra_merges)))]
    write_gguf(path, [m for m in md if m[0] not in drop], [])
    return tokens, types, [f"{a} {b}" for a, b in merges] + list(extra_merges)


class OracleTokenizer:
    """The oracle's restatement with the interface of ttlab_amd.Tokenizer (bytes in)."""

    def __init__(self, lists):
        self.t = T.Tokenizer(*lists)

    def encode(self, data):
        return self.t.encode(data)

    def decode(self, token, render_special=True, capacity=1024):
        return self.t.decode(token, render_special, capacity)

    def close(self):
        pass


@pytest.fixture(scope="module")
def vocab(tmp_path_factory):
    path = str(tmp_path_factory.mktemp("tok") / "tok.gguf")
    merges = train_merges(CORPUS, 600)
    # a normal token that repeats a merged token (the first id keeps the text), a merge
    # listed twice (the first rank counts), a user-defined special (type 4)
    dup = merges[3][0] + merges[3][1]
    lists = write_tokenizer(path, merges, extra_tokens=[(dup, 1), ("<|user-defined|>", 4)],
                            extra_merges=[f"{merges[0][0]} {merges[0][1]}"])
    return path, lists


@pytest.fixture(params=["C.UTF-8", "C"])
def locale_env(request):
    old = os.environ.get("LC_ALL")
    os.environ["LC_ALL"] = request.param
    yield request.param
    if old is None:
        os.environ.pop("LC_ALL", None)
    else:
        os.environ["LC_ALL"] = old


TEXTS = [
    "", "a", " ", "Hello world", "Hello, world!", "I'm here, you're there; they'll go.",
    "We've done it. He'd say 'DON'T' shouldn't", "it's IT'S It'S it'sa don'", "o'clock rock'n'roll",
    "HTTPServer parseJSON XMLHttpRequest iPhone ABCdef aBC ABc", "CamelCaseWordsAndACRONYMSHere",
    "12345 678 9 0.5e10 3,141 1234567", "x2y10z 2x", "  leading spaces", "trailing   ", "a  b   c",
    "a\n\nb\r\n c", "line\n  indented", "  \n  x", "\n", "\r\n\r\n", "tabs\t\tand\tmore\t",
    "punct!!! ... ?!? (x) [y] {z}", " !!", "!! ", "foo/bar//baz\n/", "a.\n/b", "<|not special",
    "naïve café Ünïcödé Ελληνικά русский 日本語 한국어 العربية", "Élan ÉCOLE éA aÉ",
    "emoji 😀👍🏽 mixed", " 'quoted' ", "\"double\" `back`", "x = y ** 2 # c", "C:\\tmp\\x",
    "<|start|>user<|message|>hi<|end|><|start|>assistant", "<|ab|>c<|ab|><|ab|>cc", "a<|end|>b<|return|>",
    "<|start|><|start|>", "<|user-defined|>text", "<|end|",
]


def fuzz_texts(seed, count):
    rng = random.Random(seed)
    atoms = list("abcxyzABCXYZ0123456789 \t\n\r'.,/!?-_()éÉΩω日本😀") + ["'s", "'LL", "<|end|>", "<|ab|>", "  ",
                                                                        "\r\n", "HTTP", "Server"]
    return ["".join(rng.choice(atoms) for _ in range(rng.randint(0, 30))) for _ in range(count)]


def test_encode_matches_oracle(vocab, locale_env):
    path, lists = vocab
    mine = ttlab_amd.Tokenizer(path)  # each constructor sets LC_CTYPE from the environment
    ref = OracleTokenizer(lists)
    texts = [t.encode() for t in TEXTS + fuzz_texts(0x70C, 400)]
    texts += [b"\xff\xfe abc \xc3(", b"\xe6\x97", b"trunc \xf0\x9f\x98", b"\x80\x80x", b"\xc3\xa9\xc3"]
    merged = 0
    try:
        for data in texts:
            got, want = mine.encode(data), ref.encode(data)
            assert got == want, (locale_env, data, got, want)
            merged += sum(1 for t in got if t >= 256)
            # byte-level BPE loses nothing: the ids decode to the input bytes
            assert b"".join(mine.decode(t) for t in got) == data
    finally:
        mine.close()
    assert merged > 200  # the merges apply (not a byte-per-token check)


def test_decode_matches_oracle_for_every_token(vocab):
    path, lists = vocab
    mine, ref = ttlab_amd.Tokenizer(path), OracleTokenizer(lists)
    try:
        n = mine.vocabulary()
        assert n == len(lists[0]) > 256 + len(SPECIALS)
        for token in range(n):
            for special in (True, False):
                assert mine.decode(token, special) == ref.decode(token, special), token
        for token in (-1, n, n + 100):
            with pytest.raises(ttlab_amd.TtlError, match="token id is out of range"):
                mine.decode(token)
            with pytest.raises(ValueError, match="token id is out of range"):
                ref.decode(token)
        ordinary = max(range(256, n - len(SPECIALS) - 2), key=lambda t: len(ref.decode(t)))
        for t in (ordinary, n - 1):  # an ordinary token of several bytes, a special token
            with pytest.raises(ttlab_amd.TtlError, match="decoded token buffer is too small"):
                mine.decode(t, True, capacity=1)
            with pytest.raises(ValueError, match="decoded token buffer is too small"):
                ref.decode(t, True, capacity=1)
    finally:
        mine.close()


def test_harmony_prompt():
    """tokenizer.cpp:404-406, and the oracle's restatement of it."""
    for user in ("What is 2+2?", "", "multi\nline <|end|> text", "ünï"):
        want = ("<|start|>user<|message|>" + user + "<|end|><|start|>assistant").encode()
        assert ttlab_amd.harmony_prompt(user) == want == T.harmony_prompt(user.encode())


def test_constructor_errors_carry_the_reference_messages(tmp_path):
    merges = train_merges("abab abab cdcd", 4)
    cases = {
        "model": (dict(model="llama"), "only the gpt-oss gpt-4o BPE tokenizer is supported"),
        "pre": (dict(pre="gpt2"), "only the gpt-oss gpt-4o BPE tokenizer is supported"),
        "merges": (dict(drop=("tokenizer.ggml.merges",)), "invalid tokenizer metadata"),
        "types": (dict(drop=("tokenizer.ggml.token_type",)), "invalid tokenizer metadata"),
        "missing-model": (dict(drop=("tokenizer.ggml.model",)), "missing GGUF key: tokenizer.ggml.model"),
    }
    for name, (kw, message) in cases.items():
        path = str(tmp_path / f"{name}.gguf")
        write_tokenizer(path, merges, **kw)
        with pytest.raises(ttlab_amd.TtlError, match=message):
            ttlab_amd.Tokenizer(path)


def test_unknown_piece_error(tmp_path):
    """A merge whose result is not in the vocabulary throws on the piece (tokenizer.cpp:362-366)."""
    path = str(tmp_path / "gap.gguf")
    alpha = byte_chars()
    lists = write_tokenizer(path, [], extra_merges=[f"{alpha[ord('q')]} {alpha[ord('z')]}"])
    mine, ref = ttlab_amd.Tokenizer(path), OracleTokenizer(lists)
    try:
        assert mine.encode(b"qa") == ref.encode(b"qa") == [ord("q"), ord("a")]
        with pytest.raises(ValueError, match="tokenizer produced an unknown BPE piece"):
            ref.encode(b"qz")
        with pytest.raises(ttlab_amd.TtlError, match="tokenizer produced an unknown BPE piece"):
            mine.encode(b"qz")
    finally:
        mine.close()


def small_vocab(tmp_path, name, extra, merges):
    """Byte tokens, then `extra` normal tokens (printable-byte text) and merges."""
    alpha = byte_chars()
    tokens = list(alpha) + extra + SPECIALS
    types = [1] * (256 + len(extra)) + [3] * len(SPECIALS)
    md = [("tokenizer.ggml.model", STRING, "gpt2"), ("tokenizer.ggml.pre", STRING, "gpt-4o"),
          ("tokenizer.ggml.tokens", ARRAY, (STRING, tokens)), ("tokenizer.ggml.token_type", ARRAY, (I32, types)),
          ("tokenizer.ggml.merges", ARRAY, (STRING, merges))]
    path = str(tmp_path / name)
    write_gguf(path, md, [])
    return path, (tokens, types, merges)


def test_bpe_merges_the_leftmost_lowest_pair_then_looks_again(tmp_path):
    """tokenizer.cpp:346-368 on tables where the rule decides the result.  With the
    merges ["ab a", "a b"], "abab" merges its first "a b" (rank 1; there is no rank-0
    pair yet), which makes "ab a" (rank 0) -> [aba, b]; merging every "a b" at once
    would give [ab, ab].  With ["a a"], "aaa" -> [aa, a] (the leftmost pair), not [a, aa]."""
    path, lists = small_vocab(tmp_path, "bpe.gguf", ["ab", "aba", "aa"], ["ab a", "a b", "a a"])
    mine, ref = ttlab_amd.Tokenizer(path), OracleTokenizer(lists)
    ab, aba, aa = 256, 257, 258
    try:
        for text, want in ((b"abab", [aba, ord("b")]), (b"aaa", [aa, ord("a")]), (b"aaaa", [aa, aa]),
                           (b"ab", [ab]), (b"ba", [ord("b"), ord("a")])):
            assert ref.encode(text) == want, text
            assert mine.encode(text) == want, text
    finally:
        mine.close()


def test_special_tokens_earliest_then_longest(tmp_path):
    """tokenizer.cpp:308-331: the special found first in the text wins, and of two that
    start there the longer ("<|ab|>c" over "<|ab|>"); text between them is ordinary."""
    path, lists = small_vocab(tmp_path, "sp.gguf", [], [])
    mine, ref = ttlab_amd.Tokenizer(path), OracleTokenizer(lists)
    sid = {s: 256 + k for k, s in enumerate(SPECIALS)}
    try:
        cases = [
            (b"<|ab|>c", [sid["<|ab|>c"]]),
            (b"<|ab|>d", [sid["<|ab|>"], ord("d")]),
            (b"x<|end|>y<|start|>", [ord("x"), sid["<|end|>"], ord("y"), sid["<|start|>"]]),
            (b"<|end|", [ord("<"), ord("|"), ord("e"), ord("n"), ord("d"), ord("|")]),
        ]
        for text, want in cases:
            assert ref.encode(text) == want, text
            assert mine.encode(text) == want, text
    finally:
        mine.close()


def test_byte_characters_and_malformed_utf8():
    """GPT-2's alphabet (tokenizer.cpp:239-250): ' ' is U+0120, '\n' U+010A, 0xAD U+0143,
    printable bytes themselves; UTF-8 read as tokenizer.cpp:40-70 reads it."""
    assert T.byte_codepoint(0x20) == 0x120 and T.byte_codepoint(0x0A) == 0x10A
    assert T.byte_codepoint(0xAD) == 0x143 and T.byte_codepoint(0x41) == 0x41 and T.byte_codepoint(0) == 0x100
    assert sorted(T.byte_codepoint(b) for b in range(256)) == sorted(set(T.byte_codepoint(b) for b in range(256)))
    assert byte_chars() == [chr(T.byte_codepoint(b)) for b in range(256)]
    assert T.next_utf8(b"\xc3\xa9", 0) == (0xE9, 2)
    assert T.next_utf8(b"\xf0\x9f\x98\x80", 0) == (0x1F600, 4)
    assert T.next_utf8(b"\xff", 0) == (0xFFFD, 1)          # not a lead byte: one byte
    assert T.next_utf8(b"\x80x", 0) == (0xFFFD, 1)         # a stray continuation byte
    assert T.next_utf8(b"\xe6\x97", 0) == (0xFFFD, 2)      # cut off: the rest of the text
    assert T.next_utf8(b"\xc3(", 0) == (0xFFFD, 1)         # broken: ends before the bad byte
    # the same reading in the product's pre-tokenizer: each malformed sequence is one glyph
    assert ttlab_amd.pretokenize(b"\xff\xfe") == [b"\xff\xfe"]
    assert ttlab_amd.pretokenize(b"\xc3(") == [b"\xc3("]


# Known cuts of the gpt-4o pattern as the reference approximates it (tokenizer.cpp:112-237),
# worked out from its alternatives: \p{N}{1,3}; one space leading punctuation; one
# non-letter, non-line-end character leading a letter run cut at ASCII case boundaries,
# the last part taking 's 't 're 've 'm 'll 'd; white space, whole when it holds a line
# end or ends the text, else without its last space; punctuation with trailing \r \n /.
KNOWN_CUTS = [
    ("Hello world", ["Hello", " world"]),
    ("I'm fine", ["I'm", " fine"]),
    ("they'll", ["they'll"]),
    ("DON'T", ["DON'T"]),
    ("it'sa", ["it", "'sa"]),
    ("HTTPServer", ["HTTP", "Server"]),
    ("parseJSONData", ["parse", "JSON", "Data"]),
    ("iPhone", ["i", "Phone"]),
    ("12345", ["123", "45"]),
    ("x12", ["x", "12"]),
    ("a  b", ["a", " ", " b"]),
    ("a   ", ["a", "   "]),
    ("x\n\ny", ["x", "\n\n", "y"]),
    ("x \n  y", ["x", " \n  ", "y"]),
    ("a, b", ["a", ",", " b"]),
    (" !!", [" !!"]),
    ("!!\n/x", ["!!\n/", "x"]),
    ("(x)", ["(x", ")"]),
    ("\tword", ["\tword"]),
]


def test_pretokenizer_known_cuts():
    for text, cuts in KNOWN_CUTS:
        want = [c.encode() for c in cuts]
        assert ttlab_amd.pretokenize(text) == want, text
        assert T.split_gpt4o(text.encode()) == want, text

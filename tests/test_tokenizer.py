"""BPE tokenizer (rusttorch-core/src/data/tokenizer.rs) behind the C ABI.

1. The reference's own unit tests (tokenizer.rs:517-921), each run against the
   library (rusttorch_amd.tokenizer) and against the Python restatement
   (oracle/tokenizer_ref.py). Tests of the reference's private helpers go
   through the public API where the library does not export them (apply_bpe
   via encode on one-word inputs, parse_vocab_json via from_strings).
2. The Unicode property tables (Alphabetic, White_Space) pinned against
   Perl's Unicode database for every code point.
3. Randomised parity of library and restatement: pre-tokenisation of mixed
   text, encode / decode with a BPE vocabulary trained on a synthetic corpus,
   decode of arbitrary byte sequences (from_utf8_lossy), and parser errors.
No GPU is needed: the tokenizer is host code.
"""
from __future__ import annotations

import json
import random
import shutil
import subprocess

import pytest

from oracle import tokenizer_ref as R
from rusttorch_amd import tokenizer as T
from rusttorch_amd._lib import Gpt2Error


class Impl:
    """One implementation of the reference's tokenizer API, library or oracle."""

    def __init__(self, name):
        self.name = name
        self.m = T if name == "library" else R

    def tok_from_vocab_and_merges(self, vocab, merges):
        return self.m.BpeTokenizer.from_vocab_and_merges(vocab, merges)

    def tok_from_strings(self, v, m):
        return self.m.BpeTokenizer.from_strings(v, m)

    def pre_tokenize(self, text):
        return self.m.pre_tokenize(text)

    def byte_encoder(self):
        return self.m.build_byte_encoder()

    def apply_bpe(self, tok, tokens):
        """apply_bpe on single-character printable tokens of one word."""
        if self.name == "oracle":
            return tok.apply_bpe(tokens)
        word = "".join(tokens)
        assert len(self.pre_tokenize(word)) == 1 and all(len(t) == 1 and "!" <= t <= "~" for t in tokens)
        return [tok.id_to_token(i) for i in tok.encode(word)]

    def parse_vocab(self, js):
        """parse_vocab_json through from_strings: {token: id} of the given keys."""
        if self.name == "oracle":
            return R.parse_vocab_json(js)
        tok = T.BpeTokenizer.from_strings(js, "")
        return tok

    def error_type(self):
        return Gpt2Error if self.name == "library" else R.ParseError


IMPLS = [Impl("library"), Impl("oracle")]
ids = [i.name for i in IMPLS]


# ---- byte encoder (tokenizer.rs:519-566, 883-894) ----

@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_byte_encoder_covers_all_256_bytes(im):
    enc = im.byte_encoder()
    assert "\0" not in enc and len(set(enc)) == 256


@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_byte_encoder_printable_identity(im):
    enc = im.byte_encoder()
    for ch in "Az0!~":
        assert enc[ord(ch)] == ch


@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_byte_encoder_nonprintable_mapped(im):
    enc = im.byte_encoder()
    assert ord(enc[0]) >= 256 and ord(enc[32]) >= 256 and ord(enc[9]) >= 256


@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_byte_encoder_roundtrip(im):
    enc = im.byte_encoder()
    dec = {c: b for b, c in enumerate(enc)}
    assert all(dec[enc[b]] == b for b in range(256))


@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_is_printable_byte(im):
    enc = im.byte_encoder()  # printable bytes are exactly those that map to themselves
    printable = lambda b: enc[b] == chr(b)
    assert printable(ord("A")) and printable(ord("~")) and printable(ord("!"))
    assert not printable(ord(" ")) and not printable(0) and not printable(9) and not printable(10)
    assert not printable(173)


def test_byte_encoder_closed_form():
    """The whole table: printable bytes map to themselves, the others to
    U+0100, U+0101, ... in byte order (tokenizer.rs:223-241)."""
    enc = T.build_byte_encoder()
    nxt = 256
    for b in range(256):
        if 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255:
            assert enc[b] == chr(b)
        else:
            assert enc[b] == chr(nxt)
            nxt += 1
    assert nxt == 256 + 68


# ---- pre-tokenisation (tokenizer.rs:570-618, 873-881, 896-911) ----

PRE_CASES = [
    ("Hello world", ["Hello", " world"]),
    ("Hello, world!", ["Hello", ",", " world", "!"]),
    ("I have 42 cats", ["I", " have", " 42", " cats"]),
    ("I'm don't we'll they've", ["I", "'m", " don", "'t", " we", "'ll", " they", "'ve"]),
    ("Hello! It's 2024.", ["Hello", "!", " It", "'s", " 2024", "."]),
    ("", []),
    ("   ", [" ", " ", " "]),
    ("A", ["A"]),
    (" hello", [" hello"]),
    ("a  b", ["a", " ", " b"]),
    ("'s test", ["'s", " test"]),  # match_contraction(.., 0) == ("'s", 2)
    ("'", ["'"]),                  # no contraction at the end
]


@pytest.mark.parametrize("im", IMPLS, ids=ids)
@pytest.mark.parametrize("text,want", PRE_CASES)
def test_pre_tokenize(im, text, want):
    assert im.pre_tokenize(text) == want


# ---- BPE merges (tokenizer.rs:620-677, 828-845, 889-920) ----

BPE_CASES = [
    (["a", "b", "c"], [], ["a", "b", "c"], ["a", "b", "c"]),
    (["a", "b", "c", "ab"], [("a", "b")], ["a", "b", "c"], ["ab", "c"]),
    (["a", "b", "c", "ab", "abc"], [("a", "b"), ("ab", "c")], ["a", "b", "c"], ["abc"]),
    (["a", "b", "c", "ab", "bc"], [("b", "c"), ("a", "b")], ["a", "b", "c"], ["a", "bc"]),
    (["a"], [("a", "b")], ["a"], ["a"]),
    (["a", "b", "ab"], [("a", "b")], list("aababab"), ["a", "ab", "ab", "ab"]),
    (["a", "b", "c", "d", "ab", "abc", "abcd"], [("a", "b"), ("ab", "c"), ("abc", "d")], list("abcd"), ["abcd"]),
    (["a", "b", "ab", "x"], [("a", "b")], list("abxab"), ["ab", "x", "ab"]),
    # overlapping pairs of one rank: the leftmost merges first ("rank < best_rank", tokenizer.rs:160-167)
    (["a", "aa"], [("a", "a")], list("aaa"), ["aa", "a"]),
    (["a", "b", "aa", "ab"], [("a", "b"), ("a", "a")], list("aaab"), ["aa", "ab"]),
    (["a", "aa", "aaaa"], [("a", "a"), ("aa", "aa")], list("aaaaa"), ["aaaa", "a"]),
]


@pytest.mark.parametrize("im", IMPLS, ids=ids)
@pytest.mark.parametrize("vocab,merges,tokens,want", BPE_CASES)
def test_apply_bpe(im, vocab, merges, tokens, want):
    tok = im.tok_from_vocab_and_merges(vocab, merges)
    assert im.apply_bpe(tok, tokens) == want


# ---- vocab.json / merges.txt (tokenizer.rs:679-752, 905-909) ----

@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_parse_vocab_json(im):
    v = im.parse_vocab('{"hello": 0, "world": 1, "foo": 2}')
    get = (lambda k: v.get(k)) if isinstance(v, dict) else v.token_to_id
    assert (get("hello"), get("world"), get("foo")) == (0, 1, 2)
    assert (len(v) if isinstance(v, dict) else v.vocab_size()) == 3
    v = im.parse_vocab(r'{"\"quoted\"": 0, "back\\slash": 1, "new\nline": 2}')
    get = (lambda k: v.get(k)) if isinstance(v, dict) else v.token_to_id
    assert (get('"quoted"'), get("back\\slash"), get("new\nline")) == (0, 1, 2)
    v = im.parse_vocab(r'{"\\u0120": 0}')
    assert (len(v) if isinstance(v, dict) else v.vocab_size()) == 1
    v = im.parse_vocab("{}")
    assert (len(v) if isinstance(v, dict) else v.vocab_size()) == 0
    v = im.parse_vocab('{"a": 50256, "b": 50257}')
    get = (lambda k: v.get(k)) if isinstance(v, dict) else v.token_to_id
    assert (get("a"), get("b")) == (50256, 50257)
    with pytest.raises(im.error_type()):
        im.parse_vocab("not json")


@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_parse_merges(im):
    """parse_merges: header skipped, ranks in line order, blank lines ignored;
    observed through encode with a vocabulary holding every merge result."""
    vocab = json.dumps({t: i for i, t in enumerate(["a", "b", "c", "d", "e", "f", "ab", "cd", "ef", "abc"])})
    tok = im.tok_from_strings(vocab, "#version: 0.2\na b\nab c\n")
    assert [tok.id_to_token(i) for i in tok.encode("abc")] == ["abc"]
    tok = im.tok_from_strings(vocab, "#version: 0.2\n\na b\n\nc d\n\n")
    assert [tok.id_to_token(i) for i in tok.encode("abcd")] == ["ab", "cd"]
    # rank order: "b c" (line 1) beats "a b" (line 2)
    v2 = json.dumps({t: i for i, t in enumerate(["a", "b", "c", "ab", "bc"])})
    tok = im.tok_from_strings(v2, "#version: 0.2\nb c\na b\n")
    assert [tok.id_to_token(i) for i in tok.encode("abc")] == ["a", "bc"]


# ---- encode / decode (tokenizer.rs:754-827) ----

@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_encode_decode_roundtrip_simple(im):
    enc = im.byte_encoder()
    js = "{" + ", ".join('"%s": %d' % (c.replace("\\", "\\\\").replace('"', '\\"'), i) for i, c in enumerate(enc)) + "}"
    tok = im.tok_from_strings(js, "#version: 0.2\n")
    assert tok.decode(tok.encode("Hi")) == "Hi"


@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_vocab_size_and_lookups(im):
    tok = im.tok_from_vocab_and_merges(["a", "b", "c", "ab"], [("a", "b")])
    assert tok.vocab_size() == 4
    tok = im.tok_from_vocab_and_merges(["hello", "world"], [])
    assert tok.token_to_id("hello") == 0 and tok.token_to_id("world") == 1 and tok.token_to_id("missing") is None
    assert tok.id_to_token(0) == "hello" and tok.id_to_token(1) == "world" and tok.id_to_token(99) is None


@pytest.mark.parametrize("im", IMPLS, ids=ids)
def test_encode_decode_empty(im):
    tok = im.tok_from_vocab_and_merges(["a"], [])
    assert tok.encode("") == [] and tok.decode([]) == ""


def test_from_files(tmp_path):
    with pytest.raises(Gpt2Error, match=r"^Failed to read vocab\.json: No such file or directory \(os error 2\)$"):
        T.BpeTokenizer.from_files(str(tmp_path / "none.json"), str(tmp_path / "none.txt"))
    (tmp_path / "v.json").write_text('{"a": 0, "b": 1, "ab": 2}')
    with pytest.raises(Gpt2Error, match=r"^Failed to read merges\.txt: No such file"):
        T.BpeTokenizer.from_files(str(tmp_path / "v.json"), str(tmp_path / "none.txt"))
    (tmp_path / "m.txt").write_text("#version: 0.2\na b\n")
    tok = T.BpeTokenizer.from_files(str(tmp_path / "v.json"), str(tmp_path / "m.txt"))
    assert tok.encode("ab") == [2] and tok.decode([2, 0]) == "aba"


# ---- Unicode tables against Perl's database ----

@pytest.mark.skipif(shutil.which("perl") is None, reason="perl not available")
def test_unicode_tables_match_perl():
    """Every code point's Alphabetic / White_Space value in unicode_tables.h
    (the tables behind char::is_alphabetic / is_whitespace) equals Perl's."""
    prog = r"""
    my ($na, $nw) = (0, 0); my $out = '';
    for my $c (0 .. 0x10FFFF) { next if $c >= 0xD800 && $c <= 0xDFFF;
      $out .= (chr($c) =~ /\p{Alphabetic}/ ? 'A' : '-') . (chr($c) =~ /\p{White_Space}/ ? 'W' : '-'); }
    print $out;
    """
    out = subprocess.run(["perl", "-e", prog], check=True, capture_output=True, text=True).stdout
    k = 0
    for c in range(0x110000):
        if 0xD800 <= c <= 0xDFFF:
            continue
        a, w = out[2 * k] == "A", out[2 * k + 1] == "W"
        k += 1
        if a != R.is_alphabetic(chr(c)) or w != R.is_whitespace(chr(c)):
            pytest.fail(f"U+{c:04X}: perl ({a}, {w}) vs table ({R.is_alphabetic(chr(c))}, {R.is_whitespace(chr(c))})")


# ---- randomised parity, library vs restatement ----

ALPHABET = (list("abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789") * 3
            + list(" " * 30 + "'" * 10 + "sStTmMdDrReEvVlL" + ".,!?;:-_()[]{}\"/\\@#$%^&*+=<>|~`")
            + list("\t\n\r\x0b\x0c\x85\xa0       　\x1c\x1d\x00\x07")
            + list("éèàçñßøåÆŒ日本語中文한국어Ελληνικάкириллица") + list("Ⅻⅰ")   # letters, letter numbers
            + list("Ⓐⓩͅाாְ") + list("٣۵߀") + list("😀🚀∑€¥") + list("́‍"))


def rand_text(rng, n):
    return "".join(rng.choice(ALPHABET) for _ in range(n))


def test_pre_tokenize_random_parity():
    rng = random.Random(1234)
    for _ in range(3000):
        s = rand_text(rng, rng.randint(0, 40))
        assert T.pre_tokenize(s) == R.pre_tokenize(s), repr(s)


def train_bpe(corpus: str, n_merges: int):
    """A small BPE trainer (most frequent adjacent pair, ties broken by first
    occurrence) over the pre-tokenised, byte-encoded corpus: vocab.json and
    merges.txt strings in the HuggingFace format."""
    enc = R.build_byte_encoder()
    words = [[enc[b] for b in w.encode()] for w in R.pre_tokenize(corpus)]
    vocab = list(enc)
    merges = []
    for _ in range(n_merges):
        counts = {}
        for w in words:
            for a, b in zip(w, w[1:]):
                counts[(a, b)] = counts.get((a, b), 0) + 1
        if not counts:
            break
        best = max(counts, key=lambda p: counts[p])
        if counts[best] < 2:
            break
        merges.append(best)
        vocab.append(best[0] + best[1])
        out = []
        for w in words:
            i, nw = 0, []
            while i < len(w):
                if i + 1 < len(w) and (w[i], w[i + 1]) == best:
                    nw.append(w[i] + w[i + 1])
                    i += 2
                else:
                    nw.append(w[i])
                    i += 1
            out.append(nw)
        words = out
    vj = json.dumps({t: i for i, t in enumerate(dict.fromkeys(vocab))}, ensure_ascii=bool(len(vocab) % 2))
    mt = "#version: 0.2\n" + "".join(f"{a} {b}\n" for a, b in merges)
    return vj, mt


@pytest.fixture(scope="module")
def trained():
    rng = random.Random(99)
    words = ["the", "token", "loop", "model", "decode", "cache", "layer", "head", "attention", "don't", "we'll"]
    corpus = " ".join(rng.choice(words) + (rng.choice([".", ",", "", "", " 42", "!"])) for _ in range(3000))
    corpus += rand_text(rng, 2000)
    vj, mt = train_bpe(corpus, 300)
    return vj, mt, T.BpeTokenizer.from_strings(vj, mt), R.BpeTokenizer.from_strings(vj, mt)


def test_encode_decode_random_parity(trained):
    _, _, lib, ref = trained
    assert lib.vocab_size() == ref.vocab_size()
    rng = random.Random(7)
    for _ in range(400):
        s = rand_text(rng, rng.randint(0, 80)) if rng.random() < 0.5 else " ".join(
            rng.choice(["the", "token", "loops", "don't", "We'll", "café", "2024", "日本"]) for _ in range(12))
        a, b = lib.encode(s), ref.encode(s)
        assert a == b, repr(s)
        assert lib.decode(a) == ref.decode(b) == s  # every byte has a token: lossless


def test_repetitive_words_parity():
    """Words of few distinct letters, where merges of one rank overlap."""
    rng = random.Random(5)
    corpus = " ".join("".join(rng.choice("ab") for _ in range(rng.randint(1, 9))) for _ in range(2000))
    vj, mt = train_bpe(corpus, 40)
    lib, ref = T.BpeTokenizer.from_strings(vj, mt), R.BpeTokenizer.from_strings(vj, mt)
    for _ in range(500):
        w = "".join(rng.choice("aab") for _ in range(rng.randint(1, 14)))
        assert lib.encode(w) == ref.encode(w), w


def test_decode_lossy_parity(trained):
    """decode of arbitrary byte sequences: one U+FFFD per maximal ill-formed
    subpart (String::from_utf8_lossy), ids past the table skipped."""
    _, _, lib, ref = trained
    enc = R.build_byte_encoder()
    byte_id = {b: ref.token_to_id(enc[b]) for b in range(256)}
    rng = random.Random(3)
    specials = [b"\xe2\x82", b"\xf0\x80\x80", b"\xed\xa0\x80", b"\xc0\xaf", b"\xf4\x90\x80\x80", b"\xe0\x80",
                b"\xf0\x9f\x98", b"\xff", b"\x80\x80", b"\xef\xbf\xbd"]
    for _ in range(500):
        parts = [rng.choice(specials) if rng.random() < 0.4 else bytes([rng.randrange(256)]) for _ in range(rng.randint(0, 12))]
        data = b"".join(parts)
        ids = [byte_id[b] for b in data] + ([10 ** 6] if rng.random() < 0.3 else [])
        got = lib.decode(ids)
        assert got == ref.decode(ids) == data.decode("utf-8", "replace"), data


BAD_VOCABS = ["not json", "{", "}", '{"a" 1}', '{"a": x}', '{"a": -1}', '{"a": 99999999999}', '{"a": 1, b: 2}',
              '{"a": 1.5}', r'{"\u12": 0}', r'{"\uZZZZ": 0}', r'{"\ud800": 0}', '{"abc', '{"a\\', '{"a": }',
              '{"\t": 1, "x":\n 2}', r'{"\q": 3}', r'{"\u+0041": 0}', '  {"a":1}  ', '{"a":1,,"b":2}']


@pytest.mark.parametrize("js", BAD_VOCABS)
def test_vocab_parser_parity(js):
    """Malformed and unusual vocab.json texts: the same result or the same
    error message (tokenizer.rs:356-470)."""
    try:
        want = R.BpeTokenizer.from_strings(js, "")
    except R.ParseError as e:
        with pytest.raises(Gpt2Error) as ei:
            T.BpeTokenizer.from_strings(js, "")
        assert str(ei.value) == str(e)
        return
    got = T.BpeTokenizer.from_strings(js, "")
    assert got.vocab_size() == want.vocab_size()
    for k, v in want.encoder.items():
        assert got.token_to_id(k) == v


def test_merges_line_endings_parity():
    vj = json.dumps({t: i for i, t in enumerate(["a", "b", "c", "ab", "bc", "abc", "a b"])})
    for mt in ["a b\r\nab c\r\n", "#h\r\nb c\na b", "version x\na b\r", "  a b  \n\n", "a  b\nb c", "a\nb c\n"]:
        lib, ref = T.BpeTokenizer.from_strings(vj, mt), R.BpeTokenizer.from_strings(vj, mt)
        for s in ["abc", "ab", "bca", "a b c"]:
            assert lib.encode(s) == ref.encode(s), (mt, s)

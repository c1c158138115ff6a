"""Test infrastructure only: a plain-Python restatement of rusttorch's byte-level
BPE tokenizer (rusttorch-core/src/data/tokenizer.rs), the checker for the
library's rtg_tokenizer_* entry points. Nothing in the product imports it.

Every function cites the lines it follows. Rust's `char::is_alphabetic` and
`char::is_whitespace` are the Unicode properties Alphabetic and White_Space;
their ranges are read from rusttorch_amd/csrc/unicode_tables.h, which the
tests pin against Perl's Unicode database code point by code point.
`String::from_utf8_lossy` is Python's `bytes.decode("utf-8", "replace")`
(both substitute one U+FFFD per maximal ill-formed subpart).
"""
from __future__ import annotations

import os
import re

_TABLES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "..", "rusttorch_amd", "csrc", "unicode_tables.h")


def _load_ranges(name: str) -> list[tuple[int, int]]:
    text = open(_TABLES).read()
    body = text[text.index(name):]
    body = body[body.index("{") + 1:body.index("};")]
    return [(int(a, 16), int(b, 16)) for a, b in re.findall(r"\{0x([0-9A-F]+), 0x([0-9A-F]+)\}", body)]


_ALPHA = _load_ranges("kAlphabetic")
_SPACE = _load_ranges("kWhiteSpace")


def _in(ranges, c: int) -> bool:
    lo, hi = 0, len(ranges)
    while lo < hi:
        mid = (lo + hi) // 2
        if c < ranges[mid][0]:
            hi = mid
        elif c > ranges[mid][1]:
            lo = mid + 1
        else:
            return True
    return False


def is_alphabetic(ch: str) -> bool:
    return _in(_ALPHA, ord(ch))


def is_whitespace(ch: str) -> bool:
    return _in(_SPACE, ord(ch))


def is_ascii_digit(ch: str) -> bool:
    return "0" <= ch <= "9"


# tokenizer.rs:248-251
def is_printable_byte(b: int) -> bool:
    return 33 <= b <= 126 or 161 <= b <= 172 or 174 <= b <= 255


# tokenizer.rs:223-241
def build_byte_encoder() -> list[str]:
    enc, offset = [], 0
    for b in range(256):
        if is_printable_byte(b):
            enc.append(chr(b))
        else:
            enc.append(chr(256 + offset))
            offset += 1
    return enc


# tokenizer.rs:334-353
def match_contraction(chars: list[str], i: int):
    remaining = len(chars) - i
    if remaining >= 3:
        two = "".join(chars[i + 1:i + 3]).lower()
        if two in ("re", "ve", "ll"):
            return "".join(chars[i:i + 3]), 3
    if remaining >= 2:
        one = chars[i + 1].lower()
        if one in ("s", "t", "m", "d"):
            return "".join(chars[i:i + 2]), 2
    return None


# tokenizer.rs:260-331
def pre_tokenize(text: str) -> list[str]:
    words, chars, i = [], list(text), 0
    n = len(chars)
    while i < n:
        if chars[i] == "'" and i + 1 < n:
            c = match_contraction(chars, i)
            if c is not None:
                words.append(c[0])
                i += c[1]
                continue
        if is_whitespace(chars[i]):
            if chars[i] == " " and i + 1 < n and is_alphabetic(chars[i + 1]):
                start = i
                i += 1
                while i < n and is_alphabetic(chars[i]):
                    i += 1
                words.append("".join(chars[start:i]))
                continue
            if chars[i] == " " and i + 1 < n and is_ascii_digit(chars[i + 1]):
                start = i
                i += 1
                while i < n and is_ascii_digit(chars[i]):
                    i += 1
                words.append("".join(chars[start:i]))
                continue
            words.append(chars[i])
            i += 1
            continue
        if is_alphabetic(chars[i]):
            start = i
            while i < n and is_alphabetic(chars[i]):
                i += 1
            words.append("".join(chars[start:i]))
            continue
        if is_ascii_digit(chars[i]):
            start = i
            while i < n and is_ascii_digit(chars[i]):
                i += 1
            words.append("".join(chars[start:i]))
            continue
        words.append(chars[i])
        i += 1
    return words


class ParseError(ValueError):
    pass


def _debug_opt_char(ch):
    """Rust's {:?} of Option<char> (the common cases)."""
    if ch is None:
        return "None"
    esc = {"'": "\\'", "\\": "\\\\", "\n": "\\n", "\r": "\\r", "\t": "\\t", "\0": "\\0"}
    if ch in esc:
        body = esc[ch]
    elif ord(ch) < 0x20 or ord(ch) == 0x7F:
        body = "\\u{%x}" % ord(ch)
    else:
        body = ch
    return f"Some('{body}')"


def _trim(s: str) -> str:
    b, e = 0, len(s)
    while b < e and is_whitespace(s[b]):
        b += 1
    while e > b and is_whitespace(s[e - 1]):
        e -= 1
    return s[b:e]


# tokenizer.rs:404-447
def _parse_json_string(s: str, i: int):
    if i >= len(s) or s[i] != '"':
        raise ParseError("Expected '\"', got " + _debug_opt_char(s[i] if i < len(s) else None))
    i += 1
    out = []
    while True:
        if i >= len(s):
            raise ParseError("Unexpected end of string")
        c = s[i]
        i += 1
        if c == '"':
            return "".join(out), i
        if c != "\\":
            out.append(c)
            continue
        if i >= len(s):
            raise ParseError("Unexpected end of string")
        c = s[i]
        i += 1
        simple = {'"': '"', "\\": "\\", "/": "/", "n": "\n", "r": "\r", "t": "\t"}
        if c in simple:
            out.append(simple[c])
        elif c == "u":
            hx = s[i:i + 4]
            i += len(hx)
            if len(hx.encode()) != 4:
                raise ParseError("Incomplete unicode escape")
            digits = hx[1:] if hx.startswith("+") else hx  # u32::from_str_radix accepts a '+'
            if not digits or any(d not in "0123456789abcdefABCDEF" for d in digits):
                raise ParseError("Invalid unicode escape: \\u" + hx)
            code = int(digits, 16)
            if 0xD800 <= code <= 0xDFFF:
                raise ParseError(f"Invalid unicode code point: {code}")
            out.append(chr(code))
        else:
            out.append("\\")
            out.append(c)


# tokenizer.rs:450-470
def _parse_json_int(s: str, i: int):
    num = ""
    if i < len(s) and s[i] == "-":
        num += "-"
        i += 1
    while i < len(s) and is_ascii_digit(s[i]):
        num += s[i]
        i += 1
    if not num or num.startswith("-") or int(num) > 0xFFFFFFFF:
        raise ParseError(f"Failed to parse integer: '{num}'")
    return int(num), i


# tokenizer.rs:356-401 (entries in file order; a repeated key keeps its last id)
def parse_vocab_json(json: str) -> dict[str, int]:
    json = _trim(json)
    if not (json.startswith("{") and json.endswith("}")) or len(json) < 2:
        raise ParseError("vocab.json must be a JSON object")
    inner = json[1:-1]
    out, i = {}, 0

    def skip(i):
        while i < len(inner) and is_whitespace(inner[i]):
            i += 1
        return i

    while True:
        i = skip(i)
        if i >= len(inner):
            break
        key, i = _parse_json_string(inner, i)
        i = skip(i)
        if i >= len(inner) or inner[i] != ":":
            raise ParseError("Expected ':', got " + _debug_opt_char(inner[i] if i < len(inner) else None))
        i = skip(i + 1)
        val, i = _parse_json_int(inner, i)
        out[key] = val
        i = skip(i)
        if i < len(inner) and inner[i] == ",":
            i += 1
    return out


def _rust_lines(text: str) -> list[str]:
    """str::lines: split at "\\n" (a "\\r" before it goes too); no empty last line."""
    parts = text.split("\n")
    if parts and parts[-1] == "":
        parts.pop()
    out = []
    for k, p in enumerate(parts):
        terminated = k < len(parts) - 1 or text.endswith("\n")
        out.append(p[:-1] if terminated and p.endswith("\r") else p)
    return out


# tokenizer.rs:486-514
def parse_merges(text: str) -> dict[tuple[str, str], int]:
    merges = {}
    for rank, line in enumerate(_rust_lines(text)):
        if line.startswith("#") or line.startswith("version"):
            continue
        line = _trim(line)
        if not line:
            continue
        parts = line.split(" ", 1)
        if len(parts) != 2:
            continue
        merges[(parts[0], parts[1])] = rank
    return merges


class BpeTokenizer:
    """tokenizer.rs:26-220."""

    def __init__(self, encoder: dict[str, int], decoder: list[str], merges: dict[tuple[str, str], int]):
        self.encoder, self.decoder, self.merges = encoder, decoder, merges
        self.byte_encoder = build_byte_encoder()
        self.byte_decoder = {c: b for b, c in enumerate(self.byte_encoder)}

    @classmethod
    def from_strings(cls, vocab_json: str, merges_txt: str) -> "BpeTokenizer":  # tokenizer.rs:55-82
        enc = parse_vocab_json(vocab_json)
        dec = [""] * ((max(enc.values()) if enc else 0) + 1)
        for tok, i in enc.items():
            dec[i] = tok
        return cls(enc, dec, parse_merges(merges_txt))

    @classmethod
    def from_vocab_and_merges(cls, vocab, merge_rules) -> "BpeTokenizer":  # tokenizer.rs:186-219
        enc = {}
        for i, t in enumerate(vocab):
            enc[t] = i
        return cls(enc, list(vocab), {(a, b): r for r, (a, b) in enumerate(merge_rules)})

    # tokenizer.rs:148-183
    def apply_bpe(self, tokens: list[str]) -> list[str]:
        tokens = list(tokens)
        if len(tokens) < 2:
            return tokens
        while True:
            best = None
            for i in range(len(tokens) - 1):
                r = self.merges.get((tokens[i], tokens[i + 1]))
                if r is not None and (best is None or r < best[1]):
                    best = (i, r)
            if best is None:
                return tokens
            p = best[0]
            tokens[p:p + 2] = [tokens[p] + tokens[p + 1]]

    # tokenizer.rs:85-112
    def encode(self, text: str) -> list[int]:
        ids = []
        for word in pre_tokenize(text):
            toks = self.apply_bpe([self.byte_encoder[b] for b in word.encode()])
            ids += [self.encoder[t] for t in toks if t in self.encoder]
        return ids

    # tokenizer.rs:115-130
    def decode(self, ids: list[int]) -> str:
        s = "".join(self.decoder[i] for i in ids if i < len(self.decoder))
        return bytes(self.byte_decoder[c] for c in s if c in self.byte_decoder).decode("utf-8", "replace")

    def vocab_size(self) -> int:
        return len(self.encoder)

    def token_to_id(self, token: str):
        return self.encoder.get(token)

    def id_to_token(self, i: int):
        return self.decoder[i] if i < len(self.decoder) else None

"""Python mirror of rusttorch's BpeTokenizer (rusttorch-core/src/data/tokenizer.rs)
over the C ABI of librtgpu.so (include/rtgpu.h, rtg_tokenizer_*).

Names, arguments and errors follow the reference: `from_files`, `from_strings`
and `from_vocab_and_merges` build a tokenizer, `encode` / `decode` convert text
and ids, `vocab_size`, `token_to_id` and `id_to_token` look tokens up (None is
Rust's None). Failures raise Gpt2Error with the reference's message.
`pre_tokenize` and `build_byte_encoder` expose two private functions of the
reference for its tests.
"""
from __future__ import annotations

import ctypes as C

from . import _lib
from ._lib import check


class BpeTokenizer:
    def __init__(self, handle):
        self._lib = _lib.load()
        self._h = handle

    @classmethod
    def from_files(cls, vocab_json: str, merges_txt: str) -> "BpeTokenizer":
        lib = _lib.load()
        h = C.c_void_p()
        check(lib.rtg_tokenizer_from_files(str(vocab_json).encode(), str(merges_txt).encode(), C.byref(h)))
        return cls(h)

    @classmethod
    def from_strings(cls, vocab_json: str, merges_txt: str) -> "BpeTokenizer":
        lib = _lib.load()
        v, m = vocab_json.encode(), merges_txt.encode()
        h = C.c_void_p()
        check(lib.rtg_tokenizer_from_strings(v, len(v), m, len(m), C.byref(h)))
        return cls(h)

    @classmethod
    def from_vocab_and_merges(cls, vocab: list[str], merge_rules: list[tuple[str, str]]) -> "BpeTokenizer":
        lib = _lib.load()
        vs = (C.c_char_p * max(1, len(vocab)))(*[t.encode() for t in vocab])
        a = (C.c_char_p * max(1, len(merge_rules)))(*[x.encode() for x, _ in merge_rules])
        b = (C.c_char_p * max(1, len(merge_rules)))(*[y.encode() for _, y in merge_rules])
        h = C.c_void_p()
        check(lib.rtg_tokenizer_from_vocab_and_merges(vs, len(vocab), a, b, len(merge_rules), C.byref(h)))
        return cls(h)

    def encode(self, text: str) -> list[int]:
        t = text.encode()
        ids, n = C.POINTER(C.c_uint32)(), C.c_size_t()
        check(self._lib.rtg_tokenizer_encode(self._h, t, len(t), C.byref(ids), C.byref(n)))
        try:
            return [ids[i] for i in range(n.value)]
        finally:
            self._lib.rtg_free_buffer(ids)

    def decode(self, ids: list[int]) -> str:
        arr = (C.c_uint32 * max(1, len(ids)))(*ids)
        p, n = C.c_void_p(), C.c_size_t()
        check(self._lib.rtg_tokenizer_decode(self._h, arr, len(ids), C.byref(p), C.byref(n)))
        try:
            return C.string_at(p, n.value).decode()
        finally:
            self._lib.rtg_free_buffer(p)

    def vocab_size(self) -> int:
        return int(self._lib.rtg_tokenizer_vocab_size(self._h))

    def token_to_id(self, token: str) -> int | None:
        t = token.encode()
        v = C.c_uint32()
        return int(v.value) if self._lib.rtg_tokenizer_token_to_id(self._h, t, len(t), C.byref(v)) else None

    def id_to_token(self, id: int) -> str | None:
        p, n = C.c_void_p(), C.c_size_t()
        if not self._lib.rtg_tokenizer_id_to_token(self._h, id, C.byref(p), C.byref(n)):
            return None
        return C.string_at(p, n.value).decode() if n.value else ""

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.rtg_tokenizer_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pre_tokenize(text: str) -> list[str]:
    """pre_tokenize, tokenizer.rs:260-331."""
    lib = _lib.load()
    t = text.encode()
    sp, n = C.POINTER(C.c_size_t)(), C.c_size_t()
    check(lib.rtg_tokenizer_pre_tokenize(t, len(t), C.byref(sp), C.byref(n)))
    try:
        return [t[sp[2 * k]:sp[2 * k + 1]].decode() for k in range(n.value)]
    finally:
        lib.rtg_free_buffer(sp)


def build_byte_encoder() -> list[str]:
    """build_byte_encoder, tokenizer.rs:223-241: the character of every byte."""
    lib = _lib.load()
    out = (C.c_uint32 * 256)()
    lib.rtg_tokenizer_byte_encoder(out)
    return [chr(out[i]) for i in range(256)]

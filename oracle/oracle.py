"""ctypes wrapper of the CPU oracle (oracle/_build/liboracle_gpt2.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline; the
product (rusttorch_amd, librtgpu.so) never imports it. Each method restates
one function of rusttorch-core/src/nn/gpt2.rs (see gpt2_oracle.c for the
file:line of each).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "liboracle_gpt2.so")


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


class OracleError(RuntimeError):
    pass


class _Cfg(C.Structure):
    _fields_ = [("vocab_size", C.c_size_t), ("n_positions", C.c_size_t), ("n_embd", C.c_size_t),
                ("n_layer", C.c_size_t), ("n_head", C.c_size_t), ("layer_norm_epsilon", C.c_float)]


_lib = None
F = C.POINTER(C.c_float)
U = C.POINTER(C.c_uint32)


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp = C.c_void_p
        sz = C.c_size_t
        L.orc_embedding_lookup.argtypes = [vp, sz, sz, vp, sz, vp, C.c_char_p]
        L.orc_layer_norm.argtypes = [vp, sz, sz, vp, vp, C.c_float, vp]
        L.orc_conv1d.argtypes = [vp, sz, sz, vp, vp, sz, vp, C.c_int]
        L.orc_matmul.argtypes = [vp, sz, sz, vp, sz, vp, C.c_int]
        L.orc_slice_columns.argtypes = [vp, sz, sz, sz, sz, vp]
        L.orc_multi_head_attention.argtypes = [vp, vp, vp, sz, sz, sz, vp]
        L.orc_gelu_new.argtypes = [vp, sz, vp]
        L.orc_argmax.argtypes = [vp, sz]
        L.orc_argmax.restype = C.c_uint32
        L.orc_apply_repetition_penalty.argtypes = [vp, sz, vp, sz, C.c_float]
        L.orc_apply_top_k.argtypes = [vp, sz, sz]
        L.orc_apply_top_p.argtypes = [vp, sz, C.c_float]
        L.orc_model_create.argtypes = [C.POINTER(_Cfg), C.POINTER(C.c_char_p), C.POINTER(vp), sz,
                                       C.POINTER(vp), C.c_char_p]
        L.orc_model_destroy.argtypes = [vp]
        L.orc_model_set_threads.argtypes = [vp, C.c_int]
        L.orc_model_set_lm_direct.argtypes = [vp, C.c_int]
        L.orc_num_parameters.argtypes = [vp]
        L.orc_num_parameters.restype = sz
        L.orc_cache_new.argtypes = [vp]
        L.orc_cache_new.restype = vp
        L.orc_cache_len.argtypes = [vp]
        L.orc_cache_len.restype = sz
        L.orc_cache_clear.argtypes = [vp]
        L.orc_cache_destroy.argtypes = [vp]
        L.orc_cache_read.argtypes = [vp, sz, sz, C.c_int, vp]
        L.orc_forward.argtypes = [vp, vp, sz, vp, C.c_char_p]
        L.orc_forward_cached.argtypes = [vp, vp, vp, sz, vp, C.c_char_p]
        L.orc_generate_cached.argtypes = [vp, vp, sz, sz, vp, C.c_char_p]
        L.orc_generate.argtypes = [vp, vp, sz, sz, vp, C.c_char_p]
        L.orc_generate_cached_gaps.argtypes = [vp, vp, sz, sz, vp, vp, C.c_char_p]
        L.orc_top2_gap.argtypes = [vp, sz]
        L.orc_top2_gap.restype = C.c_float
        _lib = L
    return _lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64).astype(np.uint32))


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _err() -> C.Array:
    return C.create_string_buffer(256)


# ---- helpers (one per gpt2.rs function) ----

def embedding_lookup(weight, ids) -> np.ndarray:
    w = _f32(weight)
    i = _u32(ids)
    out = np.empty((i.size, w.shape[1]), dtype=np.float32)
    e = _err()
    if lib().orc_embedding_lookup(_p(w), w.shape[0], w.shape[1], _p(i), i.size, _p(out), e) != 0:
        raise OracleError(e.value.decode())
    return out


def layer_norm(x, w, b, eps=1e-5) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    n = x.shape[-1]
    lib().orc_layer_norm(_p(x), x.size // n, n, _p(_f32(w)), _p(_f32(b)), eps, _p(out))
    return out


def matmul(a, b, threads=1) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    out = np.empty((a.shape[0], b.shape[1]), dtype=np.float32)
    lib().orc_matmul(_p(a), a.shape[0], a.shape[1], _p(b), b.shape[1], _p(out), threads)
    return out


def conv1d(x, w, bias, threads=1) -> np.ndarray:
    x, w, bias = _f32(x), _f32(w), _f32(bias)
    out = np.empty((x.shape[0], w.shape[1]), dtype=np.float32)
    lib().orc_conv1d(_p(x), x.shape[0], x.shape[1], _p(w), _p(bias), w.shape[1], _p(out), threads)
    return out


def slice_columns(t, start, end) -> np.ndarray:
    t = _f32(t)
    out = np.empty((t.shape[0], end - start), dtype=np.float32)
    lib().orc_slice_columns(_p(t), t.shape[0], t.shape[1], start, end, _p(out))
    return out


def multi_head_attention(q, k, v, n_head, head_dim, seq_len) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.empty((seq_len, n_head * head_dim), dtype=np.float32)
    lib().orc_multi_head_attention(_p(q), _p(k), _p(v), n_head, head_dim, seq_len, _p(out))
    return out


def gelu_new(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_gelu_new(_p(x), x.size, _p(out))
    return out


def top2_gap(x) -> float:
    """Top-1 minus top-2 value of a logits row (inf with fewer than two)."""
    a = _f32(x)
    return float(lib().orc_top2_gap(_p(a), a.size))


def argmax(x) -> int:
    x = _f32(x)
    return int(lib().orc_argmax(_p(x), x.size))


def apply_repetition_penalty(logits, tokens, penalty) -> np.ndarray:
    l = _f32(logits).copy()
    t = _u32(tokens)
    lib().orc_apply_repetition_penalty(_p(l), l.size, _p(t), t.size, penalty)
    return l


def apply_top_k(logits, k) -> np.ndarray:
    l = _f32(logits).copy()
    lib().orc_apply_top_k(_p(l), l.size, k)
    return l


def apply_top_p(logits, p) -> np.ndarray:
    l = _f32(logits).copy()
    lib().orc_apply_top_p(_p(l), l.size, p)
    return l


# ---- model ----

class OracleCache:
    def __init__(self, model: "OracleModel"):
        self.model = model
        self._h = lib().orc_cache_new(model._h)

    def len(self) -> int:
        return int(lib().orc_cache_len(self._h))

    def is_empty(self) -> bool:
        return self.len() == 0

    def clear(self) -> None:
        lib().orc_cache_clear(self._h)

    def read(self, layer, head, values=False) -> np.ndarray:
        hd = self.model.n_embd // self.model.n_head
        out = np.empty((self.len(), hd), dtype=np.float32)
        lib().orc_cache_read(self._h, layer, head, int(values), _p(out))
        return out

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_cache_destroy(self._h)
            self._h = None


class OracleModel:
    """Gpt2Model::from_state_dict over borrowed float32 arrays."""

    def __init__(self, sd: dict, vocab_size, n_positions, n_embd, n_layer, n_head, eps=1e-5, threads=1,
                 lm_direct=True):
        """lm_direct: the tied LM head sums each logit from its wte row
        (bit-identical to the reference's matmul over a materialised
        transpose, which lm_direct=False performs per call, as gpt2.rs:395
        does; the CPU baseline times that form)."""
        self.vocab_size, self.n_positions, self.n_embd = vocab_size, n_positions, n_embd
        self.n_layer, self.n_head = n_layer, n_head
        self._arrays = {k: _f32(v) for k, v in sd.items()}
        names = (C.c_char_p * max(1, len(sd)))(*[k.encode() for k in self._arrays])
        ptrs = (C.c_void_p * max(1, len(sd)))(*[a.ctypes.data for a in self._arrays.values()])
        cfg = _Cfg(vocab_size, n_positions, n_embd, n_layer, n_head, eps)
        h = C.c_void_p()
        e = _err()
        if lib().orc_model_create(C.byref(cfg), names, ptrs, len(sd), C.byref(h), e) != 0:
            raise OracleError(e.value.decode())
        self._h = h
        lib().orc_model_set_threads(h, threads)
        lib().orc_model_set_lm_direct(h, 1 if lm_direct else 0)

    @classmethod
    def from_shape(cls, sd, shape, threads=1, lm_direct=True):
        return cls(sd, shape.vocab_size, shape.n_positions, shape.n_embd, shape.n_layer, shape.n_head,
                   shape.layer_norm_epsilon, threads, lm_direct)

    def set_threads(self, threads: int) -> None:
        lib().orc_model_set_threads(self._h, threads)

    def num_parameters(self) -> int:
        return int(lib().orc_num_parameters(self._h))

    def new_cache(self) -> OracleCache:
        return OracleCache(self)

    def forward(self, ids) -> np.ndarray:
        i = _u32(ids)
        out = np.empty((i.size, self.vocab_size), dtype=np.float32)
        e = _err()
        if lib().orc_forward(self._h, _p(i), i.size, _p(out), e) != 0:
            raise OracleError(e.value.decode())
        return out

    def forward_cached(self, ids, cache: OracleCache) -> np.ndarray:
        i = _u32(ids)
        out = np.empty((max(1, i.size), self.vocab_size), dtype=np.float32)
        e = _err()
        if lib().orc_forward_cached(self._h, cache._h, _p(i), i.size, _p(out), e) != 0:
            raise OracleError(e.value.decode())
        return out[: i.size]

    def generate_cached(self, ids, max_new, gaps=False):
        """Greedy ids; with gaps=True also the top-1 minus top-2 logit of
        every greedy step's row, as (ids, gaps)."""
        i = _u32(ids)
        out = np.empty(i.size + max(1, max_new), dtype=np.uint32)
        g = np.full(max(1, max_new), np.nan, dtype=np.float32)
        e = _err()
        if lib().orc_generate_cached_gaps(self._h, _p(i), i.size, max_new, _p(out), _p(g), e) != 0:
            raise OracleError(e.value.decode())
        return (out.tolist(), g) if gaps else out.tolist()

    def generate(self, ids, max_new) -> list:
        i = _u32(ids)
        out = np.empty(i.size + max_new, dtype=np.uint32)
        e = _err()
        if lib().orc_generate(self._h, _p(i), i.size, max_new, _p(out), e) != 0:
            raise OracleError(e.value.decode())
        return out.tolist()

    def __del__(self):
        if getattr(self, "_h", None):
            lib().orc_model_destroy(self._h)
            self._h = None

"""Host-side mirror of rusttorch's GPT-2 API over the MI355X library.

Names, argument meaning and error behaviour follow
rusttorch-core/src/nn/gpt2.rs: `Gpt2Config` (:82-104), `GenerationConfig`
(:31-79), `KVCache` (:111-162) and `Gpt2Model` (:179-562). Rust's
`Result<_, String>` errors surface as `Gpt2Error` carrying the reference's
message. Every call goes through librtgpu.so (include/rtgpu.h); nothing here
computes model math.
"""
from __future__ import annotations

import ctypes as C
import dataclasses

import numpy as np

from . import _lib
from ._lib import Gpt2Error, check

__all__ = ["Gpt2Config", "GenerationConfig", "KVCache", "Gpt2Model", "Gpt2Error"]


@dataclasses.dataclass
class Gpt2Config:
    """gpt2.rs:82-104."""

    vocab_size: int
    n_positions: int
    n_embd: int
    n_layer: int
    n_head: int
    layer_norm_epsilon: float = 1e-5

    @staticmethod
    def gpt2_small() -> "Gpt2Config":
        return Gpt2Config(50257, 1024, 768, 12, 12, 1e-5)

    @staticmethod
    def gpt2_medium() -> "Gpt2Config":
        return Gpt2Config(50257, 1024, 1024, 24, 16, 1e-5)

    @staticmethod
    def gpt2_large() -> "Gpt2Config":
        return Gpt2Config(50257, 1024, 1280, 36, 20, 1e-5)

    @staticmethod
    def gpt2_xl() -> "Gpt2Config":
        return Gpt2Config(50257, 1024, 1600, 48, 25, 1e-5)

    def _c(self) -> _lib.Config:
        return _lib.Config(self.vocab_size, self.n_positions, self.n_embd, self.n_layer, self.n_head,
                           self.layer_norm_epsilon)


@dataclasses.dataclass
class GenerationConfig:
    """gpt2.rs:31-79; `seed` replaces the reference's thread_rng."""

    max_new_tokens: int = 50
    temperature: float = 0.8
    top_k: int = 0
    top_p: float = 1.0
    repetition_penalty: float = 1.0
    seed: int = 0

    @staticmethod
    def greedy(max_new_tokens: int) -> "GenerationConfig":
        return GenerationConfig(max_new_tokens=max_new_tokens, temperature=0.0)

    @staticmethod
    def creative(max_new_tokens: int) -> "GenerationConfig":
        return GenerationConfig(max_new_tokens=max_new_tokens, temperature=0.9, top_k=50, top_p=0.95,
                                repetition_penalty=1.2)


def _ids(ids) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(ids, dtype=np.int64))
    if a.size and (a.min() < 0 or a.max() >= 2 ** 32):
        raise Gpt2Error("token ids must fit in u32")
    return np.ascontiguousarray(a.astype(np.uint32))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class KVCache:
    """KVCache (gpt2.rs:111-162), preallocated in HBM for n_positions tokens.

    `batch` > 1 is the batched extension: B sequences advancing together."""

    def __init__(self, model: "Gpt2Model", batch: int = 1):
        self._lib = _lib.load()
        self.model = model
        self.batch = batch
        h = C.c_void_p()
        check(self._lib.rtg_cache_new(model._h, batch, C.byref(h)))
        self._h = h

    def len(self) -> int:
        return int(self._lib.rtg_cache_len(self._h))

    def __len__(self) -> int:
        return self.len()

    def is_empty(self) -> bool:
        return bool(self._lib.rtg_cache_is_empty(self._h))

    def clear(self) -> None:
        self._lib.rtg_cache_clear(self._h)

    def read(self, layer: int, head: int, seq: int = 0, values: bool = False) -> np.ndarray:
        """Cached keys (or values) of one layer/head/sequence: [len, head_dim]."""
        hd = self.model.config.n_embd // self.model.config.n_head
        out = np.empty((self.len(), hd), dtype=np.float32)
        check(self._lib.rtg_cache_read(self._h, layer, head, seq, int(values), _ptr(out)))
        return out

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.rtg_cache_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Gpt2Model:
    """Gpt2Model (gpt2.rs:179-562) with weights resident in HBM."""

    def __init__(self, handle: C.c_void_p, config: Gpt2Config, storage: str):
        self._lib = _lib.load()
        self._h = handle
        self.config = config
        self.storage = storage

    # -- construction (gpt2.rs:214-263) --
    @staticmethod
    def _storage(storage: str) -> int:
        if storage not in ("f32", "bf16"):
            raise ValueError("storage must be 'f32' or 'bf16'")
        return _lib.RTG_STORE_BF16 if storage == "bf16" else _lib.RTG_STORE_F32

    @classmethod
    def from_safetensors(cls, path: str, config: Gpt2Config, storage: str = "f32") -> "Gpt2Model":
        lib = _lib.load()
        h = C.c_void_p()
        cfg = config._c()
        check(lib.rtg_model_from_safetensors(str(path).encode(), C.byref(cfg), cls._storage(storage), C.byref(h)))
        return cls(h, config, storage)

    @classmethod
    def from_state_dict(cls, sd: dict, config: Gpt2Config, storage: str = "f32") -> "Gpt2Model":
        lib = _lib.load()
        keep = []
        arr = (_lib.NamedTensor * max(1, len(sd)))()
        for i, (name, a) in enumerate(sd.items()):
            # f16 / f64 arrays go to the library as they are (f16 is widened on
            # the device); anything else is passed as f32
            a = np.asarray(a)
            if a.dtype == np.float16:
                dt = _lib.RTG_F16
            elif a.dtype == np.float64:
                dt = _lib.RTG_F64
            else:
                a, dt = a.astype(np.float32, copy=False), _lib.RTG_F32
            a = np.ascontiguousarray(a)
            shape = (C.c_size_t * max(1, a.ndim))(*a.shape)
            nm = name.encode()
            keep += [a, shape, nm]
            arr[i] = _lib.NamedTensor(nm, a.ctypes.data, dt, a.ndim, shape)
        h = C.c_void_p()
        cfg = config._c()
        check(lib.rtg_model_from_host(C.byref(cfg), arr, len(sd), cls._storage(storage), C.byref(h)))
        return cls(h, config, storage)

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._lib.rtg_model_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def num_parameters(self) -> int:
        return int(self._lib.rtg_num_parameters(self._h))

    def new_cache(self, batch: int = 1) -> KVCache:
        return KVCache(self, batch)

    # -- forward passes --
    def forward(self, token_ids) -> np.ndarray:
        """gpt2.rs:269-304: logits [seq_len, vocab]."""
        ids = _ids(token_ids)
        out = np.empty((ids.size, self.config.vocab_size), dtype=np.float32)
        check(self._lib.rtg_forward(self._h, _ptr(ids), ids.size, _ptr(out)))
        return out

    def forward_cached(self, token_ids, cache: KVCache) -> np.ndarray:
        """gpt2.rs:358-399: logits [new_len, vocab]; the cache grows by new_len."""
        ids = _ids(token_ids)
        out = np.empty((ids.size, self.config.vocab_size), dtype=np.float32)
        check(self._lib.rtg_forward_cached(self._h, cache._h, _ptr(ids), ids.size, _ptr(out)))
        return out

    def forward_cached_batched(self, token_ids, cache: KVCache, want_logits: bool = True):
        """Batched extension: ids [B, n] -> logits [B, n, vocab] (or None)."""
        ids = _ids(token_ids).reshape(cache.batch, -1)
        n = ids.shape[1]
        out = np.empty((cache.batch, n, self.config.vocab_size), dtype=np.float32) if want_logits else None
        check(self._lib.rtg_forward_cached_batched(self._h, cache._h, _ptr(ids), n,
                                                    _ptr(out) if want_logits else None))
        return out

    # -- generation --
    def generate(self, token_ids, max_new_tokens: int, temperature: float, seed: int = 0) -> list:
        """gpt2.rs:311-346 (uncached, sliding window)."""
        ids = _ids(token_ids)
        out = np.empty(ids.size + max_new_tokens, dtype=np.uint32)
        check(self._lib.rtg_generate(self._h, _ptr(ids), ids.size, max_new_tokens, temperature, seed, _ptr(out)))
        return out.tolist()

    def generate_cached(self, token_ids, max_new_tokens: int, temperature: float, seed: int = 0) -> list:
        """gpt2.rs:405-441. Returns prompt + max(1, max_new_tokens) ids."""
        ids = _ids(token_ids)
        out = np.empty(ids.size + max(1, max_new_tokens), dtype=np.uint32)
        check(self._lib.rtg_generate_cached(self._h, _ptr(ids), ids.size, max_new_tokens, temperature, seed,
                                            _ptr(out)))
        return out.tolist()

    def generate_with_config(self, token_ids, config: GenerationConfig) -> list:
        """gpt2.rs:447-474."""
        ids = _ids(token_ids)
        out = np.empty(ids.size + max(1, config.max_new_tokens), dtype=np.uint32)
        gc = _lib.GenConfig(config.max_new_tokens, config.temperature, config.top_k, config.top_p,
                            config.repetition_penalty, config.seed)
        check(self._lib.rtg_generate_with_config(self._h, _ptr(ids), ids.size, C.byref(gc), _ptr(out)))
        return out.tolist()

    def generate_cached_batched(self, prompts, max_new_tokens: int, timing: bool = False,
                                profile_kernels: bool = False):
        """Batched greedy generate_cached: prompts [B, n] -> ids [B, n + max(1, max_new)].

        timing=True also returns the device-event timings; profile_kernels=True
        additionally replays the decode steps launch by launch to time the
        decode-step kernel itself."""
        ids = np.atleast_2d(_ids(prompts))
        B, n = ids.shape
        ids = np.ascontiguousarray(ids)
        out = np.empty((B, n + max(1, max_new_tokens)), dtype=np.uint32)
        t = _lib.Timing()
        t.profile_kernels = int(profile_kernels)
        check(self._lib.rtg_generate_cached_batched(self._h, _ptr(ids), B, n, max_new_tokens, _ptr(out),
                                                    C.byref(t)))
        if timing:
            return out, {"prefill_ms": t.prefill_ms, "decode_ms": t.decode_ms, "decode_steps": t.decode_steps,
                         "decode_kernel_ms": t.decode_kernel_ms,
                         "decode_kernel_launches": t.decode_kernel_launches}
        return out

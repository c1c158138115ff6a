"""ctypes binding of include/rtgpu.h (librtgpu.so, built in-tree for gfx950).

Loading fails loudly when the library has not been built: there is no CPU
fallback for the token loop.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "librtgpu.so")


class Result(C.Structure):
    _fields_ = [("success", C.c_bool), ("error_msg", C.c_void_p)]


class Config(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_size_t),
        ("n_positions", C.c_size_t),
        ("n_embd", C.c_size_t),
        ("n_layer", C.c_size_t),
        ("n_head", C.c_size_t),
        ("layer_norm_epsilon", C.c_float),
    ]


class GenConfig(C.Structure):
    _fields_ = [
        ("max_new_tokens", C.c_size_t),
        ("temperature", C.c_float),
        ("top_k", C.c_size_t),
        ("top_p", C.c_float),
        ("repetition_penalty", C.c_float),
        ("seed", C.c_uint64),
    ]


class NamedTensor(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("data", C.c_void_p),
        ("dtype", C.c_int),
        ("ndim", C.c_size_t),
        ("shape", C.POINTER(C.c_size_t)),
    ]


class Timing(C.Structure):
    _fields_ = [
        ("profile_kernels", C.c_int),
        ("prefill_ms", C.c_double),
        ("decode_ms", C.c_double),
        ("decode_steps", C.c_size_t),
        ("decode_kernel_ms", C.c_double),
        ("decode_kernel_launches", C.c_size_t),
    ]


RTG_F32, RTG_BF16, RTG_F16, RTG_F64 = 0, 1, 2, 3
RTG_STORE_F32, RTG_STORE_BF16 = 0, 1

# name -> (restype, argtypes); every symbol declared in include/rtgpu.h.
SIGNATURES = {
    "rtg_init": (None, []),
    "rtg_cleanup": (None, []),
    "rtg_version": (C.c_char_p, []),
    "rtg_free_error_message": (None, [C.c_void_p]),
    "rtg_model_from_safetensors": (Result, [C.c_char_p, C.POINTER(Config), C.c_int, C.POINTER(C.c_void_p)]),
    "rtg_model_from_host": (Result, [C.POINTER(Config), C.POINTER(NamedTensor), C.c_size_t, C.c_int,
                                     C.POINTER(C.c_void_p)]),
    "rtg_model_destroy": (None, [C.c_void_p]),
    "rtg_num_parameters": (C.c_size_t, [C.c_void_p]),
    "rtg_cache_new": (Result, [C.c_void_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    "rtg_cache_len": (C.c_size_t, [C.c_void_p]),
    "rtg_cache_is_empty": (C.c_bool, [C.c_void_p]),
    "rtg_cache_clear": (None, [C.c_void_p]),
    "rtg_cache_destroy": (None, [C.c_void_p]),
    "rtg_cache_read": (Result, [C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int, C.c_void_p]),
    "rtg_forward": (Result, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "rtg_forward_cached": (Result, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "rtg_forward_cached_noalloc": (Result, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "rtg_generate": (Result, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_float, C.c_uint64,
                              C.c_void_p]),
    "rtg_generate_cached": (Result, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_float, C.c_uint64,
                                     C.c_void_p]),
    "rtg_generate_with_config": (Result, [C.c_void_p, C.c_void_p, C.c_size_t, C.POINTER(GenConfig), C.c_void_p]),
    "rtg_forward_cached_batched": (Result, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "rtg_generate_cached_batched": (Result, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_size_t, C.c_size_t,
                                             C.c_void_p, C.POINTER(Timing)]),
    "rtg_tokenizer_from_files": (Result, [C.c_char_p, C.c_char_p, C.POINTER(C.c_void_p)]),
    "rtg_tokenizer_from_strings": (Result, [C.c_char_p, C.c_size_t, C.c_char_p, C.c_size_t, C.POINTER(C.c_void_p)]),
    "rtg_tokenizer_from_vocab_and_merges": (Result, [C.POINTER(C.c_char_p), C.c_size_t, C.POINTER(C.c_char_p),
                                                     C.POINTER(C.c_char_p), C.c_size_t, C.POINTER(C.c_void_p)]),
    "rtg_tokenizer_destroy": (None, [C.c_void_p]),
    "rtg_tokenizer_encode": (Result, [C.c_void_p, C.c_char_p, C.c_size_t, C.POINTER(C.POINTER(C.c_uint32)),
                                      C.POINTER(C.c_size_t)]),
    "rtg_tokenizer_decode": (Result, [C.c_void_p, C.POINTER(C.c_uint32), C.c_size_t, C.POINTER(C.c_void_p),
                                      C.POINTER(C.c_size_t)]),
    "rtg_tokenizer_vocab_size": (C.c_size_t, [C.c_void_p]),
    "rtg_tokenizer_token_to_id": (C.c_bool, [C.c_void_p, C.c_char_p, C.c_size_t, C.POINTER(C.c_uint32)]),
    "rtg_tokenizer_id_to_token": (C.c_bool, [C.c_void_p, C.c_uint32, C.POINTER(C.c_void_p), C.POINTER(C.c_size_t)]),
    "rtg_tokenizer_pre_tokenize": (Result, [C.c_char_p, C.c_size_t, C.POINTER(C.POINTER(C.c_size_t)),
                                            C.POINTER(C.c_size_t)]),
    "rtg_tokenizer_byte_encoder": (None, [C.POINTER(C.c_uint32)]),
    "rtg_free_buffer": (None, [C.c_void_p]),
}

_lib = None


def load() -> C.CDLL:
    """Load librtgpu.so (once). Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m rusttorch_amd.build` "
            "(there is no CPU fallback for the GPT-2 token loop)")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    lib.rtg_init()
    _lib = lib
    return lib


class Gpt2Error(RuntimeError):
    """A `Result<_, String>` error of the reference, carrying its message."""


def check(res: Result) -> None:
    if res.success:
        return
    lib = load()
    msg = C.cast(res.error_msg, C.c_char_p).value.decode() if res.error_msg else "unknown error"
    lib.rtg_free_error_message(res.error_msg)
    raise Gpt2Error(msg)

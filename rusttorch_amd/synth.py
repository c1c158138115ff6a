"""Seeded synthetic GPT-2 weights and token ids (no network, no checkpoints).

The same generator feeds the GPU library, the CPU oracle and the transformers
cross-check, so every side sees identical bytes.

Generator: SplitMix64 (Steele, Lea, Flood 2014), whose i-th output is the
mix of seed + (i+1)*0x9E3779B97F4A7C15; each output becomes a 53-bit uniform
u = (z >> 11) * 2**-53.  Normals come from Box-Muller on consecutive pairs
(u1, u2): r = sqrt(-2 ln(1 - u1)), z0 = r cos(2 pi u2), z1 = r sin(2 pi u2),
computed in float64 and rounded to float32.  Each tensor starts on a fresh
pair and consumes ceil(n/2) pairs.  Tensors are filled in the HuggingFace
name order below.  Matrices, embeddings and biases ~ N(0, 0.02); LayerNorm
gains 1 + N(0, 0.02) and LayerNorm biases N(0, 0.02), so every parameter is
exercised while the logits keep a modest scale.
"""
from __future__ import annotations

import ctypes as C
import dataclasses
import json
import os
import struct

import numpy as np

_SYNTH_SO = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libsynth.so")
_synth = None


def _csynth():
    """The C generator (lib/libsynth.so); the numpy path below is its specification."""
    global _synth
    if _synth is None:
        if not os.path.exists(_SYNTH_SO):
            raise RuntimeError(f"{_SYNTH_SO} missing: run `python -m rusttorch_amd.build`")
        lib = C.CDLL(_SYNTH_SO)
        lib.synth_normals.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_double, C.c_double, C.c_void_p]
        lib.synth_normals.restype = None
        _synth = lib
    return _synth

GAMMA = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)
WEIGHT_SEED = 1234
TOKEN_SEED = 5678
STD = 0.02
_CHUNK = 1 << 22


@dataclasses.dataclass(frozen=True)
class ModelShape:
    """Hyper-parameters of one GPT-2 size (gpt2.rs:82-104 fields)."""

    vocab_size: int
    n_positions: int
    n_embd: int
    n_layer: int
    n_head: int
    layer_norm_epsilon: float = 1e-5


SHAPES = {
    # rusttorch's tiny unit-test config (gpt2.rs:1023-1032)
    "tiny": ModelShape(10, 16, 8, 2, 2),
    # small fast parity config with the full head_dim of 64
    "mini": ModelShape(512, 64, 128, 2, 2),
    "small": ModelShape(50257, 1024, 768, 12, 12),
    "medium": ModelShape(50257, 1024, 1024, 24, 16),
    "large": ModelShape(50257, 1024, 1280, 36, 20),
    "xl": ModelShape(50257, 1024, 1600, 48, 25),
}


def _splitmix(start: int, count: int, seed: int) -> np.ndarray:
    """Outputs start .. start+count-1 of SplitMix64 seeded with `seed`."""
    with np.errstate(over="ignore"):
        idx = np.arange(start + 1, start + count + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * GAMMA
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def _uniform(start: int, count: int, seed: int) -> np.ndarray:
    return (_splitmix(start, count, seed) >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)


def normals(pair_start: int, n: int, seed: int) -> np.ndarray:
    """n standard normals (float64) starting at Box-Muller pair `pair_start`."""
    out = np.empty(n, dtype=np.float64)
    npairs = (n + 1) // 2
    done = 0
    while done < npairs:
        c = min(_CHUNK, npairs - done)
        u = _uniform(2 * (pair_start + done), 2 * c, seed)
        r = np.sqrt(-2.0 * np.log1p(-u[0::2]))
        th = 2.0 * np.pi * u[1::2]
        z = np.empty(2 * c, dtype=np.float64)
        z[0::2] = r * np.cos(th)
        z[1::2] = r * np.sin(th)
        lo = 2 * done
        hi = min(n, lo + 2 * c)
        out[lo:hi] = z[: hi - lo]
        done += c
    return out


def tensor_specs(shape: ModelShape):
    """(name, shape, kind) in fill order; kind is 'w' (N(0,std)), 'g' (1+N) or 'b' (N)."""
    d, f = shape.n_embd, 4 * shape.n_embd
    specs = [("wte.weight", (shape.vocab_size, d), "w"), ("wpe.weight", (shape.n_positions, d), "w")]
    for i in range(shape.n_layer):
        p = f"h.{i}"
        specs += [
            (f"{p}.ln_1.weight", (d,), "g"), (f"{p}.ln_1.bias", (d,), "b"),
            (f"{p}.attn.c_attn.weight", (d, 3 * d), "w"), (f"{p}.attn.c_attn.bias", (3 * d,), "b"),
            (f"{p}.attn.c_proj.weight", (d, d), "w"), (f"{p}.attn.c_proj.bias", (d,), "b"),
            (f"{p}.ln_2.weight", (d,), "g"), (f"{p}.ln_2.bias", (d,), "b"),
            (f"{p}.mlp.c_fc.weight", (d, f), "w"), (f"{p}.mlp.c_fc.bias", (f,), "b"),
            (f"{p}.mlp.c_proj.weight", (f, d), "w"), (f"{p}.mlp.c_proj.bias", (d,), "b"),
        ]
    specs += [("ln_f.weight", (d,), "g"), ("ln_f.bias", (d,), "b")]
    return specs


def make_weights(shape: ModelShape, seed: int = WEIGHT_SEED, bf16: bool = False,
                 use_numpy: bool = False) -> dict[str, np.ndarray]:
    """Name -> float32 array (reference [in, out] Conv1D layout).

    bf16=True rounds every value to bfloat16 (round to nearest even) and
    returns the float32 upcast, i.e. exactly what a reader of a BF16
    safetensors file sees (safetensors.rs:389-391: bits << 16)."""
    out = {}
    pair = 0
    for name, shp, kind in tensor_specs(shape):
        n = int(np.prod(shp))
        a0, b0 = (1.0, STD) if kind == "g" else (0.0, STD)
        if use_numpy:
            a = (a0 + b0 * normals(pair, n, seed)).astype(np.float32).reshape(shp)
        else:
            a = np.empty(shp, dtype=np.float32)
            _csynth().synth_normals(seed, pair, n, a0, b0, a.ctypes.data)
        pair += (n + 1) // 2
        if bf16:
            a = bf16_bits_to_f32(f32_to_bf16_bits(a))
        out[name] = a
    return out


def make_tokens(n: int, vocab: int, seed: int = TOKEN_SEED, stream: int = 0) -> np.ndarray:
    """n uniform token ids in [0, vocab) from the token seed (u32)."""
    u = _uniform(stream * (1 << 32), n, seed)
    return np.minimum((u * vocab).astype(np.uint64), vocab - 1).astype(np.uint32)


def f32_to_bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bfloat16 bit patterns (uint16); NaN stays NaN."""
    b = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    rounded = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)
    nan = (b & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    rounded = np.where(nan, (b >> np.uint32(16)) | np.uint32(0x40), rounded)
    return rounded.astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    """bf16_to_f32 of safetensors.rs:389-391: the bits become the top half of an f32."""
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def write_safetensors(path: str, tensors: dict[str, np.ndarray], bf16: bool = False) -> None:
    """Minimal safetensors writer: 8-byte LE header length, JSON header, raw data."""
    header = {}
    blobs = []
    off = 0
    for name, a in tensors.items():
        if bf16:
            raw = f32_to_bf16_bits(a).tobytes()
            dt = "BF16"
        else:
            raw = np.ascontiguousarray(a, dtype=np.float32).tobytes()
            dt = "F32"
        header[name] = {"dtype": dt, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hj = json.dumps(header, separators=(",", ":")).encode()
    hj += b" " * ((8 - len(hj) % 8) % 8)
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Q", len(hj)))
        fh.write(hj)
        for raw in blobs:
            fh.write(raw)


def num_parameters(shape: ModelShape) -> int:
    return sum(int(np.prod(s)) for _, s, _ in tensor_specs(shape))

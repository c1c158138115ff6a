"""Test infrastructure only: a numpy restatement of the reference's token choice
for generate_with_config and sampled generate_cached (rusttorch-core/src/nn/
gpt2.rs:871-1017), the checker for the library's device sampler. Nothing in
the product imports it.

Arithmetic is float32 with the reference's sequential sums (np.cumsum).
The reference draws its uniforms from rand::thread_rng; here draw number k of
a sequence is SplitMix64 output k for the caller's seed, 24 bits / 2^24, the
convention the library uses, so a seeded run can be replayed exactly.
"""
from __future__ import annotations

import numpy as np

_GAMMA = 0x9E3779B97F4A7C15
_M64 = (1 << 64) - 1


def splitmix_uniform(seed: int, k: int) -> np.float32:
    z = (seed + k * _GAMMA) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    z ^= z >> 31
    return np.float32(z >> 40) * np.float32(1.0 / 16777216.0)


def _seq_sum(x: np.ndarray) -> np.float32:
    return np.cumsum(x, dtype=np.float32)[-1] if x.size else np.float32(0)


def _softmax(x: np.ndarray) -> np.ndarray:
    """max fold, exp(x - max), sequential sum, divide (gpt2.rs:945-948, 976-979)."""
    mx = np.max(x)
    e = np.exp((x - mx).astype(np.float32)).astype(np.float32)
    return (e / _seq_sum(e)).astype(np.float32)


def apply_repetition_penalty(x: np.ndarray, tokens, penalty: float) -> None:  # gpt2.rs:909-921
    pen = np.float32(penalty)
    for t in tokens:
        if t < x.size:
            x[t] = x[t] / pen if x[t] > 0 else x[t] * pen


def apply_top_k(x: np.ndarray, k: int) -> None:  # gpt2.rs:924-935
    thr = np.sort(x)[::-1][min(k, x.size) - 1]
    x[x < thr] = -np.inf


def apply_top_p(x: np.ndarray, p: float, exact: bool = False) -> None:  # gpt2.rs:939-970
    """exact=False: the reference's sequential f32 running sum. exact=True:
    the same rule on float64 probabilities and sums, the cut that the
    reference's f32 sum approximates: over thousands of kept entries its
    drift (~1e-6) can move the cut by an entry, and which of the two a
    summation order lands on is not fixed by the reference."""
    if exact:
        x64 = x.astype(np.float64)
        probs = np.exp(x64 - np.max(x64))
        probs /= probs.sum()
    else:
        probs = _softmax(x)
    order = np.argsort(-probs, kind="stable")
    cum = np.cumsum(probs[order], dtype=np.float64 if exact else np.float32)
    keep = np.zeros(x.size, dtype=bool)
    for j, i in enumerate(order):
        keep[i] = True
        if cum[j] >= (p if exact else np.float32(p)):
            break
    x[~keep] = -np.inf


def sample_from_logits(x: np.ndarray, r: np.float32):
    """gpt2.rs:973-993: (index, cdf below it, cdf at it)."""
    cum = np.cumsum(_softmax(x), dtype=np.float32)
    hit = np.nonzero(r < cum)[0]
    i = int(hit[0]) if hit.size else x.size - 1
    return i, (cum[i - 1] if i > 0 else np.float32(0)), cum[i]


def argmax_f32(x: np.ndarray) -> int:  # gpt2.rs:858-868: strict '>' from -inf, first index wins
    best, bv = 0, -np.inf
    for i, v in enumerate(x):
        if v > bv:
            best, bv = i, v
    return best


def choose(logits: np.ndarray, tokens, temperature: float, top_k: int, top_p: float, penalty: float, r,
           exact_top_p: bool = False):
    """sample_logits (gpt2.rs:871-906). Returns (token, cdf_lo, cdf_hi, filtered
    logits); for the greedy branch the cdf bounds are None. exact_top_p: the
    float64 top-p cut (see apply_top_p)."""
    x = np.array(logits, dtype=np.float32)
    if temperature <= 0:
        if penalty != 1.0:
            apply_repetition_penalty(x, tokens, penalty)
        return argmax_f32(x), None, None, x
    if penalty != 1.0:
        apply_repetition_penalty(x, tokens, penalty)
    x = (x / np.float32(temperature)).astype(np.float32)
    if 0 < top_k < x.size:
        apply_top_k(x, top_k)
    if 0.0 < top_p < 1.0:
        apply_top_p(x, top_p, exact_top_p)
    i, lo, hi = sample_from_logits(x, r)
    return i, lo, hi, x

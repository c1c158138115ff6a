"""bench.py's accounting, checked on the CPU.

The roofline's algorithmic bytes come from decode_bytes / prefill_bytes; they
are pinned here against the published parameter counts of the four GPT-2
checkpoints (Hugging Face model cards: 124,439,808 / 354,823,168 /
774,030,080 / 1,557,611,200 parameters, wte tied with the LM head) and
against the tensors the synthetic loader actually builds, so a dropped
matrix or a double-counted one fails here rather than inflating `frac`.
"""
import os
import subprocess
import sys

import numpy as np
import pytest

import bench
from rusttorch_amd import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PUBLISHED_PARAMS = {"small": 124_439_808, "medium": 354_823_168, "large": 774_030_080, "xl": 1_557_611_200}


def _weight_bytes(name, wbytes):
    """decode_bytes at batch 1 minus its per-step activation terms: the
    weights read once per step (every parameter but wpe, of which only the
    position's row is read)."""
    sh = synth.SHAPES[name]
    d, L, V = sh.n_embd, sh.n_layer, sh.vocab_size
    kv = L * 2 * d * 4 * 2  # past = 0: one cached row read plus the new row written
    emb = 2 * d * 4
    logits = V * 4
    return bench.decode_bytes(sh, 1, 0, wbytes) - kv - emb - logits


@pytest.mark.parametrize("name", sorted(PUBLISHED_PARAMS))
def test_decode_weight_bytes_match_published_parameter_counts(name):
    sh = synth.SHAPES[name]
    streamed = PUBLISHED_PARAMS[name] - sh.n_positions * sh.n_embd  # all but wpe
    assert _weight_bytes(name, 4) == 4 * streamed


def test_decode_bytes_bf16_storage_counts_matrices_at_two_bytes():
    sh = synth.SHAPES["xl"]
    d, L, V = sh.n_embd, sh.n_layer, sh.vocab_size
    mats = L * 12 * d * d + V * d  # c_attn, c_proj, c_fc, mlp c_proj and the tied wte
    vec = PUBLISHED_PARAMS["xl"] - sh.n_positions * d - mats  # LayerNorms and biases stay f32
    assert _weight_bytes("xl", 2) == 2 * mats + 4 * vec


def test_decode_bytes_against_synthetic_tensors():
    """The mini model's state dict, counted tensor by tensor."""
    sh = synth.SHAPES["mini"]
    sd = synth.make_weights(sh)
    total = sum(int(np.asarray(v).size) for v in sd.values())
    wpe = sh.n_positions * sh.n_embd
    assert _weight_bytes("mini", 4) == 4 * (total - wpe)


def test_decode_bytes_grow_with_the_cache():
    sh = synth.SHAPES["small"]
    per_pos = bench.decode_bytes(sh, 3, 101, 4) - bench.decode_bytes(sh, 3, 100, 4)
    assert per_pos == 3 * sh.n_layer * 2 * sh.n_embd * 4  # one more K and V row per layer and sequence


def test_prefill_flops_small_case_by_brute_force():
    """forward_cached over T tokens of a 1-layer model, counted per product:
    the four Conv1D GEMMs, causal scores and P.V per query, the LM head."""
    sh = synth.ModelShape(vocab_size=50, n_positions=16, n_embd=8, n_layer=1, n_head=2, layer_norm_epsilon=1e-5)
    T, d, V = 5, 8, 50
    gemm = 2 * T * (d * 3 * d + d * d + d * 4 * d + 4 * d * d)
    att = sum(2 * d * (t + 1) * 2 for t in range(T))  # q.k over t+1 keys and p.v, all heads together
    head = 2 * T * d * V
    assert bench.prefill_flops(sh, 1, T) == gemm + att + head
    assert bench.prefill_flops(sh, 3, T) == 3 * (gemm + att + head)


def test_prefill_roofline_bound_and_peak():
    sh = synth.SHAPES["large"]
    r = bench.prefill_roofline(sh, 32, 1024, 4, 420.0)
    assert r["bound"] == "mfma" and r["mfma"] == "fp32" and r["peak"] == bench.MFMA_FP32_PEAK_TFLOPS
    assert r["frac"] == pytest.approx(bench.prefill_flops(sh, 32, 1024) / 0.42 / 1e12 / r["peak"], rel=1e-3)
    r16 = bench.prefill_roofline(synth.SHAPES["xl"], 16, 64, 2, 16.0)
    assert r16["mfma"] == "bf16x3" and r16["peak"] == pytest.approx(bench.MFMA_BF16_PEAK_TFLOPS / 3, rel=1e-3)
    small = bench.prefill_roofline(synth.SHAPES["small"], 1, 4, 4, 0.5)
    assert small["bound"] == "hbm" and small["peak"] == bench.HBM_PEAK_GBS


def test_more_than_one_gpu_is_refused_without_touching_a_device():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""

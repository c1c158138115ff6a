"""Logits of the batch-1 persistent decode step, the kernel behind the
headline decode number, against the CPU oracle.

forward_cached with one new token on a batch-1 cache runs the same
persistent step that generate_cached launches per token (gpt2.rs:358-399 is
the reference's per-step API, used by generate_with_config's loop,
gpt2.rs:447-474). So every decode step's full logits row can be held to the
bar: |d| <= 1e-3 + 1e-4 |ref| over all vocab_size entries. The token
sequence is the GPU's own greedy output (teacher forcing on the oracle side),
and the step's argmax must be the token generate_cached chose, since both
entry points run the same kernel on the same inputs.
"""
import os

import numpy as np
import pytest

from rusttorch_amd import synth
from rusttorch_amd.gpt2 import Gpt2Config, Gpt2Model

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-4
THREADS = min(16, os.cpu_count() or 1)


def cfg_of(sh):
    return Gpt2Config(sh.vocab_size, sh.n_positions, sh.n_embd, sh.n_layer, sh.n_head, sh.layer_norm_epsilon)


def excess_and_diff(got, ref):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    return float(np.max(d - (ATOL + RTOL * np.abs(ref)))), float(np.max(d))


def _steps_against_oracle(om, m, ids, n_prompt, check_rows, what):
    """Prefill ids[:n_prompt] on both sides, then feed ids[n_prompt:-1] one
    token at a time through the GPU's forward_cached (the persistent step).
    The oracle processes the same tokens in chunks of 64 (its rows do not
    depend on the chunking: every element is summed in the same k order) and
    the GPU's rows at the steps in check_rows are compared. Returns the
    largest |d| and the per-step list."""
    c = m.new_cache()
    m.forward_cached(ids[:n_prompt], c)
    oc = om.new_cache()
    om.forward_cached(ids[:n_prompt], oc)
    toks = [int(t) for t in ids[n_prompt:-1]]
    worst, diffs = 0.0, []
    for base in range(0, len(toks), 64):
        chunk = toks[base:base + 64]
        ref_rows = om.forward_cached(chunk, oc)
        for j, tok in enumerate(chunk):
            s = base + j
            got = m.forward_cached([tok], c)[0]
            if s not in check_rows:
                continue
            excess, diff = excess_and_diff(got, ref_rows[j])
            assert excess <= 0, f"{what} decode step {s} (position {n_prompt + s}): max excess {excess:.3e}, " \
                                f"max |d| {diff:.3e}"
            # the step's argmax is the token generate_cached chose at this step
            assert int(np.argmax(got)) == int(ids[n_prompt + s + 1]), f"{what} step {s}: argmax differs from generate"
            worst = max(worst, diff)
            diffs.append(diff)
    assert c.len() == len(ids) - 1
    c.close()
    return worst, diffs


def test_c1_every_decode_step_logits(oracle_lib):
    """c1: GPT-2 small, prompt 32, 64 greedy tokens. All 63 decode steps'
    logits rows (50257 each) from the persistent step against the oracle."""
    sh = synth.SHAPES["small"]
    sd = synth.make_weights(sh)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    prompt = synth.make_tokens(32, sh.vocab_size)
    ids = m.generate_cached(prompt, 64, 0.0)
    print("[gpu] c1 per-step logits", flush=True)
    worst, diffs = _steps_against_oracle(om, m, ids, 32, set(range(63)), "c1")
    assert len(diffs) == 63
    print(f"[gpu] c1 persistent step: 63 decode steps, max |d| {worst:.3e}, median {np.median(diffs):.3e}",
          flush=True)
    m.close()


def test_c3_logits_to_full_context(oracle_lib):
    """c3: GPT-2 medium, prompt 512, 512 greedy tokens (positions up to
    1023). The persistent step's logits at every 64th decode step and the
    last, against the oracle along the GPU's token sequence."""
    sh = synth.SHAPES["medium"]
    sd = synth.make_weights(sh)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    prompt = synth.make_tokens(512, sh.vocab_size, stream=620)
    print("[gpu] c3 generate 512 + per-step logits", flush=True)
    ids = m.generate_cached(prompt, 512, 0.0)
    rows = set(range(0, 511, 64)) | {510}
    worst, diffs = _steps_against_oracle(om, m, ids, 512, rows, "c3")
    assert len(diffs) == len(rows)
    print(f"[gpu] c3 persistent step: {len(rows)} decode steps up to position 1022, max |d| {worst:.3e}",
          flush=True)
    m.close()


@pytest.mark.parametrize("name,storage,steps", [("large", "f32", 8), ("xl", "bf16", 8)])
def test_wide_persistent_step_logits(oracle_lib, name, storage, steps):
    """The persistent step at GPT-2 large (f32) and XL (bf16-rounded weights,
    the oracle fed the same values): a 24-token prompt, then every decode
    step's logits for `steps` greedy tokens."""
    sh = synth.SHAPES[name]
    sd = synth.make_weights(sh, bf16=(storage == "bf16"))
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh), storage=storage)
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    prompt = synth.make_tokens(24, sh.vocab_size, stream=660)
    ids = m.generate_cached(prompt, steps + 1, 0.0)
    worst, diffs = _steps_against_oracle(om, m, ids, 24, set(range(steps)), f"{name} {storage}")
    assert len(diffs) == steps
    print(f"[gpu] {name} {storage} persistent step: {steps} decode steps, max |d| {worst:.3e}", flush=True)
    m.close()


@pytest.mark.parametrize("vocab,d,heads", [(1000, 768, 12), (300, 128, 2)])
def test_persistent_step_smaller_vocabulary(oracle_lib, monkeypatch, tmp_path, vocab, d, heads):
    """A vocabulary below the one a persistent instance is compiled for
    (50257 at d = 768, 512 at d = 128) runs on that instance, the LM head's
    rows on the first workgroups only: every decode step's logits against
    the oracle, and the persistent step is the one that ran (it writes its
    phase trace when RTG_TRACE_FILE is set)."""
    sh = synth.ModelShape(vocab, 128, d, 2, heads)
    sd = synth.make_weights(sh)
    trace = tmp_path / "trace.bin"
    monkeypatch.setenv("RTG_TRACE_FILE", str(trace))
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    prompt = synth.make_tokens(20, vocab, stream=690)
    ids = m.generate_cached(prompt, 17, 0.0)
    assert trace.exists(), "the persistent step did not run"
    worst, diffs = _steps_against_oracle(om, m, ids, 20, set(range(16)), f"V={vocab} d={d}")
    assert len(diffs) == 16
    print(f"[gpu] V={vocab} d={d} persistent step: 16 decode steps, max |d| {worst:.3e}", flush=True)
    m.close()


def test_small_generate_equals_generate_cached():
    """The reference harness's check at model size (examples/gpt2_bench.rs:
    53-70): GPT-2 small, uncached generate (a full forward over the window
    per token) against generate_cached (the persistent step per token) over
    30 greedy tokens."""
    sh = synth.SHAPES["small"]
    m = Gpt2Model.from_state_dict(synth.make_weights(sh), cfg_of(sh))
    prompt = synth.make_tokens(16, sh.vocab_size, stream=670).tolist()
    a = m.generate(prompt, 30, 0.0)
    b = m.generate_cached(prompt, 30, 0.0)
    assert a == b
    m.close()


def test_tiled_step_logits(oracle_lib, monkeypatch):
    """The tiled persistent step (opt-in, RTG_TILE_STEP=1 at model creation:
    16 x 16 weight tiles per layer matrix, each LayerNorm folded on exact
    per-block statistics): c1's 63 decode steps, and 8 steps of GPT-2 small
    with wpe offset by 30 (|mean| / std of the residual about 1000), every
    logits row against the oracle; ids equal the row-split step's."""
    monkeypatch.setenv("RTG_TILE_STEP", "1")
    sh = synth.SHAPES["small"]
    sd = synth.make_weights(sh)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    prompt = synth.make_tokens(32, sh.vocab_size)
    ids = m.generate_cached(prompt, 64, 0.0)
    worst, diffs = _steps_against_oracle(om, m, ids, 32, set(range(63)), "c1 tiled")
    print(f"[gpu] c1 tiled step: 63 decode steps, max |d| {worst:.3e}", flush=True)
    m.close()
    monkeypatch.delenv("RTG_TILE_STEP")
    ref = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    assert ref.generate_cached(prompt, 64, 0.0) == ids
    ref.close()
    monkeypatch.setenv("RTG_TILE_STEP", "1")
    sd = dict(sd)
    sd["wpe.weight"] = (sd["wpe.weight"] + np.float32(30.0)).astype(np.float32)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    ids = m.generate_cached(prompt, 9, 0.0)
    worst, _ = _steps_against_oracle(om, m, ids, 32, set(range(8)), "offset-30 tiled")
    print(f"[gpu] tiled step, wpe offset 30: 8 decode steps, max |d| {worst:.3e}", flush=True)
    m.close()

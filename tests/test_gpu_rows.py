"""The multi-row forward (rows_kernel.h): forward_cached over at most 32 rows
in one launch (gpt2.rs:358-399 over a short prompt, or a few tokens of each
sequence of a batched cache), against the CPU oracle at the logits bar
|d| <= 1e-3 + 1e-4 |ref| on every row, and against the per-op prefill
kernels (RTG_NO_ROWS=1) for the greedy ids that generate_cached derives from
the same launch (its argmax and finalize run inside it).

Covered: prompts of 2..32 tokens at position 0; chunks appended behind a
cache longer than one 64-key block (attention over cache rows and new rows),
and behind up to 6 blocks (cached keys split between an item's waves);
S sequences x T tokens with S*T = 32 on a batched cache; the two code paths
of the kernel (n_embd 768: activations through LDS; 1024: in registers)
and the 128-wide mini model.
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


def check_rows(got, ref, what):
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    excess = float(np.max(d - (ATOL + RTOL * np.abs(ref))))
    assert excess <= 0, f"{what}: max excess {excess:.3e}, max |d| {d.max():.3e}"
    return float(d.max())


@pytest.mark.parametrize("name,chunks", [("mini", (2, 5, 17, 32)), ("small", (2, 5, 17, 32, 31)),
                                         ("medium", (2, 5, 17, 32, 31))])
def test_prompt_chunks_against_oracle(oracle_lib, name, chunks):
    """Chunks of 2 to 32 tokens fed in turn; at small and medium the last one
    attends over more than one 64-key block of cached rows plus its own rows
    (mini holds 64 positions)."""
    sh = synth.SHAPES[name]
    sd = synth.make_weights(sh)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    c, oc = m.new_cache(), om.new_cache()
    worst = 0.0
    for i, n in enumerate(chunks):
        ids = synth.make_tokens(n, sh.vocab_size, stream=900 + i)
        print(f"[gpu] rows {name}: chunk {i} of {n} tokens at position {c.len()}", flush=True)
        got = m.forward_cached(ids, c)
        ref = om.forward_cached(ids, oc)
        worst = max(worst, check_rows(got, ref, f"{name} chunk {i} (n={n}, past={c.len() - n})"))
    assert c.len() == sum(chunks)
    print(f"[gpu] rows {name}: {sum(chunks)} rows over {len(chunks)} chunks, max |d| {worst:.3e}", flush=True)
    c.close()
    m.close()


@pytest.mark.parametrize("name", ["mini", "small"])
def test_chunks_behind_long_cache(oracle_lib, name):
    """Chunks behind a cache of several 64-key blocks: the cached keys are
    split between the four waves of each attention item (one to three blocks
    each) for all of the item's queries, and the waves' softmax states are
    merged; every chunk's rows against the oracle, the later ones at 256 and
    more cached positions (mini holds 64 positions: one to its end)."""
    sh = synth.SHAPES[name]
    sd = synth.make_weights(sh)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    chunks = (32, 30, 2) if name == "mini" else (32,) * 8 + (31, 7, 32, 3)
    c, oc = m.new_cache(), om.new_cache()
    worst = 0.0
    for i, n in enumerate(chunks):
        ids = synth.make_tokens(n, sh.vocab_size, stream=990 + i)
        got = m.forward_cached(ids, c)
        ref = om.forward_cached(ids, oc)
        if c.len() - n >= 64 or name == "mini":
            worst = max(worst, check_rows(got, ref, f"{name} chunk {i} (n={n}, past={c.len() - n})"))
    print(f"[gpu] rows {name}: chunks up to position {c.len()}, max |d| {worst:.3e}", flush=True)
    c.close()
    m.close()


@pytest.mark.parametrize("S,T", [(4, 8), (16, 2), (2, 16)])
def test_batched_chunks_against_oracle(oracle_lib, S, T):
    """S sequences x T tokens (S * T = 32) on a batch-S cache, twice (the
    second call behind the first): every sequence's rows against the oracle
    run on that sequence alone."""
    sh = synth.SHAPES["small"]
    sd = synth.make_weights(sh)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    c = m.new_cache(S)
    ocs = [om.new_cache() for _ in range(S)]
    for call in range(2):
        ids = synth.make_tokens(S * T, sh.vocab_size, stream=950 + call).reshape(S, T)
        print(f"[gpu] rows S={S} T={T}: call {call}", flush=True)
        got = m.forward_cached_batched(ids, c)
        checked = sorted({0, S // 2, S - 1})
        for s in range(S):
            ref = om.forward_cached(ids[s], ocs[s])
            if s in checked:
                check_rows(got[s], ref, f"S={S} T={T} call {call} sequence {s}")
    c.close()
    m.close()


def test_greedy_finish_matches_per_op_path(monkeypatch):
    """generate_cached's prefill with the argmax and finalize inside the
    multi-row launch, against the per-op prefill kernels plus the argmax and
    finalize kernels: the same greedy ids, at batch 1 (c1's shape), for 4
    sequences of 8 tokens (both with the last-row LM head) and for 8 of 4
    (the all-rows LM head)."""
    sh = synth.SHAPES["small"]
    m = Gpt2Model.from_state_dict(synth.make_weights(sh), cfg_of(sh))
    prompt = synth.make_tokens(32, sh.vocab_size)
    prompts = synth.make_tokens(32, sh.vocab_size, stream=970).reshape(4, 8)
    wide = synth.make_tokens(32, sh.vocab_size, stream=971).reshape(8, 4)
    a1 = m.generate_cached(prompt, 16, 0.0)
    ab = m.generate_cached_batched(prompts, 8)
    aw = m.generate_cached_batched(wide, 8)  # 8 sequences: the all-rows LM head, keys of 8 rows
    monkeypatch.setenv("RTG_NO_ROWS", "1")
    b1 = m.generate_cached(prompt, 16, 0.0)
    bb = m.generate_cached_batched(prompts, 8)
    bw = m.generate_cached_batched(wide, 8)
    assert a1 == b1
    assert np.array_equal(ab, bb)
    assert np.array_equal(aw, bw)
    m.close()


def test_rows_and_per_op_logits_agree(monkeypatch):
    """The same 32-token prompt through the multi-row launch and through the
    per-op prefill kernels: both compute the reference's sums in f32, in
    different orders, so the logits differ by rounding only."""
    sh = synth.SHAPES["small"]
    m = Gpt2Model.from_state_dict(synth.make_weights(sh), cfg_of(sh))
    ids = synth.make_tokens(32, sh.vocab_size, stream=980)
    c = m.new_cache()
    a = m.forward_cached(ids, c)
    c.clear()
    monkeypatch.setenv("RTG_NO_ROWS", "1")
    b = m.forward_cached(ids, c)
    d = float(np.max(np.abs(a - b)))
    print(f"[gpu] rows vs per-op prefill: max |d| {d:.3e}", flush=True)
    assert d < 1e-4
    c.close()
    m.close()

"""The bounded waits of the two one-launch kernels end in an error, not a
hang. Test hooks make one wait target a value that no producer writes: the
multi-row forward's wait with a given code (RTG_TEST_ROWS_WAIT=<code>), the
persistent decode step's layer-1 input fetch (RTG_TEST_DECODE_WAIT=<polling
rounds>). The wait runs out its bounded polling rounds, every other wait of
the launch returns at once once the error word is set, the kernel finishes,
the host turns the word into an error (and clears it), and the next call on
the same model and cache runs normally and matches the oracle or a run
before the failure."""
import os

import numpy as np
import pytest

from rusttorch_amd import synth
from rusttorch_amd._lib import Gpt2Error
from rusttorch_amd.gpt2 import Gpt2Config, Gpt2Model

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-3, 1e-4
THREADS = min(16, os.cpu_count() or 1)


def cfg_of(sh):
    return Gpt2Config(sh.vocab_size, sh.n_positions, sh.n_embd, sh.n_layer, sh.n_head, sh.layer_norm_epsilon)


@pytest.mark.parametrize("code", [1, 5, 8])
def test_rows_wait_timeout_is_an_error(oracle_lib, monkeypatch, code):
    """Code 1: c_attn's wait for the row phases; 5: c_fc's; 8: the LM head's
    wait for ln_f. The failed call raises and leaves the cache length as it
    was; the next call matches the oracle."""
    sh = synth.SHAPES["mini"]
    sd = synth.make_weights(sh)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=THREADS)
    ids = synth.make_tokens(12, sh.vocab_size, stream=1100 + code)
    c = m.new_cache()
    print(f"[gpu] rows forced timeout, wait code {code}", flush=True)
    monkeypatch.setenv("RTG_TEST_ROWS_WAIT", str(code))
    # the forced wait times out, and so may the waits downstream of it that
    # started polling at about the same time: the word holds one of their codes
    with pytest.raises(Gpt2Error, match=r"multi-row forward timed out waiting for a peer \(phase [1-8]\)"):
        m.forward_cached(ids, c)
    monkeypatch.delenv("RTG_TEST_ROWS_WAIT")
    assert c.len() == 0
    got = np.asarray(m.forward_cached(ids, c), np.float64)
    ref = np.asarray(om.forward_cached(ids, om.new_cache()), np.float64)
    d = np.abs(got - ref)
    assert float(np.max(d - (ATOL + RTOL * np.abs(ref)))) <= 0, f"max |d| {d.max():.3e}"
    c.close()
    m.close()


def test_decode_wait_timeout_is_an_error(monkeypatch):
    """The persistent decode step behind generate_cached (GPT-2 small):
    the failed call raises, and the next call produces the ids of a run made
    before the failure."""
    sh = synth.SHAPES["small"]
    m = Gpt2Model.from_state_dict(synth.make_weights(sh), cfg_of(sh))
    prompt = synth.make_tokens(8, sh.vocab_size, stream=1110)
    want = m.generate_cached(prompt, 6, 0.0)
    print("[gpu] decode forced timeout", flush=True)
    monkeypatch.setenv("RTG_TEST_DECODE_WAIT", "20000")
    with pytest.raises(Gpt2Error, match=r"persistent decode step timed out waiting for a peer \(code 1\)"):
        m.generate_cached(prompt, 6, 0.0)
    monkeypatch.delenv("RTG_TEST_DECODE_WAIT")
    assert m.generate_cached(prompt, 6, 0.0) == want
    m.close()

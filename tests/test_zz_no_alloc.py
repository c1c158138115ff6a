"""rtg_forward_cached_noalloc (the entry point that allocates nothing) against
rtg_forward_cached, both called through the C ABI: the same kernels on the
same inputs, so the logits must be bit-identical, on two calls in a row (a
20-token prompt, then a smaller 1-token step) and on a second model width;
the cache advances the same way; a size beyond the scratch array is an
error; and both agree with the CPU oracle within the logits tolerance."""
import ctypes as C

import numpy as np
import pytest

from rusttorch_amd import _lib, synth
from rusttorch_amd.gpt2 import Gpt2Config, Gpt2Error, Gpt2Model, check

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20


def cfg_of(sh):
    return Gpt2Config(sh.vocab_size, sh.n_positions, sh.n_embd, sh.n_layer, sh.n_head, sh.layer_norm_epsilon)


def call(fn_name, m, cache, ids, vocab):
    lib = _lib.load()
    ids = np.ascontiguousarray(np.asarray(ids, np.uint32))
    out = np.empty((ids.size, vocab), dtype=np.float32)
    check(getattr(lib, fn_name)(m._h, cache._h, ids.ctypes.data_as(C.c_void_p), ids.size,
                                out.ctypes.data_as(C.c_void_p)))
    return out


@pytest.mark.parametrize("name", ["mini", "small"])
def test_noalloc_matches_forward_cached(oracle_lib, name):
    sh = synth.SHAPES[name]
    sd = synth.make_weights(sh)
    m = Gpt2Model.from_state_dict(sd, cfg_of(sh))
    om = oracle_lib.OracleModel.from_shape(sd, sh, threads=8)
    ids = synth.make_tokens(21, sh.vocab_size, stream=800)
    print(f"[gpu] noalloc {name}", flush=True)
    ca, cb, co = m.new_cache(), m.new_cache(), om.new_cache()
    for chunk in (ids[:20], ids[20:]):  # two calls, the second smaller
        a = call("rtg_forward_cached_noalloc", m, ca, chunk, sh.vocab_size)
        b = call("rtg_forward_cached", m, cb, chunk, sh.vocab_size)
        assert np.array_equal(a, b), f"{name}: noalloc logits differ (max |d| {np.max(np.abs(a - b)):.3e})"
        assert ca.len() == cb.len()
        ref = om.forward_cached(chunk, co)
        excess = np.max(np.abs(a - ref) - (1e-3 + 1e-4 * np.abs(ref)))
        assert excess <= 0, f"{name}: max excess {excess:.3e} against the oracle"
    # the caches hold the same keys and values
    for layer in (0, sh.n_layer - 1):
        assert np.array_equal(ca.read(layer, 0), cb.read(layer, 0))
        assert np.array_equal(ca.read(layer, 1, values=True), cb.read(layer, 1, values=True))
    ca.close()
    cb.close()
    m.close()


def test_noalloc_rejects_sizes_beyond_scratch():
    sh = synth.SHAPES["small"]
    m = Gpt2Model.from_state_dict(synth.make_weights(sh), cfg_of(sh))
    c = m.new_cache()
    per_token = 4 * (10 * sh.n_embd + sh.vocab_size)
    n = SCRATCH_BYTES // per_token + 1  # 73 tokens of GPT-2 small
    with pytest.raises(Gpt2Error, match="need .* bytes of scratch; it holds 16777216"):
        call("rtg_forward_cached_noalloc", m, c, synth.make_tokens(n, sh.vocab_size), sh.vocab_size)
    assert c.len() == 0
    with pytest.raises(Gpt2Error, match="^Empty input$"):
        call("rtg_forward_cached_noalloc", m, c, [], sh.vocab_size)
    # the largest size that fits still runs
    out = call("rtg_forward_cached_noalloc", m, c, synth.make_tokens(n - 1, sh.vocab_size), sh.vocab_size)
    assert out.shape == (n - 1, sh.vocab_size) and np.isfinite(out).all()
    c.close()
    m.close()

"""rtg_forward_cached_noalloc (the entry point that allocates nothing) against
rtg_forward_cached, both called through the C ABI: for n >= 2 the same
prefill kernels on the same inputs, so the logits must be bit-identical, on
two calls in a row (a 20-token prompt, then a smaller 2-token call) and on a
second model width; a third, 1-token call (rtg_forward_cached then runs the
persistent decode step) agrees within the logits tolerance; the cache
advances the same way; a size beyond the scratch array is an error, a cache
of another model is refused; and both agree with the CPU oracle within the
logits tolerance."""
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
    ids = synth.make_tokens(23, sh.vocab_size, stream=800)
    print(f"[gpu] noalloc {name}", flush=True)
    ca, cb, co = m.new_cache(), m.new_cache(), om.new_cache()
    for chunk in (ids[:20], ids[20:22], ids[22:]):  # three calls, each smaller than the one before
        a = call("rtg_forward_cached_noalloc", m, ca, chunk, sh.vocab_size)
        b = call("rtg_forward_cached", m, cb, chunk, sh.vocab_size)
        if len(chunk) > 1:
            assert np.array_equal(a, b), f"{name}: noalloc logits differ (max |d| {np.max(np.abs(a - b)):.3e})"
        assert ca.len() == cb.len()
        ref = om.forward_cached(chunk, co)
        for got, what in ((a, "noalloc"), (b, "forward_cached")):
            excess = np.max(np.abs(got - ref) - (1e-3 + 1e-4 * np.abs(ref)))
            assert excess <= 0, f"{name} {what} n={len(chunk)}: max excess {excess:.3e} against the oracle"
    # the caches hold the same keys and values: bit for bit where the same
    # prefill kernels wrote them, within 1e-4 in the row of the 1-token call
    for layer in (0, sh.n_layer - 1):
        for a, b in ((ca.read(layer, 0), cb.read(layer, 0)),
                     (ca.read(layer, 1, values=True), cb.read(layer, 1, values=True))):
            assert np.array_equal(a[:22], b[:22])
            np.testing.assert_allclose(a[22], b[22], atol=1e-4, rtol=1e-4)
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
    # a cache of another model is refused before anything runs
    other = Gpt2Model.from_state_dict(synth.make_weights(synth.SHAPES["mini"]), cfg_of(synth.SHAPES["mini"]))
    oc = other.new_cache()
    with pytest.raises(Gpt2Error, match="the cache belongs to another model"):
        call("rtg_forward_cached_noalloc", m, oc, [1, 2], sh.vocab_size)
    assert oc.len() == 0
    oc.close()
    other.close()
    c.close()
    m.close()


def test_noalloc_limit_is_monotone_at_large_and_xl():
    """The limit is the activations' size alone (the split-k partials use what
    is left, else the GEMMs run unsplit): every n up to the bound is
    accepted, the next is refused. Checked on the host-side arithmetic the
    library states for GPT-2 large and XL widths, and run at the bound on a
    2-layer model of XL's width."""
    def fits(n, d, V):
        up = lambda x: (x + 63) // 64 * 64  # noqa: E731
        return 3 * up(n * d) + up(3 * n * d) + up(4 * n * d) + up(n * V) <= SCRATCH_BYTES // 4
    for d, want in ((1280, 66), (1600, 63)):
        bound = max(n for n in range(1, 200) if fits(n, d, 50257))
        assert bound == want and all(fits(n, d, 50257) for n in range(1, bound + 1))
    sh = synth.ModelShape(50257, 128, 1600, 2, 25)
    m = Gpt2Model.from_state_dict(synth.make_weights(sh), cfg_of(sh))
    for n in (57, 63):  # sizes whose split-k partials do not fit beside the activations
        c = m.new_cache()
        out = call("rtg_forward_cached_noalloc", m, c, synth.make_tokens(n, sh.vocab_size, stream=n), sh.vocab_size)
        assert out.shape == (n, sh.vocab_size) and np.isfinite(out).all()
        c.close()
    c = m.new_cache()
    with pytest.raises(Gpt2Error, match="need .* bytes of scratch"):
        call("rtg_forward_cached_noalloc", m, c, synth.make_tokens(64, sh.vocab_size), sh.vocab_size)
    c.close()
    m.close()

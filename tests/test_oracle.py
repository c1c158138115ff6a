"""Pins for the CPU oracle (oracle/gpt2_oracle.c) before it is trusted.

1. rusttorch's own GPT-2 unit tests (rusttorch-core/src/nn/gpt2.rs:1019-1660),
   restated against the oracle with the reference's constant-valued state
   dict and tiny config.
2. Closed forms / brute force in float64 for each helper.
3. Whole-model pins: a float64 numpy restatement written from the maths
   (tests/ref64.py) and a locally constructed transformers GPT2LMHeadModel
   (eager attention, same weights).
4. The committed golden fixtures (tests/golden/).
"""
import os

import numpy as np
import pytest

from rusttorch_amd import synth
from tests import ref64

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---------------------------------------------------------------------------
# the reference's test model (gpt2.rs:1023-1082)
# ---------------------------------------------------------------------------

def small_config():
    return synth.SHAPES["tiny"]  # vocab 10, n_pos 16, d 8, 2 layers, 2 heads


def small_state_dict(cfg):
    n, ff = cfg.n_embd, 4 * cfg.n_embd
    sd = {"wte.weight": np.full((cfg.vocab_size, n), 0.1, np.float32),
          "wpe.weight": np.full((cfg.n_positions, n), 0.01, np.float32),
          "ln_f.weight": np.ones(n, np.float32), "ln_f.bias": np.zeros(n, np.float32)}
    for i in range(cfg.n_layer):
        p = f"h.{i}."
        sd[p + "ln_1.weight"] = np.ones(n, np.float32)
        sd[p + "ln_1.bias"] = np.zeros(n, np.float32)
        sd[p + "attn.c_attn.weight"] = np.full((n, 3 * n), 0.01, np.float32)
        sd[p + "attn.c_attn.bias"] = np.zeros(3 * n, np.float32)
        sd[p + "attn.c_proj.weight"] = np.full((n, n), 0.01, np.float32)
        sd[p + "attn.c_proj.bias"] = np.zeros(n, np.float32)
        sd[p + "ln_2.weight"] = np.ones(n, np.float32)
        sd[p + "ln_2.bias"] = np.zeros(n, np.float32)
        sd[p + "mlp.c_fc.weight"] = np.full((n, ff), 0.01, np.float32)
        sd[p + "mlp.c_fc.bias"] = np.zeros(ff, np.float32)
        sd[p + "mlp.c_proj.weight"] = np.full((ff, n), 0.01, np.float32)
        sd[p + "mlp.c_proj.bias"] = np.zeros(n, np.float32)
    return sd


@pytest.fixture(scope="module")
def O(oracle_lib):
    return oracle_lib


@pytest.fixture(scope="module")
def const_model(O):
    cfg = small_config()
    return O.OracleModel.from_shape(small_state_dict(cfg), cfg)


@pytest.fixture(scope="module")
def rand_tiny(O):
    cfg = small_config()
    sd = synth.make_weights(cfg)
    return sd, O.OracleModel.from_shape(sd, cfg)


# ---------------------------------------------------------------------------
# 1. ported reference tests
# ---------------------------------------------------------------------------

def test_gpt2_config_small():  # gpt2.rs:1085-1092
    c = synth.SHAPES["small"]
    assert (c.vocab_size, c.n_embd, c.n_layer, c.n_head, c.n_positions) == (50257, 768, 12, 12, 1024)


def test_forward_shape(const_model):  # :1103-1110
    assert const_model.forward([0, 1, 2]).shape == (3, 10)


def test_forward_single_token(const_model):  # :1113-1120
    assert const_model.forward([0]).shape == (1, 10)


def test_forward_empty_fails(const_model, O):  # :1123-1129
    with pytest.raises(O.OracleError, match="Empty input"):
        const_model.forward([])


def test_forward_too_long_fails(const_model, O):  # :1132-1139
    with pytest.raises(O.OracleError, match="Sequence length 20 exceeds max position 16"):
        const_model.forward(list(range(20)))


def test_generate_greedy_length(const_model):  # :1142-1149
    assert len(const_model.generate([0, 1], 3)) == 5


def test_num_parameters(const_model):  # :1165-1171
    assert const_model.num_parameters() == synth.num_parameters(small_config()) > 0


def test_embedding_lookup(O):  # :1174-1183
    w = np.array([[1, 2], [3, 4], [5, 6]], np.float32)
    assert O.embedding_lookup(w, [2, 0]).tolist() == [[5, 6], [1, 2]]


def test_embedding_lookup_out_of_range(O):  # :1186-1189
    with pytest.raises(O.OracleError, match=r"Token ID 5 out of range \(vocab_size=1\)"):
        O.embedding_lookup(np.array([[1, 2]], np.float32), [5])


def test_layer_norm_zero_mean(O):  # :1192-1201
    out = O.layer_norm(np.array([[1, 2], [3, 4]], np.float32), [1, 1], [0, 0])
    assert abs(out[0, 0] + out[0, 1]) < 0.01 and abs(out[1, 0] + out[1, 1]) < 0.01


def test_slice_columns(O):  # :1204-1212
    t = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    assert O.slice_columns(t, 1, 3).tolist() == [[2, 3], [5, 6]]


def test_gelu_new_values(O):  # :1215-1222
    g = O.gelu_new([0.0, 1.0, -1.0, 3.0])
    assert abs(g[0]) < 0.01 and abs(g[1] - 0.841) < 0.01 and abs(g[2] + 0.159) < 0.01


def test_conv1d_forward(O):  # :1225-1231
    y = O.conv1d(np.array([[1, 2], [3, 4]], np.float32), np.array([[1, 0, 0], [1, 0, 0]], np.float32).reshape(2, 3),
                 [0.1, 0.2, 0.3])
    assert y.shape == (2, 3)


def test_argmax(O):  # :1234-1238
    assert O.argmax([1.0, 3.0, 2.0]) == 1
    assert O.argmax([5.0, 1.0, 2.0]) == 0
    assert O.argmax([1.0, 2.0, 5.0]) == 2


def test_argmax_special_cases(O):  # strict '>' from -inf (:858-868)
    assert O.argmax([2.0, 2.0]) == 0
    assert O.argmax([np.nan, 1.0, np.nan]) == 1
    assert O.argmax([np.nan, np.nan]) == 0
    assert O.argmax([-np.inf, -np.inf]) == 0


def test_top2_gap_brute_force(O):
    """The near-tie diagnostic: top-1 minus top-2 over the values above
    -inf with NaN skipped, 0 for a tie at the top, against a sort."""
    assert O.top2_gap([1.0, 3.0, 3.0]) == 0.0
    assert O.top2_gap([np.nan, 2.0, 1.5]) == 0.5
    assert O.top2_gap([1.0]) == np.inf and O.top2_gap([-np.inf, 4.0]) == np.inf
    rng = np.random.default_rng(11)
    for _ in range(200):
        x = rng.standard_normal(int(rng.integers(2, 300))).astype(np.float32)
        x[rng.random(x.size) < 0.05] = np.nan
        v = np.sort(x[~np.isnan(x)])
        if v.size >= 2:
            assert O.top2_gap(x) == np.float32(v[-1] - v[-2])


def test_generate_cached_gaps_follow_the_rows(rand_tiny, O):
    """generate_cached(gaps=True): same ids as without, and gap s is the
    top-2 gap of the row greedy step s chose from (teacher forcing)."""
    _, om = rand_tiny
    prompt = [1, 5, 9]
    ids, gaps = om.generate_cached(prompt, 6, gaps=True)
    assert ids == om.generate_cached(prompt, 6) and gaps.shape == (6,)
    c = om.new_cache()
    row = om.forward_cached(prompt, c)[-1]
    for s in range(6):
        assert gaps[s] == np.float32(O.top2_gap(row))
        row = om.forward_cached([ids[3 + s]], c)[0]


def test_deterministic_greedy(const_model):  # :1248-1257
    assert const_model.generate([0, 1], 5) == const_model.generate([0, 1], 5)


def test_missing_weight_error(O):  # :1260-1267
    c = small_config()
    with pytest.raises(O.OracleError, match="Missing weight: wte.weight"):
        O.OracleModel.from_shape({}, c)


def test_mha_single_token(O):  # :1270-1277
    q = np.full((1, 8), 0.1, np.float32)
    assert O.multi_head_attention(q, q, q, 2, 4, 1).shape == (1, 8)


def test_mha_causal(O):  # :1280-1291
    q = np.array([[1, 0, 0, 1], [0, 1, 1, 0]], np.float32)
    v = np.array([[1, 2, 3, 4], [5, 6, 7, 8]], np.float32)
    out = O.multi_head_attention(q, q, v, 2, 2, 2)
    assert abs(out[0, 0] - 1.0) < 0.01 and abs(out[0, 1] - 2.0) < 0.01


def test_repetition_penalty(O):  # :1321-1347
    l = O.apply_repetition_penalty([5.0, 3.0, 1.0, 0.5], [0, 2], 2.0)
    assert np.allclose(l, [2.5, 3.0, 0.5, 0.5])
    assert np.allclose(O.apply_repetition_penalty([-2.0, 3.0], [0], 2.0), [-4.0, 3.0])
    assert O.apply_repetition_penalty([5.0, 3.0], [0], 1.0).tolist() == [5.0, 3.0]


def test_top_k(O):  # :1350-1368
    l = O.apply_top_k([1.0, 5.0, 3.0, 2.0, 4.0], 3)
    assert l[0] == -np.inf and l[3] == -np.inf and l[1] == 5 and l[2] == 3 and l[4] == 4
    assert O.apply_top_k([1.0, 2.0, 3.0], 10).tolist() == [1.0, 2.0, 3.0]


def test_top_p(O):  # :1371-1399
    l = O.apply_top_p([10.0, 1.0, 1.0, 1.0], 0.9)
    assert l[0] == 10 and np.all(np.isneginf(l[1:]))
    l = O.apply_top_p([5.0, 5.0, -100.0, -100.0], 0.9)
    assert l[0] == 5 and l[1] == 5 and np.all(np.isneginf(l[2:]))
    assert O.apply_top_p([1.0, 2.0, 3.0], 1.0).tolist() == [1.0, 2.0, 3.0]


def test_kv_cache_new_and_clear(const_model):  # :1445-1470
    c = const_model.new_cache()
    assert c.len() == 0 and c.is_empty()
    const_model.forward_cached([0, 1], c)
    assert c.len() == 2
    c.clear()
    assert c.is_empty()


def test_kv_cache_append_layout(rand_tiny):  # LayerKVCache::append (:1473-1503)
    sd, m = rand_tiny
    c = m.new_cache()
    m.forward_cached([3, 1, 4], c)
    # keys of head h at position t are the k-columns h*hd.. of that token's
    # c_attn output, computed here in float64
    d, H = 8, 2
    x = sd["wte.weight"][[3, 1, 4]].astype(np.float64) + sd["wpe.weight"][:3]
    h = ref64.layer_norm(x, sd["h.0.ln_1.weight"], sd["h.0.ln_1.bias"], 1e-5)
    qkv = h @ sd["h.0.attn.c_attn.weight"] + sd["h.0.attn.c_attn.bias"]
    for head in range(H):
        np.testing.assert_allclose(c.read(0, head), qkv[:, d + head * 4: d + head * 4 + 4], atol=1e-6)
        np.testing.assert_allclose(c.read(0, head, values=True), qkv[:, 2 * d + head * 4: 2 * d + head * 4 + 4],
                                   atol=1e-6)


def _last_rows_close(a, b, tol=1e-4):
    assert np.max(np.abs(a - b)) < tol


def test_forward_cached_matches_forward(rand_tiny):  # :1506-1532
    _, m = rand_tiny
    toks = [0, 1, 2, 3]
    c = m.new_cache()
    _last_rows_close(m.forward(toks)[-1], m.forward_cached(toks, c)[-1])


def test_forward_cached_incremental(rand_tiny):  # :1535-1560
    _, m = rand_tiny
    toks = [0, 1, 2, 3, 4]
    c = m.new_cache()
    m.forward_cached(toks[:3], c)
    _last_rows_close(m.forward(toks)[-1], m.forward_cached(toks[3:], c)[1])


def test_forward_cached_single_steps(rand_tiny):  # :1563-1588
    _, m = rand_tiny
    c = m.new_cache()
    m.forward_cached([0], c)
    m.forward_cached([1], c)
    _last_rows_close(m.forward([0, 1, 2])[2], m.forward_cached([2], c)[0])


def test_generate_cached_matches_generate(rand_tiny, const_model):  # :1591-1602
    for m in (rand_tiny[1], const_model):
        assert m.generate([0, 1], 5) == m.generate_cached([0, 1], 5)


def test_generate_cached_length(const_model):  # :1605-1612
    assert len(const_model.generate_cached([0, 1, 2], 7)) == 10
    assert len(const_model.generate_cached([0, 1, 2], 0)) == 4  # prefill token is always pushed


def test_forward_cached_updates_cache_length(const_model):  # :1615-1628
    c = const_model.new_cache()
    const_model.forward_cached([0, 1, 2], c)
    assert c.len() == 3
    const_model.forward_cached([3], c)
    assert c.len() == 4


def test_forward_cached_exceeds_max_position(const_model, O):  # :1631-1648
    c = const_model.new_cache()
    const_model.forward_cached([i % 10 for i in range(15)], c)
    const_model.forward_cached([0], c)
    assert c.len() == 16
    with pytest.raises(O.OracleError, match="Total sequence length 17 exceeds max position 16"):
        const_model.forward_cached([0], c)
    assert c.len() == 16  # untouched on error


def test_error_order(const_model, O):  # :364-377: empty, then length, then token id
    c = const_model.new_cache()
    with pytest.raises(O.OracleError, match="Empty input"):
        const_model.forward_cached([], c)
    with pytest.raises(O.OracleError, match="Total sequence length 17"):
        const_model.forward_cached([99] * 17, c)
    with pytest.raises(O.OracleError, match=r"Token ID 99 out of range \(vocab_size=10\)"):
        const_model.forward_cached([1, 99], c)
    assert c.len() == 0


# ---------------------------------------------------------------------------
# 2. helpers against float64 closed forms / brute force
# ---------------------------------------------------------------------------

def test_layer_norm_closed_form(O):
    rng = np.random.default_rng(0)
    x = rng.normal(size=(5, 96)).astype(np.float32) * 3 + 1
    w = rng.normal(size=96).astype(np.float32)
    b = rng.normal(size=96).astype(np.float32)
    np.testing.assert_allclose(O.layer_norm(x, w, b), ref64.layer_norm(x, w, b, 1e-5), atol=2e-5)
    z = O.layer_norm(x, np.ones(96), np.zeros(96)).astype(np.float64)
    np.testing.assert_allclose(z.mean(-1), 0, atol=1e-6)
    np.testing.assert_allclose(z.var(-1), 1, atol=1e-4)


def test_gelu_closed_form(O):
    x = np.linspace(-8, 8, 4001).astype(np.float32)
    np.testing.assert_allclose(O.gelu_new(x), ref64.gelu_new(x.astype(np.float64)), atol=1e-6)


def test_matmul_sums_each_element_in_k_order(O):
    """orc_matmul's register tiles (4 rows x 32 columns, row groups across
    threads) leave each element's arithmetic as the plain loop's: start from
    0.0f, then one rounded f32 product and one rounded f32 add per k in
    ascending order. numpy's f32 elementwise ops round each op the same way,
    so the results are bit-identical, for every tile remainder and thread
    count."""
    rng = np.random.default_rng(11)
    for m, k, n in [(1, 64, 40), (5, 33, 70), (9, 128, 96), (67, 20, 33)]:
        a = rng.standard_normal((m, k)).astype(np.float32)
        b = rng.standard_normal((k, n)).astype(np.float32)
        ref = np.zeros((m, n), np.float32)
        for kk in range(k):
            ref = ref + a[:, kk:kk + 1] * b[kk:kk + 1, :]
        for th in (1, 3):
            assert np.array_equal(O.matmul(a, b, threads=th), ref), (m, k, n, th)


def test_lm_head_direct_equals_transposed(O):
    """The oracle's direct LM head (each logit summed from its wte row) gives
    bit for bit the logits of the reference's form, a matmul over the
    materialised transpose wte.t().to_owned() (gpt2.rs:395), threaded or not."""
    from rusttorch_amd import synth
    sh = synth.SHAPES["mini"]
    sd = synth.make_weights(sh)
    ids = synth.make_tokens(9, sh.vocab_size, stream=21)
    outs = []
    for direct, th in ((False, 1), (True, 1), (True, 4)):
        om = O.OracleModel.from_shape(sd, sh, threads=th, lm_direct=direct)
        c = om.new_cache()
        outs.append(np.concatenate([om.forward_cached(ids, c), om.forward_cached([3], c)]))
    assert np.array_equal(outs[0], outs[1]) and np.array_equal(outs[0], outs[2])


def test_matmul_exact_integers(O):  # integer-exact case as in autograd/tests.rs:126-153
    a = np.array([[1, 2], [3, 4]], np.float32)
    b = np.array([[5, 6], [7, 8]], np.float32)
    assert O.matmul(a, b).tolist() == [[19, 22], [43, 50]]
    rng = np.random.default_rng(1)
    a = rng.integers(-8, 8, size=(17, 33)).astype(np.float32)
    b = rng.integers(-8, 8, size=(33, 300)).astype(np.float32)
    assert np.array_equal(O.matmul(a, b), a.astype(np.int64) @ b.astype(np.int64))


def test_matmul_float64(O):
    rng = np.random.default_rng(2)
    a = rng.normal(size=(9, 70)).astype(np.float32)
    b = rng.normal(size=(70, 513)).astype(np.float32)
    np.testing.assert_allclose(O.matmul(a, b), a.astype(np.float64) @ b, atol=1e-4)
    np.testing.assert_array_equal(O.matmul(a, b, threads=4), O.matmul(a, b, threads=1))


def test_attention_brute_force(O):
    rng = np.random.default_rng(3)
    T, H, hd = 11, 3, 16
    q, k, v = (rng.normal(size=(T, H * hd)).astype(np.float32) for _ in range(3))
    np.testing.assert_allclose(O.multi_head_attention(q, k, v, H, hd, T), ref64.attention(q, k, v, H), atol=1e-5)


# ---------------------------------------------------------------------------
# 3. whole model: float64 restatement and transformers GPT2LMHeadModel
# ---------------------------------------------------------------------------

def _mini():
    sh = synth.SHAPES["mini"]
    return sh, synth.make_weights(sh)


def test_forward_vs_float64(O):
    sh, sd = _mini()
    m = O.OracleModel.from_shape(sd, sh)
    ids = synth.make_tokens(40, sh.vocab_size)
    ref = ref64.forward(sd, ids, sh.n_layer, sh.n_head)
    got = m.forward(ids)
    assert np.max(np.abs(got - ref)) < 1e-4
    # cached incremental path against the same float64 reference
    c = m.new_cache()
    m.forward_cached(ids[:33], c)
    for t in range(33, 40):
        row = m.forward_cached(ids[t:t + 1], c)[0]
        assert np.max(np.abs(row - ref[t])) < 1e-4


def test_forward_vs_transformers(O):
    torch = pytest.importorskip("torch")
    transformers = pytest.importorskip("transformers")
    sh, sd = _mini()
    cfg = transformers.GPT2Config(vocab_size=sh.vocab_size, n_positions=sh.n_positions, n_embd=sh.n_embd,
                                  n_layer=sh.n_layer, n_head=sh.n_head, layer_norm_epsilon=sh.layer_norm_epsilon,
                                  activation_function="gelu_new", resid_pdrop=0.0, embd_pdrop=0.0, attn_pdrop=0.0)
    cfg._attn_implementation = "eager"
    hf = transformers.GPT2LMHeadModel(cfg).eval()
    state = {"transformer." + k: torch.from_numpy(v.copy()) for k, v in sd.items()}
    state["lm_head.weight"] = state["transformer.wte.weight"]
    missing, unexpected = hf.load_state_dict(state, strict=False)
    assert not unexpected
    assert all(k.endswith("attn.bias") or k.endswith("masked_bias") for k in missing), missing
    ids = synth.make_tokens(48, sh.vocab_size, stream=1)
    with torch.no_grad():
        ref = hf(torch.from_numpy(ids.astype(np.int64))[None]).logits[0].double().numpy()
    m = O.OracleModel.from_shape(sd, sh)
    got = m.forward(ids)
    assert np.max(np.abs(got - ref)) < 2e-4
    # greedy continuation agrees with transformers' greedy decode
    with torch.no_grad():
        hf_ids = hf.generate(torch.from_numpy(ids[:16].astype(np.int64))[None], max_new_tokens=12, do_sample=False,
                             pad_token_id=0)[0].tolist()
    assert m.generate_cached(ids[:16], 12) == hf_ids


# ---------------------------------------------------------------------------
# 4. committed golden fixtures
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["tiny_const", "tiny_rand", "mini"])
def test_golden_fixture(O, name):
    path = os.path.join(GOLDEN, f"{name}.npz")
    g = np.load(path, allow_pickle=False)
    from tests.golden.make_golden import build_case
    sd, sh, prompt = build_case(name)
    assert np.array_equal(prompt, g["prompt"])
    m = O.OracleModel.from_shape(sd, sh)
    c = m.new_cache()
    logits = [m.forward_cached(prompt, c)[-1]]
    toks = list(prompt)
    toks.append(O.argmax(logits[-1]))
    for _ in range(int(g["decode_steps"])):
        logits.append(m.forward_cached([toks[-1]], c)[0])
        toks.append(O.argmax(logits[-1]))
    np.testing.assert_allclose(np.stack(logits), g["logits"], rtol=0, atol=1e-6)
    assert m.generate_cached(prompt, int(g["n_greedy"])) == g["greedy_ids"].tolist()

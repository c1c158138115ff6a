"""Pins of the sampling restatement (oracle/sampling_ref.py), the checker of
the library's device sampler: the reference's own sampling tests
(rusttorch-core/src/nn/gpt2.rs:1320-1416) and closed forms (the SplitMix64
sequence against a direct implementation, the CDF search, top-p ties in index
order, repeated tokens penalised once per occurrence)."""
import numpy as np

from oracle import sampling_ref as S


def arr(*v):
    return np.array(v, dtype=np.float32)


def test_repetition_penalty():  # gpt2.rs:1320-1345
    x = arr(5.0, 3.0, 1.0, 0.5)
    S.apply_repetition_penalty(x, [0, 2], 2.0)
    assert np.allclose(x, [2.5, 3.0, 0.5, 0.5])
    x = arr(-2.0, 3.0)
    S.apply_repetition_penalty(x, [0], 2.0)
    assert np.allclose(x, [-4.0, 3.0])
    x = arr(5.0, 3.0)
    S.apply_repetition_penalty(x, [0], 1.0)
    assert list(x) == [5.0, 3.0]
    x = arr(8.0, -1.0)  # once per occurrence
    S.apply_repetition_penalty(x, [0, 0, 1, 0, 1], 2.0)
    assert list(x) == [1.0, -4.0]


def test_top_k():  # gpt2.rs:1347-1366
    x = arr(1.0, 5.0, 3.0, 2.0, 4.0)
    S.apply_top_k(x, 3)
    assert list(x) == [-np.inf, 5.0, 3.0, -np.inf, 4.0]
    x = arr(1.0, 2.0, 3.0)
    S.apply_top_k(x, 10)
    assert list(x) == [1.0, 2.0, 3.0]
    x = arr(2.0, 7.0, 2.0, 1.0, 2.0)  # ties at the threshold are all kept
    S.apply_top_k(x, 2)
    assert list(x) == [2.0, 7.0, 2.0, -np.inf, 2.0]


def test_top_p():  # gpt2.rs:1368-1397
    x = arr(10.0, 1.0, 1.0, 1.0)
    S.apply_top_p(x, 0.9)
    assert list(x) == [10.0, -np.inf, -np.inf, -np.inf]
    x = arr(5.0, 5.0, -100.0, -100.0)
    S.apply_top_p(x, 0.9)
    assert list(x) == [5.0, 5.0, -np.inf, -np.inf]
    x = arr(1.0, 2.0, 3.0)
    S.apply_top_p(x, 1.0)
    assert list(x) == [1.0, 2.0, 3.0]
    x = arr(0.0, 0.0, 0.0, 0.0)  # equal probabilities: the lowest indices first (stable sort)
    S.apply_top_p(x, 0.5)
    assert list(x) == [0.0, 0.0, -np.inf, -np.inf]


def test_sample_logits():  # gpt2.rs:1399-1426
    assert S.choose(arr(1.0, 5.0, 3.0), [], 0.0, 0, 1.0, 1.0, None)[0] == 1
    assert S.choose(arr(4.5, 5.0, 3.0), [1], 0.0, 0, 1.0, 10.0, None)[0] == 0
    for k in range(1, 20):  # GenerationConfig::creative
        assert S.choose(arr(100.0, -100.0, -100.0, -100.0), [], 0.9, 50, 0.95, 1.2, S.splitmix_uniform(3, k))[0] == 0


def test_splitmix_and_cdf():
    # SplitMix64 (Steele, Lea, Flood 2014) run as a state machine from the seed
    s, outs = 1234, []
    for _ in range(5):
        s = (s + 0x9E3779B97F4A7C15) & (2 ** 64 - 1)
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2 ** 64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2 ** 64 - 1)
        outs.append(np.float32((z ^ (z >> 31)) >> 40) / np.float32(2 ** 24))
    assert [S.splitmix_uniform(1234, k) for k in range(1, 6)] == outs
    assert all(0.0 <= u < 1.0 for u in outs)
    # the first index whose running sum exceeds r
    x = np.log(arr(0.1, 0.2, 0.3, 0.4))
    for r, want in ((0.05, 0), (0.1, 1), (0.29, 1), (0.31, 2), (0.61, 3), (0.99, 3)):
        assert S.sample_from_logits(x, np.float32(r))[0] == want


def test_splitmix_published_vector():
    # the published outputs of splitmix64.c (Vigna) for seed 1234567; the
    # uniform is their top 24 bits
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423, 4593380528125082431,
            16408922859458223821]
    for k, z in enumerate(want, start=1):
        assert S.splitmix_uniform(1234567, k) == np.float32(z >> 40) / np.float32(2 ** 24)


def test_filters_against_brute_force():
    """top-k by counting larger entries, top-p by walking (probability desc,
    index asc) pairs with a float32 running sum, the draw by np.searchsorted on
    the float32 CDF: other formulations of the same rules, on random logits
    with planted ties."""
    rng = np.random.default_rng(5)
    for trial in range(200):
        n = int(rng.integers(1, 40))
        x = rng.normal(0, 2, n).astype(np.float32)
        if n > 3:
            x[rng.integers(0, n, 3)] = x[0]  # ties
        k = int(rng.integers(1, n + 1))
        got = x.copy()
        S.apply_top_k(got, k)
        for i in range(n):
            larger = int(np.sum(x > x[i]))
            assert (got[i] == x[i]) == (larger < k) and (got[i] == -np.inf) == (larger >= k)
        p = float(rng.uniform(0.05, 0.99))
        got = x.copy()
        S.apply_top_p(got, p)
        probs = S._softmax(x)
        kept, cum = set(), np.float32(0)
        for _, i in sorted((-float(probs[i]), i) for i in range(n)):
            kept.add(i)
            cum = np.float32(cum + probs[i])
            if cum >= np.float32(p):
                break
        assert {i for i in range(n) if got[i] != -np.inf} == kept
        got = x.copy()  # the float64 cut, by the same walk in float64
        S.apply_top_p(got, p, exact=True)
        e64 = np.exp(x.astype(np.float64) - float(np.max(x)))
        p64 = e64 / e64.sum()
        kept, cum = set(), 0.0
        for _, i in sorted((-float(p64[i]), i) for i in range(n)):
            kept.add(i)
            cum += float(p64[i])
            if cum >= p:
                break
        assert {i for i in range(n) if got[i] != -np.inf} == kept
        r = np.float32(rng.uniform(0, 1))
        cdf = np.cumsum(S._softmax(x), dtype=np.float32)
        want = min(int(np.searchsorted(cdf, r, side="right")), n - 1)
        assert S.sample_from_logits(x, r)[0] == want

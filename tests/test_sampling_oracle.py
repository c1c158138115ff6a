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

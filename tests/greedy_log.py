"""Greedy-id checks that log the oracle's top-1 minus top-2 logit gap.

Greedy ids are compared exactly. Every comparison records the smallest gap
between the oracle's best and second-best logit over its steps, and a
mismatch reports the gap at the step where the ids first differ: a gap inside
the logits tolerance (|d| <= 1e-3 + 1e-4 |ref|, twice over for two sides) is
a near tie, which either side may break its own way; a larger gap means a
wrong logit. conftest prints the collected records after the run.
"""
import numpy as np

ATOL, RTOL = 1e-3, 1e-4

# (what, greedy steps checked, smallest gap, step of the smallest gap, near ties)
RECORDS = []


def tie_tolerance(top1: float) -> float:
    """A gap at or below this is a near tie under the logits bar (both the GPU's
    and the oracle's logit may move by the tolerance)."""
    return 2 * (ATOL + RTOL * abs(float(top1)))


def record(what, gaps, near_ties=0):
    gaps = np.asarray(gaps, np.float64)
    if gaps.size == 0:
        return
    s = int(np.nanargmin(gaps))
    RECORDS.append((what, int(gaps.size), float(gaps[s]), s, int(near_ties)))


def top2_gap(row):
    """(top-1 minus top-2 value, index of the top-1) of a logits row."""
    row = np.asarray(row, np.float64)
    i = int(np.argmax(row))
    rest = np.delete(row, i)
    return float(row[i] - np.max(rest)), i


def assert_ids_equal(got, want, gaps, n_prompt, what):
    """Exact greedy-id equality against the oracle's generate_cached(..., gaps=True)
    result; the failure message names the first differing step and its gap."""
    got, want = list(map(int, got)), list(map(int, want))
    record(what, gaps)
    if got == want:
        return
    assert len(got) == len(want), f"{what}: {len(got)} ids against the oracle's {len(want)}"
    first = next(i for i in range(len(want)) if got[i] != want[i])
    s = first - n_prompt
    gap = float(gaps[s]) if 0 <= s < len(gaps) else float("nan")
    kind = "inside" if gap <= 2 * ATOL else "outside"
    raise AssertionError(f"{what}: ids differ first at greedy step {s} (GPU {got[first]}, oracle {want[first]}); "
                         f"oracle top1-top2 gap there {gap:.3e} ({kind} twice the absolute logits tolerance); "
                         f"min gap over the run {float(np.nanmin(gaps)):.3e}")


def check_greedy_along(om, prompt, gpu_ids, what):
    """Feeds the oracle the GPU's own token sequence (teacher forcing) and
    checks every greedy choice: it must be the oracle's argmax, or, when the
    oracle's top-2 gap is within the near-tie tolerance, a token whose oracle
    logit lies within that tolerance of the maximum. Returns (smallest gap,
    number of near ties)."""
    n = len(prompt)
    c = om.new_cache()
    row = om.forward_cached(prompt, c)[-1]
    gaps, ties = [], 0
    for s in range(len(gpu_ids) - n):
        tok = int(gpu_ids[n + s])
        gap, best = top2_gap(row)
        gaps.append(gap)
        tol = tie_tolerance(row[best])
        if tok != best:
            assert gap <= tol and float(row[best]) - float(row[tok]) <= tol, (
                f"{what}: step {s} GPU token {tok} vs oracle {best}, gap {gap:.3e}")
            ties += 1
        if n + s + 1 < len(gpu_ids):
            row = om.forward_cached([tok], c)[0]
    record(what, gaps, ties)
    min_gap = float(np.min(gaps)) if gaps else float("inf")
    print(f"[gpu] {what}: {len(gaps)} greedy steps checked, min top-2 gap {min_gap:.3e}, near ties {ties}",
          flush=True)
    return min_gap, ties

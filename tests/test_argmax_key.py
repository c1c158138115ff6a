"""The packed argmax key (rusttorch_amd/csrc/argmax_key.h), shared by every
kernel that picks a greedy token, against argmax_f32 (gpt2.rs:858-868: strict
'>' scan from -inf, first index of the maximum wins, NaN never wins, an
all-NaN / all -inf row gives 0). The header is compiled for the host with
g++ and reduced in several orders; the reference rule is the oracle's
orc_argmax, itself pinned by the reference's argmax tests."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = r'''
#include <stddef.h>
#include <stdint.h>
#include "argmax_key.h"
// max over the keys of x[perm[0..n)], i.e. the reduction in that order
extern "C" uint32_t key_argmax(const float* x, const uint32_t* perm, size_t n) {
  uint64_t best = 0;
  for (size_t i = 0; i < n; ++i) {
    const uint64_t k = rtg::argmax_key(x[perm[i]], perm[i]);
    best = k > best ? k : best;
  }
  return rtg::argmax_key_index(best);
}
extern "C" uint64_t key_of(float v, uint32_t idx) { return rtg::argmax_key(v, idx); }
'''


@pytest.fixture(scope="module")
def keylib(tmp_path_factory):
    d = tmp_path_factory.mktemp("argmax_key")
    src = d / "k.cpp"
    src.write_text(SRC)
    so = d / "libk.so"
    subprocess.run(["g++", "-O2", "-std=c++20", "-shared", "-fPIC", "-DRTG_HD=inline",
                    "-I", os.path.join(ROOT, "rusttorch_amd", "csrc"), "-o", str(so), str(src)], check=True)
    lib = C.CDLL(str(so))
    lib.key_argmax.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    lib.key_argmax.restype = C.c_uint32
    lib.key_of.argtypes = [C.c_float, C.c_uint32]
    lib.key_of.restype = C.c_uint64
    return lib


def key_argmax(lib, x, perm):
    x = np.ascontiguousarray(x, np.float32)
    perm = np.ascontiguousarray(perm, np.uint32)
    return int(lib.key_argmax(x.ctypes.data, perm.ctypes.data, len(x)))


SPECIAL = np.array([0.0, -0.0, np.nan, np.inf, -np.inf, 1.0, -1.0, 1e-45, -1e-45, 3.4e38, -3.4e38],
                   dtype=np.float32)


def test_key_order_of_special_values(keylib):
    k = lambda v, i=0: int(keylib.key_of(float(v), i))  # noqa: E731
    assert k(np.nan) == 0 and k(-np.inf) == 0  # never win
    assert k(-0.0, 5) == k(0.0, 5)  # -0.0 and +0.0 compare equal
    assert k(0.0, 3) > k(0.0, 4)  # equal values: the earlier index wins
    assert k(np.inf) > k(3.4e38) > k(1.0) > k(1e-45) > k(0.0) > k(-1e-45) > k(-1.0) > k(-3.4e38) > 0


def test_pm_zero_first_index_wins(keylib, oracle_lib):
    for x in ([-0.0, 0.0], [0.0, -0.0], [-1.0, -0.0, 0.0, -0.0], [np.nan, -0.0, 0.0], [-np.inf, 0.0, -0.0]):
        x = np.array(x, np.float32)
        want = oracle_lib.argmax(x)
        for perm in (np.arange(len(x)), np.arange(len(x))[::-1]):
            assert key_argmax(keylib, x, perm) == want, (x, perm)


def test_against_argmax_f32_random_rows(keylib, oracle_lib):
    """Rows drawn from the special values plus a few random ones (many
    ties, zeros of both signs, NaN, infinities), each reduced in order, in
    reverse and in a random order: always argmax_f32's index."""
    rng = np.random.default_rng(3)
    for trial in range(3000):
        n = int(rng.integers(1, 40))
        pool = np.concatenate([SPECIAL, rng.standard_normal(3).astype(np.float32)])
        x = rng.choice(pool, size=n).astype(np.float32)
        want = oracle_lib.argmax(x)
        for perm in (np.arange(n), np.arange(n)[::-1], rng.permutation(n)):
            assert key_argmax(keylib, x, perm) == want, (trial, x.tolist(), perm.tolist())


def test_all_nan_or_neg_inf_gives_zero(keylib, oracle_lib):
    for x in ([np.nan] * 5, [-np.inf] * 3, [np.nan, -np.inf, np.nan]):
        x = np.array(x, np.float32)
        assert key_argmax(keylib, x, np.arange(len(x))[::-1]) == 0 == oracle_lib.argmax(x)

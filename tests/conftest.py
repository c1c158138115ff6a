import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: long-running parity case")


def gpu_available() -> bool:
    try:
        import ctypes
        hip = ctypes.CDLL("libamdhip64.so")
        n = ctypes.c_int(0)
        return hip.hipGetDeviceCount(ctypes.byref(n)) == 0 and n.value > 0
    except OSError:
        return False


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import oracle
    oracle.build()
    return oracle


def pytest_terminal_summary(terminalreporter):
    """The greedy near-tie log: per id comparison against the oracle, the
    smallest top-1 minus top-2 logit gap of the oracle's rows."""
    from tests.greedy_log import RECORDS
    if not RECORDS:
        return
    tr = terminalreporter
    tr.section("greedy near-tie log (oracle top1 - top2 logit gap)")
    for what, steps, gap, at, ties in RECORDS:
        tr.write_line(f"{what}: {steps} greedy steps, min gap {gap:.3e} at step {at}, near ties {ties}")

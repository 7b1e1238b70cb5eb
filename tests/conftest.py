import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# Under pytest-xdist every worker loads the OpenMP oracle: one thread each,
# or the workers' spinning thread teams oversubscribe the cores and the
# oracle's many short parallel regions slow down a hundredfold.
if os.environ.get("PYTEST_XDIST_WORKER"):
    os.environ.setdefault("OMP_NUM_THREADS", "1")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C-ABI)")


def close(got, want, rel, abs_floor):
    """kerneltest.Close (kernels/kerneltest/compare.go:29-37), vectorized:
    |got-want| <= abs + rel*max(|want|, 1)."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = np.maximum(np.abs(want), 1.0)
    return np.abs(got - want) <= abs_floor + rel * scale


def assert_close(got, want, rel, abs_floor, what=""):
    ok = close(got, want, rel, abs_floor)
    if not np.all(ok):
        idx = np.argwhere(~ok)[0]
        g = np.asarray(got).reshape(np.shape(ok))[tuple(idx)]
        w = np.asarray(want).reshape(np.shape(ok))[tuple(idx)]
        raise AssertionError(f"{what} mismatch at {tuple(idx)}: got {g!r} want {w!r} "
                             f"({(~ok).sum()} of {ok.size} outside tolerance)")


def rel_err(got, want):
    """Normwise relative error ||got-want|| / ||want||."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    d = np.linalg.norm(got - want)
    n = np.linalg.norm(want)
    return d / n if n > 0 else d


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    return oracle

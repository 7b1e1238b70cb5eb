"""CPU checks of the drop-in boundary: libgnhip.so loads without a GPU,
exports every entry point include/gonano_hip.h declares, and reports a clean
error (not a crash) when no device is present."""
import ctypes as C
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    text = open(os.path.join(ROOT, "include", "gonano_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gn_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from gonano_amd import _lib
    L = _lib.lib()
    names = header_functions()
    assert len(names) >= 33 + 10
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes signature table covers the whole header
    assert sorted(_lib.exported_symbols()) == names


def test_backend_covers_the_33_interface_methods():
    from gonano_amd.backend import HipBackend
    methods = """Add Subtract Multiply Divide Scale AddScaled Negate Abs Square ReluSquared SwiGLU
    SwiGLUBackward Exp Sigmoid Tanh Rsqrt Sum Max ArgMax MatMul MatMulTransposed DotProduct
    IndexerScores IndexerBlockMax TopKIndices MoEGateTopK GroupedMatMulTransposed SoftmaxLastDim
    RMSNormLastDim AttentionForward AttentionBackward AttentionForwardSplit AttentionCombine""".split()
    assert len(methods) == 33
    for m in methods:
        assert callable(getattr(HipBackend, m)), m


def test_no_device_fails_cleanly():
    from gonano_amd import _lib
    L = _lib.lib()
    if L.gn_device_count() > 0:
        pytest.skip("a GPU is visible")
    out = C.c_float()
    st = L.gn_sum(np.ones(4, np.float32), 4, C.byref(out))
    assert st != 0
    assert L.gn_last_error()
    from gonano_amd.config import dense_d2
    from gonano_amd.session import Session
    with pytest.raises(_lib.HipError):
        Session(dense_d2())


def test_oracle_library_builds_and_loads(orc):
    assert orc.lib().orc_num_threads() >= 1

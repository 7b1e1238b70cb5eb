"""Consistency of the committed flash long-prompt fixture
(tests/golden/flash_long.npz, read by tests/test_gpu_flash_long.py) with the
case it was written from (tests/golden/flash_long_case.py), on the CPU:
shapes, the sampled gradient entries' indices, every sampled token inside
the top 50 logits the oracle recorded for its step (the sampler's top-k),
rows ending only at the terminal token, and the float32 and float64 oracle
builds agreeing to float32 accuracy."""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import flash_long_case as case  # noqa: E402


def _gold():
    return np.load(os.path.join(HERE, "golden", "flash_long.npz"))


def test_fixture_shapes_and_indices():
    g = _gold()
    cfg = case.config()
    V = cfg.vocab_size
    assert g["fwd_last"].shape == (V,)
    assert g["rows"].shape == (case.S, case.N)
    assert g["step_top"].shape == (case.N, case.S, case.TOPN)
    assert g["nll32"].shape == (1, case.T_PG - case.P)
    idx = case.sample_indices(cfg)
    assert np.array_equal(g["g_idx"], np.concatenate(idx))
    assert g["g_val32"].size == g["g_idx"].size == g["g_val64"].size
    assert g["g_norm32"].size == len(cfg.param_table())


def test_fixture_tokens_within_top50():
    g = _gold()
    rows, top = g["rows"], g["step_top"]
    for i in range(case.S):
        n = int((rows[i] >= 0).sum())
        assert n >= 1 and np.all(rows[i, n:] == -1)
        for t in range(n):
            assert rows[i, t] in top[t, i, :50], (i, t)


def test_fixture_f32_matches_f64():
    g = _gold()
    l32, l64 = float(g["loss32"]), float(g["loss64"])
    assert abs(l32 - l64) <= 1e-4 * abs(l64)
    n32, n64 = g["nll32"], g["nll64"]
    assert np.linalg.norm(n32 - n64) <= 1e-4 * np.linalg.norm(n64)
    # A 1 x 1 tensor (the indexer's head scale) sums some 10^7 float32
    # terms of both signs in one accumulator: its float32 gradient is good
    # to about 1e-2; the other tensors' norms to 1e-3.
    a, b = g["g_norm32"], g["g_norm64"]
    size = np.array([r * c for _, r, c, _ in case.config().param_table()])
    tol = np.where(size == 1, 1e-2, 1e-3)
    live = b > 1e-20
    assert np.all(np.abs(a[live] - b[live]) <= tol[live] * b[live])
    assert np.all(np.isfinite(g["fwd_last"])) and np.abs(g["fwd_last"]).max() > 0

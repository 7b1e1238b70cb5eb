"""Parity at the flash workload's prompt length (8192-token prompts,
SequenceLen 16384) on a 3-layer flash model (one Full, one Reindex, one
Reuse layer; V 4096).  The oracle needs minutes for these lengths, so its
results come from tests/golden/flash_long.npz
(written by tests/golden/make_flash_long.py from the same case,
tests/golden/flash_long_case.py):

* Transformer.Forward over the 8192-token prompt: the last position's
  logits (compressed training attention, the lightning indexer's selection
  over 2048 compressed blocks in pools of 8, the 512-key window);
* one rollout group (16 samples, 4 new tokens): the CED prefill over the
  prompt, decode over the selection and the window; every sampled token
  equals the oracle's;
* PolicyGradientStep over one 8703-token sequence (the prompt and 511
  generated tokens, targets only after the prompt): loss, NLL of the 511
  target rows, and every parameter tensor's gradient through its norm and
  256 entries drawn at random (normwise on the drawn entries, at 1e-4 or
  twice the oracle's own float32 error there, as the other width tests)."""
import os
import sys

import numpy as np
import pytest

from conftest import rel_err

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import flash_long_case as case  # noqa: E402
from test_gpu_shapes import _bar, report  # noqa: E402


@pytest.fixture(scope="module")
def gold():
    return np.load(os.path.join(HERE, "golden", "flash_long.npz"))


@pytest.fixture(scope="module")
def model():
    cfg = case.config()
    assert (cfg.n_layer, cfg.sequence_len, cfg.compression_ratio, cfg.swa_window) == (3, 16384, 4, 512)
    assert cfg.ced and cfg.reuse_pattern == "FRU" and cfg.sparse_topk == 16
    return cfg, case.weights(cfg), case.inputs(cfg)


def test_flash_long_forward_last_logits(gold, model):
    from gonano_amd.session import Session
    cfg, w, (prompt, _, _) = model
    with Session(cfg) as s:
        s.set_params(w)
        got = s.forward(prompt[None, :])[0, -1]
    e = rel_err(got, gold["fwd_last"])
    report(f"flash 8192-token forward, last logits: gpu-f32 {e:.2e} (bar 1e-4)")
    assert e < 1e-4


def test_flash_long_rollout(gold, model):
    from gonano_amd.session import Session
    cfg, w, (prompt, _, _) = model
    with Session(cfg) as s:
        s.set_params(w)
        rows = s.generate_batch(prompt[None, :], case.S, case.N, 1.0, 50,
                                np.array([case.SEED_GROUP], np.uint64))
    want = gold["rows"]
    assert len(rows) == case.S
    checked = 0
    for i, r in enumerate(rows):
        assert np.array_equal(r[:case.P], prompt)
        comp = np.asarray(r[case.P:])
        n = int((want[i] >= 0).sum())
        assert comp.size == n, (i, comp, want[i])
        for t in range(n):
            assert comp[t] == want[i, t], (i, t, comp, want[i], gold["step_top"][t, i, :4],
                                            gold["step_val"][t, i, :4])
            checked += 1
    report(f"flash 8192-token rollout: {checked} sampled tokens equal the oracle's")
    assert checked >= case.S


def test_flash_long_pg_step(gold, model):
    from gonano_amd.session import Session
    cfg, w, (_, pg_in, pg_tg) = model
    with Session(cfg) as s:
        s.set_params(w)
        s.zero_grad()
        loss, nll = s.policy_gradient_step(pg_in, pg_tg, np.array([case.ADV], np.float32),
                                           float(case.T_PG + 1))
        g = s.grads()
    l32, l64 = float(gold["loss32"]), float(gold["loss64"])
    lbar = max(1e-4 * max(abs(l32), 1e-3), 2 * abs(l32 - l64))
    report(f"flash 8703-token PG step: loss gpu {loss:.9g} f32 {l32:.9g} f64 {l64:.9g} "
           f"bar {lbar:.1e}")
    assert abs(loss - l32) <= lbar
    nll = np.asarray(nll, np.float64).reshape(1, case.T_PG)
    assert np.all(nll[:, :case.P] == 0)
    e_n, e32_n = rel_err(nll[:, case.P:], gold["nll32"]), rel_err(gold["nll32"], gold["nll64"])
    report(f"  nll: gpu-f32 {e_n:.2e} f32-f64 {e32_n:.2e} bar {_bar(e32_n, 1e-4):.1e}")
    assert e_n < _bar(e32_n, 1e-4)
    idx = case.sample_indices(cfg)
    v32, v64 = gold["g_val32"], gold["g_val64"]
    n32, n64 = gold["g_norm32"], gold["g_norm64"]
    bad, at = [], 0
    for k, ((name, r, c, off), ix) in enumerate(zip(cfg.param_table(), idx)):
        t = np.asarray(g[off:off + r * c], np.float64)
        a, b = v32[at:at + ix.size], v64[at:at + ix.size]
        at += ix.size
        got = t[ix]
        e, e32 = rel_err(got, a), rel_err(a, b)
        en, en32 = abs(np.linalg.norm(t) - n32[k]) / max(n32[k], 1e-30), \
            abs(n32[k] - n64[k]) / max(n64[k], 1e-30)
        tol = 1e-4 if r * c >= 64 else 5e-4
        bar, nbar = _bar(e32, tol), _bar(en32, tol)
        floor = 1e-5 * float(np.abs(a).max() if a.size else 0) + 1e-30
        report(f"  {name:45s} sample gpu-f32 {e:.2e} f32-f64 {e32:.2e} bar {bar:.1e} | "
               f"norm {en:.2e} bar {nbar:.1e}")
        if n32[k] < 1e-20 and np.linalg.norm(t) < 1e-20:
            continue
        if (e >= bar and np.abs(got - a).max() > floor) or en >= nbar:
            bad.append((name, e, e32, en))
    assert not bad, bad

"""On-policy distillation on the GPU (gn_distill_step, trainer/distill.go)
against the oracle's DistillStep on the same inputs: a dense student
distilled from a wider dense teacher and from an MLA + MoE teacher
(trainer/distill_test.go:122-160), with a mask and a temperature; the loss
and every parameter gradient within the 1e-4 normwise bar, a student
distilled from itself getting a zero gradient, an all-zero mask a zero loss
and gradient."""
import numpy as np
import pytest

from conftest import rel_err
from gonano_amd import config as G
from test_gpu_session import _compare_grads, small_cfg

pytestmark = pytest.mark.gpu


def _teacher_cfg(kind):
    if kind == "dense":
        return G.Config(sequence_len=512, vocab_size=4096, n_layer=2, n_head=4, n_kv_head=2,
                        n_embd=512, window_pattern="SL", rotary_dims=64)
    from test_gpu_latent import latent_small_cfg
    return latent_small_cfg()


@pytest.mark.parametrize("kind", ["dense", "latent"])
def test_distill_step_matches_oracle(orc, kind):
    from gonano_amd.session import Session
    cfg, tcfg = small_cfg(), _teacher_cfg(kind)
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    wt = G.init_weights(tcfg, seed=4, perturb=0.05)
    rng = np.random.default_rng(6)
    B, T = 2, 160
    x = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    mask = (rng.random((B, T)) < 0.8).astype(np.int32)
    with Session(cfg) as s, Session(tcfg) as t:
        s.set_params(w)
        t.set_params(wt)
        s.zero_grad()
        loss = s.distill_step(t, x, mask, temperature=1.5, grad_accum_steps=2)
        grads = s.grads()
    student = orc.OracleModel(orc.ModelShape.from_config(cfg), w)
    teacher = orc.OracleModel(orc.ModelShape.from_config(tcfg), wt)
    wl, wg = student.distill_step(teacher.forward(x).astype(np.float32), x, mask, 1.5, 2)
    assert abs(loss - wl) <= 1e-4 * abs(wl), (loss, wl)
    _compare_grads(cfg, grads, wg)


def test_distill_self_and_masked():
    from gonano_amd.session import Session
    cfg = small_cfg()
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    x = np.random.default_rng(7).integers(0, cfg.vocab_size, (2, 96)).astype(np.int32)
    with Session(cfg) as s, Session(cfg) as twin:
        s.set_params(w)
        twin.set_params(w)
        s.zero_grad()
        s.distill_step(twin, x)  # distill_test.go:65-81
        g = s.grads()
        assert np.abs(g).max() < 1e-4
        s.zero_grad()  # distill_test.go:83-101
        assert s.distill_step(twin, x, np.zeros_like(x), 2.0) == 0.0
        assert not s.grads().any()

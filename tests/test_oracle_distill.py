"""Pins the oracle's trainer.DistillStep restatement (oracle/model.c,
orc_distill_step) to the reference's own tests (tensors/loss_test.go:66-140,
trainer/distill_test.go:65-101) and to finite differences: a one-hot
teacher reduces the loss and its gradient to the cross-entropy's; a
student distilled from its own logits gets a zero gradient; an all-zero
mask gives a zero loss and gradient; the gradient equals central finite
differences of the loss (float64 build) with a mask and a temperature."""
import numpy as np
import pytest

from gonano_amd import config as G


def _cfg():
    return G.Config(sequence_len=256, vocab_size=512, n_layer=2, n_head=2, n_kv_head=1, n_embd=128,
                    window_pattern="SL", rotary_dims=64)


def _models(orc, dtype=np.float32):
    cfg = _cfg()
    tcfg = G.Config(sequence_len=256, vocab_size=512, n_layer=2, n_head=2, n_kv_head=2, n_embd=256,
                    window_pattern="L", rotary_dims=64)
    w = G.init_weights(cfg, seed=1, perturb=0.05)
    wt = G.init_weights(tcfg, seed=2, perturb=0.1)
    s = orc.OracleModel(orc.ModelShape.from_config(cfg), w, dtype)
    t = orc.OracleModel(orc.ModelShape.from_config(tcfg), wt)
    return cfg, w, s, t


def _batch(seed=0):
    rng = np.random.default_rng(seed)
    x = rng.integers(0, 512, (2, 24)).astype(np.int32)
    mask = (rng.random((2, 24)) < 0.7).astype(np.int32)
    return x, mask


def test_one_hot_teacher_is_cross_entropy(orc):  # loss_test.go:66-91
    cfg, w, s, _ = _models(orc)
    x, _ = _batch(1)
    targets = np.random.default_rng(5).integers(0, 512, x.shape).astype(np.int32)
    targets[:, :3] = -1
    teacher = np.zeros(x.shape + (512,), np.float32)
    np.put_along_axis(teacher, np.maximum(targets, 0)[..., None], 100.0, axis=-1)
    loss, g = s.distill_step(teacher, x, (targets != -1).astype(np.int32), 1.0, 1)
    grads = np.zeros_like(g)
    ce = s._fn("orc_ce_loss")(s._m, x, targets, 2, 24, grads.ctypes.data)  # the mean
    assert abs(loss - ce) < 1e-3
    assert np.linalg.norm(g - grads) <= 1e-3 * np.linalg.norm(grads)


def test_self_distillation_zero_gradient(orc):  # distill_test.go:65-81, loss_test.go:117-125
    cfg, w, s, _ = _models(orc)
    x, mask = _batch(2)
    own = s.forward(x).astype(np.float32)
    loss, g = s.distill_step(own, x, mask, 1.0, 1)
    assert np.abs(g).max() < 1e-6
    # the loss is the entropy of the student's distribution (cross-entropy
    # of a distribution with itself)
    z = own.astype(np.float64)
    p = np.exp(z - z.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    ent = -(p * np.log(p)).sum(-1)
    assert abs(loss - ent[mask != 0].mean()) < 1e-4 * ent.mean()


def test_all_masked(orc):  # distill_test.go:83-101
    cfg, w, s, t = _models(orc)
    x, _ = _batch(3)
    loss, g = s.distill_step(t.forward(x).astype(np.float32), x, np.zeros_like(x), 2.0, 1)
    assert loss == 0 and not g.any()


@pytest.mark.parametrize("temperature", [1.0, 1.7])
def test_gradient_matches_finite_differences(orc, temperature):  # loss_test.go:93-115
    cfg, w, s, t = _models(orc, np.float64)
    x, mask = _batch(4)
    tl = t.forward(x).astype(np.float32)
    _, g = s.distill_step(tl, x, mask, temperature, 2)
    rng = np.random.default_rng(9)
    for _ in range(2):
        d = rng.standard_normal(w.size)
        d /= np.linalg.norm(d)
        eps = 1e-4

        def L(v):
            m = orc.OracleModel(orc.ModelShape.from_config(cfg), v, np.float64)
            return m.distill_step(tl, x, mask, temperature, 2)[0]
        fd = (L(w.astype(np.float64) + eps * d) - L(w.astype(np.float64) - eps * d)) / (2 * eps)
        # the loss is the mean over valid positions; with 2 accumulation
        # steps the gradient carries another 1/2
        assert abs(float(g @ d) - fd / 2) <= 1e-6 + 1e-5 * abs(fd), (float(g @ d), fd)

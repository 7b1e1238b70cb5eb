"""Pins the oracle's MuonAdamW restatement (oracle/optimizer.c) to the
reference's own known answers (optimizer/optim_test.go,
optimizer/sinkhorn_test.go) and to what the mathematics fixes: AdamW's
closed form under a constant gradient, the Polar Express polynomial acting
on singular values (U p(S) V^T), Muon's norm invariants (Muon+ and the
variance reduction leave ||update||_F = sqrt(min(rows, cols))), Sinkhorn's
unit rows, and the SetupOptimizer table (model/optimizer.go) covering every
parameter exactly once."""
import math

import numpy as np
import pytest

from gonano_amd import config as G
from gonano_amd import optimizer as OPT

f32 = np.float32


def table(*entries):
    return np.array(list(entries), OPT.OPT_PARAM_DTYPE)


def adamw(off, n, **h):
    return OPT._entry(off, 1, n, OPT.KIND_ADAMW, **h)


def muon(off, r, c, **h):
    base = dict(lr=0.01, momentum=0.95, ns_steps=5, muon_beta2=0.9)
    base.update(h)
    return OPT._entry(off, r, c, OPT.KIND_MUON, **base)


def sinkhorn(off, r, c, **h):
    return OPT._entry(off, r, c, OPT.KIND_SINKHORN, **h)


def test_adamw_exact_value(orc):  # optim_test.go:10-27
    o = orc.OracleOptimizer(table(adamw(0, 1, lr=0.01, beta1=0.9, beta2=0.999, eps=1e-8)))
    p = np.array([1], f32)
    o.step(p, np.array([1], f32))
    assert abs(p[0] - 0.99) <= 1e-5


def test_adamw_reduces_quadratic_loss(orc):  # optim_test.go:29-50
    p = np.ones(100, f32)
    o = orc.OracleOptimizer(table(adamw(0, 100, lr=0.05, beta1=0.9, beta2=0.999, eps=1e-8)))
    before = float((p.astype(np.float64) ** 2).sum())
    for _ in range(10):
        o.step(p, 2 * p)
    assert float((p.astype(np.float64) ** 2).sum()) < before


def test_adamw_constant_gradient_closed_form(orc):
    """With a constant gradient g the bias-corrected moments are g and g^2
    at every step, so each step is p <- p*(1 - lr*wd) - lr*g/(|g| + eps)."""
    rng = np.random.default_rng(3)
    g = rng.standard_normal(64).astype(f32)
    p = rng.standard_normal(64).astype(f32)
    lr, wd, eps = 0.003, 0.01, 1e-8
    o = orc.OracleOptimizer(table(adamw(0, 64, lr=lr, beta1=0.8, beta2=0.95, eps=eps,
                                        weight_decay=wd)))
    want = p.astype(np.float64)
    for _ in range(7):
        o.step(p, g)
        want = want * (1 - lr * wd) - lr * g / (np.abs(g.astype(np.float64)) + eps)
    np.testing.assert_allclose(p, want, rtol=2e-6, atol=2e-7)
    # moments: m_t = g (1 - b1^t), v_t = g^2 (1 - b2^t)
    np.testing.assert_allclose(o.state[:64], g * (1 - 0.8 ** 7), rtol=1e-5)
    np.testing.assert_allclose(o.state[64:], g.astype(np.float64) ** 2 * (1 - 0.95 ** 7), rtol=1e-5)


PE = [(8.156554524902461, -22.48329292557795, 15.878769915207462),
      (4.042929935166739, -2.808917465908714, 0.5000178451051316),
      (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
      (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
      (2.3465413258596377, -1.7097828382687081, 0.42323551169305323)]


@pytest.mark.parametrize("rows,cols", [(48, 20), (20, 48), (32, 32)])
def test_polar_express_acts_on_singular_values(orc, rows, cols):
    """X = U S V^T: every quintic step maps X to U p(S) V^T with p(s) =
    a s + b s^3 + c s^5, after the input scaling 1/(1.01 ||X||_F + 1e-6)
    (optimizer/muon.go:50-74).  A transposed product or a misordered
    coefficient changes the result far beyond float32 rounding."""
    rng = np.random.default_rng(rows * 100 + cols)
    k = min(rows, cols)
    U, _ = np.linalg.qr(rng.standard_normal((rows, k)))
    V, _ = np.linalg.qr(rng.standard_normal((cols, k)))
    s = np.linspace(0.2, 3.0, k)
    X = (U * s) @ V.T
    got = orc.polar_express(X.astype(f32), 5)
    x32 = X.astype(f32)
    sc = 1.0 / (float(np.sqrt((x32.astype(np.float64) ** 2).sum())) * 1.01 + 1e-6)
    t = s * sc
    for a, b, c in PE:
        t = a * t + b * t ** 3 + c * t ** 5
    want = (U * t) @ V.T
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert err < 2e-4, err
    # the singular values land near 1 (what the coefficients are tuned for)
    sv = np.linalg.svd(got.astype(np.float64), compute_uv=False)
    assert sv.min() > 0.6 and sv.max() < 1.3, sv


@pytest.mark.parametrize("rows,cols", [(6, 3), (3, 6)])  # optim_test.go:66-119
def test_muon_step_finite_updates_state(orc, rows, cols):
    rng = np.random.default_rng(1)
    p = (0.1 * rng.standard_normal(rows * cols)).astype(f32)
    g = (0.1 * rng.standard_normal(rows * cols)).astype(f32)
    before = p.copy()
    o = orc.OracleOptimizer(table(muon(0, rows, cols)))
    o.step(p, g)
    assert np.isfinite(p).all() and (p != before).all()
    second = o.state[rows * cols:]
    assert second.size == max(rows, cols) and (second > 0).all()


@pytest.mark.parametrize("rows,cols", [(40, 24), (24, 40)])
def test_muon_update_norm_and_state_closed_forms(orc, rows, cols):
    """Without weight decay the parameter moves by lr * U with ||U||_F =
    sqrt(min(rows, cols)): Muon+ sets that norm and the variance reduction's
    ratio restores it.  From a zero state the momentum is (1-mu) g and the
    second moment (1 - beta2) times the per-row (or per-column) mean
    square of the renormalized update."""
    rng = np.random.default_rng(7)
    n = rows * cols
    p = rng.standard_normal(n).astype(f32)
    g = rng.standard_normal(n).astype(f32)
    lr = 0.02
    o = orc.OracleOptimizer(table(muon(0, rows, cols, lr=lr, weight_decay=0.0)))
    p0 = p.copy()
    o.step(p, g)
    d = (p0.astype(np.float64) - p) / lr
    assert abs(np.linalg.norm(d) - math.sqrt(min(rows, cols))) < 1e-3 * math.sqrt(min(rows, cols))
    np.testing.assert_allclose(o.state[:n], (1 - f32(0.95)) * g, rtol=1e-6)
    second = o.state[n:]
    assert second.size == max(rows, cols) and (second > 0).all()
    # the means sum to ||U||^2 / min(rows, cols) = 1 after Muon+
    assert abs(second.sum() / (1 - 0.9) - 1.0) < 1e-3
    # cautious weight decay: with wd > 0, coordinates whose update opposes
    # the parameter's sign are not decayed
    p = p0.copy()
    o2 = orc.OracleOptimizer(table(muon(0, rows, cols, lr=lr, weight_decay=0.5)))
    o2.step(p, g)
    nodecay = np.zeros(n, f32)
    o3 = orc.OracleOptimizer(table(muon(0, rows, cols, lr=lr, weight_decay=0.0)))
    o3.step(nodecay, g)  # -lr * U from a zero parameter
    u = -nodecay / lr
    mask = (u * p0 >= 0).astype(np.float64)
    want = p0 - lr * u - lr * 0.5 * p0 * mask
    np.testing.assert_allclose(p, want, rtol=1e-5, atol=1e-6)


def test_sinkhorn_single_row(orc):  # sinkhorn_test.go:12-27
    o = orc.OracleOptimizer(table(sinkhorn(0, 1, 2, lr=1, momentum=0, gamma=1, sinkhorn_steps=1,
                                           tau=0, sinkhorn_eps=1e-20)))
    p = np.zeros(2, f32)
    o.step(p, np.array([3, 4], f32))
    np.testing.assert_allclose(p, [-math.sqrt(2) * 0.6, -math.sqrt(2) * 0.8], atol=1e-5)


def test_sinkhorn_masks_near_zero_rows(orc):  # sinkhorn_test.go:29-46
    o = orc.OracleOptimizer(table(sinkhorn(0, 2, 2, lr=1, momentum=0, gamma=1, sinkhorn_steps=1,
                                           tau=0.5, sinkhorn_eps=1e-20)))
    p = np.zeros(4, f32)
    o.step(p, np.array([3, 4, 0, 0], f32))
    assert p[2] == 0 and p[3] == 0 and p[0] != 0 and p[1] != 0


def test_sinkhorn_rows_unit_rms(orc):  # sinkhorn_test.go:48-70
    o = orc.OracleOptimizer(table(sinkhorn(0, 4, 3, lr=1, momentum=0, gamma=1, sinkhorn_steps=11,
                                           tau=0, sinkhorn_eps=1e-20)))
    p = np.zeros(12, f32)
    o.step(p, np.array([1e-3, 2e-3, 3e-3, 4, 5, 6, 7, 8, 9, 0.1, 0.2, 0.3], f32))
    rms = np.sqrt((p.reshape(4, 3).astype(np.float64) ** 2).mean(axis=1))
    np.testing.assert_allclose(rms, 1.0, atol=1e-3)


def test_sinkhorn_momentum_and_row_step(orc):
    """Nesterov in float64: M = (1-b) g, update (1-b^2) g before balancing;
    an odd K ends on a row normalization, so every unmasked row of the
    step has norm gamma * lr * sqrt(cols); masked rows do not move."""
    rng = np.random.default_rng(11)
    rows, cols = 30, 8
    g = rng.standard_normal((rows, cols)).astype(f32)
    g[5] *= 1e-6  # below tau times the mean row norm
    p = rng.standard_normal((rows, cols)).astype(f32).ravel()
    p0 = p.copy()
    gamma, lr = 0.18, 0.01
    o = orc.OracleOptimizer(table(sinkhorn(0, rows, cols, lr=lr, momentum=0.95, gamma=gamma,
                                           sinkhorn_steps=11, tau=1e-3, sinkhorn_eps=1e-20)))
    o.step(p, g.ravel())
    np.testing.assert_allclose(o.state, (1 - 0.95) * g.ravel().astype(np.float64), rtol=1e-6)
    d = (p0.astype(np.float64) - p).reshape(rows, cols)
    norms = np.linalg.norm(d, axis=1)
    assert norms[5] == 0
    keep = np.arange(rows) != 5
    np.testing.assert_allclose(norms[keep], gamma * lr * math.sqrt(cols), rtol=1e-4)


@pytest.mark.parametrize("factory", ["dense_d2", "latent_d12", "flash_d12"])
def test_setup_optimizer_table(factory):
    """model/optimizer.go:16-181 with cmd/chat_rl's arguments: every
    parameter float in exactly one entry (the router bias in none), the
    kinds and learning rates of the named tensors."""
    cfg = getattr(G, factory)()
    tab = OPT.chat_rl_table(cfg)  # _check_cover asserts the coverage
    sl = cfg.param_slices()
    by_off = {int(e["offset"]): e for e in tab}
    scale = f32(math.pow(cfg.n_embd / 768.0, -0.5))
    lm = by_off[sl["lm_head.weight"][0]]
    assert lm["kind"] == OPT.KIND_SINKHORN and lm["lr"] == f32(f32(0.004) * scale) * f32(0.05)
    assert lm["sinkhorn_steps"] == 11 and lm["gamma"] == f32(0.18)
    rl = by_off[sl["resid_lambdas"][0]]
    assert rl["kind"] == OPT.KIND_ADAMW and rl["lr"] == f32(f32(0.5) * f32(0.01)) * f32(0.05)
    assert rl["weight_decay"] == f32(0.05)
    mu = tab[tab["kind"] == OPT.KIND_MUON]
    assert (mu["lr"] == f32(0.02) * f32(0.05)).all() and (mu["ns_steps"] == 5).all()
    if cfg.head_wise_muon:  # c_q split into one [head_dim, C] view per head
        q = sl["transformer.h.0.attn.c_q.weight"]
        views = [e for e in tab if q[0] <= e["offset"] < q[0] + q[1] * q[2]]
        assert len(views) == cfg.n_head and all(v["rows"] == cfg.head_dim for v in views)
    if cfg.moe:  # one view per expert
        up = sl["transformer.h.0.moe.experts.up.weight"]
        views = [e for e in tab if up[0] <= e["offset"] < up[0] + up[1] * up[2]]
        assert len(views) == cfg.n_experts


def test_full_table_step_is_finite(orc):
    cfg = G.dense_d2()
    tab = OPT.chat_rl_table(cfg)
    rng = np.random.default_rng(0)
    w = G.init_weights(cfg, seed=0)
    g = (1e-3 * rng.standard_normal(w.size)).astype(f32)
    o = orc.OracleOptimizer(tab)
    p = w.copy()
    o.step(p, g)
    assert np.isfinite(p).all() and np.isfinite(o.state).all()
    assert (p != w).mean() > 0.99


def test_schedules_known_answers():
    """Trainer.StepOptimizer's schedules against trainer/trainer_test.go:47-78
    (warmup, plateau and end of LRMultiplier; MuonMomentum at 0 and in the
    plateau; WeightDecayCosine at both ends), plus the warmdown ramps at
    points the closed forms fix."""
    assert abs(OPT.lr_multiplier(0, 100, 10, 0.5, 0.05) - 0.1) < 1e-5
    assert OPT.lr_multiplier(50, 100, 10, 0.5, 0.05) == 1.0
    assert abs(OPT.lr_multiplier(100, 100, 10, 0.5, 0.05) - 0.05) < 1e-5
    assert abs(OPT.lr_multiplier(75, 100, 10, 0.5, 0.05) - 0.525) < 1e-6  # half-way down
    assert abs(OPT.muon_momentum(0, 1000, 0.5) - 0.85) < 1e-5
    assert abs(OPT.muon_momentum(500, 1000, 0.5) - 0.97) < 1e-5
    assert abs(OPT.muon_momentum(200, 1000, 0.5) - 0.91) < 1e-6   # half-way up
    assert abs(OPT.muon_momentum(750, 1000, 0.5) - 0.935) < 1e-6  # half-way down
    assert abs(OPT.weight_decay_cosine(0, 100, 0.3) - 0.3) < 1e-5
    assert abs(OPT.weight_decay_cosine(100, 100, 0.3)) < 1e-5
    assert abs(OPT.weight_decay_cosine(50, 100, 0.3) - 0.15) < 1e-6

"""The device MuonAdamW step (gn_optimizer_*) against the oracle's
(oracle/optimizer.c) on the same parameters and gradients: two steps of
cmd/chat_rl's parameter groups (Sinkhorn embedding/unembedding tables,
AdamW scalars, Muon matrices incl. head-wise and per-expert views) for the
dense, latent and flash families.  Every table entry's parameter change and
optimizer state must match within 1e-4 normwise relative (float32; the
Polar Express products run on the fp32 GEMM, the oracle accumulates them
in float64)."""
import numpy as np
import pytest

from conftest import rel_err
from gonano_amd import config as G
from gonano_amd import optimizer as OPT

pytestmark = pytest.mark.gpu


def _cfg(kind):
    from test_gpu_flash import flash_small_cfg
    from test_gpu_latent import latent_small_cfg
    from test_gpu_session import small_cfg
    if kind == "dense":
        return small_cfg()
    if kind == "latent":
        return latent_small_cfg()
    cfg = flash_small_cfg(moe=True)
    cfg.sparse_topk, cfg.indexer_pool, cfg.reuse_pattern = 4, 2, "FRU"
    cfg.head_wise_muon = True
    return cfg


def _pg_grads(s, cfg, seed):
    rng = np.random.default_rng(seed)
    B, T = 2, 96
    inputs = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets[:, :16] = -1
    s.zero_grad()
    s.policy_gradient_step(inputs, targets, np.array([0.5, -0.5], np.float32), float(T + 1))
    return s.grads()


def _state_slices(table):
    out, off = [], 0
    for e in table:
        n = int(e["rows"]) * int(e["cols"])
        size = 2 * n if e["kind"] == OPT.KIND_ADAMW else (
            n + max(int(e["rows"]), int(e["cols"])) if e["kind"] == OPT.KIND_MUON else n)
        out.append((off, size))
        off += size
    return out


def _compare(table, p0, got, want, st_got, st_want, what):
    kinds = {OPT.KIND_ADAMW: "adamw", OPT.KIND_MUON: "muon", OPT.KIND_SINKHORN: "sinkhorn"}
    for e, (so, sn) in zip(table, _state_slices(table)):
        o, n = int(e["offset"]), int(e["rows"]) * int(e["cols"])
        dg = got[o:o + n].astype(np.float64) - p0[o:o + n]
        dw = want[o:o + n].astype(np.float64) - p0[o:o + n]
        tag = f"{what} {kinds[int(e['kind'])]} entry at {o} [{e['rows']}x{e['cols']}]"
        if np.linalg.norm(dw) > 0:
            assert rel_err(dg, dw) < 1e-4, (tag, rel_err(dg, dw))
        else:
            assert np.linalg.norm(dg) == 0, tag
        sg, sw = st_got[so:so + sn], st_want[so:so + sn]
        if np.linalg.norm(sw) > 0:
            assert rel_err(sg, sw) < 1e-4, (tag + " state", rel_err(sg, sw))


@pytest.mark.parametrize("kind", ["dense", "latent", "flash"])
def test_optimizer_two_steps_match_oracle(orc, kind):
    from gonano_amd.session import Session
    cfg = _cfg(kind)
    table = OPT.chat_rl_table(cfg)
    w = G.init_weights(cfg, seed=5, perturb=0.05)
    ref = orc.OracleOptimizer(table)
    with Session(cfg) as s:
        s.set_params(w)
        with OPT.Optimizer(s, table) as opt:
            g1 = _pg_grads(s, cfg, 1)
            opt.step()
            p1 = s.get_params()
            st1 = opt.state()
            want1 = w.copy()
            ref.step(want1, g1)
            _compare(table, w, p1, want1, st1, ref.state, f"{kind} step 1")
            # step 2 from the device's parameters (its gradients were taken
            # there); the oracle keeps its own state
            g2 = _pg_grads(s, cfg, 2)
            opt.step()
            p2 = s.get_params()
            st2 = opt.state()
            want2 = p1.copy()
            ref.step(want2, g2)
            _compare(table, p1, p2, want2, st2, ref.state, f"{kind} step 2")
            assert (ref.steps[table["kind"] == OPT.KIND_ADAMW] == 2).all()


def test_optimizer_rejects_bad_tables():
    from gonano_amd._lib import HipError
    from gonano_amd.session import Session
    from test_gpu_session import small_cfg
    cfg = small_cfg()
    with Session(cfg) as s:
        bad = OPT.chat_rl_table(cfg)[:1].copy()
        bad["offset"] = cfg.param_total()  # outside every parameter
        with pytest.raises(HipError):
            OPT.Optimizer(s, bad)
        bad = OPT.chat_rl_table(cfg)
        bad = bad[bad["kind"] == OPT.KIND_MUON][:1].copy()
        bad["ns_steps"] = 6  # five Polar Express coefficient sets
        with pytest.raises(HipError):
            OPT.Optimizer(s, bad)


def test_step_optimizer_schedules_and_router_bias(orc):
    """Trainer.StepOptimizer (trainer/trainer.go:80-102) at a warmdown step:
    the groups' LR / Momentum / WeightDecay set through gn_optimizer_set_hyper
    (the step equals the oracle's with the scheduled table), then
    UpdateRouterBias (moe.go:330-341) from the tokens the training forward
    counted (MoE.forwardTraining, moe.go:192-193: B*T*K per layer and
    forward) and ZeroGrad; a second update with no training forward in
    between changes nothing (the counts were cleared)."""
    from gonano_amd.session import Session
    cfg = _cfg("latent")
    assert cfg.n_experts > 0
    table = OPT.chat_rl_table(cfg)
    w = G.init_weights(cfg, seed=5, perturb=0.05)
    step, iters, warmup, ratio, final, wd0 = 700, 1000, 0, 0.5, 0.1, 0.2
    mult = OPT.lr_multiplier(step, iters, warmup, ratio, final)
    mom = OPT.muon_momentum(step, iters, ratio)
    wd = OPT.weight_decay_cosine(step, iters, wd0)
    assert abs(mult - 0.64) < 1e-6 and abs(mom - 0.942) < 1e-6  # 200/500 into the warmdown
    sched = table.copy()
    sched["lr"] = (table["lr"] * np.float32(mult)).astype(np.float32)
    muon, sink = table["kind"] == OPT.KIND_MUON, table["kind"] == OPT.KIND_SINKHORN
    sched["momentum"][muon | sink] = np.float32(mom)
    sched["weight_decay"][muon] = np.float32(wd)
    sched["weight_decay"][sink] = 0
    ref = orc.OracleOptimizer(sched)
    slices = cfg.param_slices()
    bias_names = [f"transformer.h.{l}.moe.router_bias" for l in range(cfg.n_layer)]
    assert all(n in slices for n in bias_names)
    with Session(cfg) as s:
        s.set_params(w)
        assert not s.moe_loads().any()
        with OPT.Optimizer(s, table) as opt:
            g = _pg_grads(s, cfg, 1)  # one training forward of B x T = 2 x 96 tokens
            loads = s.moe_loads()
            assert loads.shape == (cfg.n_layer, cfg.n_experts)
            assert (loads >= 0).all() and (loads == np.round(loads)).all()
            assert (loads.sum(1) == 2 * 96 * cfg.experts_per_token).all()
            OPT.step_optimizer(opt, s, table["lr"], step, iters, warmup, ratio, final, wd0)
            p = s.get_params()
            want = w.copy()
            ref.step(want, g)
            _compare(table, w, p, want, opt.state(), ref.state, "scheduled step")
            speed = np.float32(0.001)  # Config.MoERouterBiasUpdate() default
            for l, name in enumerate(bias_names):
                off, r, c = slices[name]
                mean = loads[l].sum() / cfg.n_experts
                expect = (w[off:off + r * c] + speed * np.sign(mean - loads[l]).astype(np.float32))
                assert np.array_equal(p[off:off + r * c], expect.astype(np.float32)), name
            assert not s.moe_loads().any()
            assert not s.grads().any()
            s.update_router_bias()
            assert np.array_equal(s.get_params(), p)

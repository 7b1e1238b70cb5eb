"""MuonAdamW on the device over the HIP C ABI (include/gonano_hip.h).

Mirrors the reference's optimizer set-up and step:

* ``setup_optimizer`` is Transformer.SetupOptimizer (model/optimizer.go:16-181):
  the parameter groups (Sinkhorn or AdamW for the embedding, unembedding and
  value-embedding tables; AdamW for the scalars; Muon for every matrix,
  binned by shape, with head-wise q/k views and per-expert views), flattened
  to one table entry per tensor or view in the order MuonAdamW.Step visits
  them (optimizer/optimizer.go:118-137).
* ``chat_rl_table`` is cmd/chat_rl's call (cmd/chat_rl/main.go:68-71):
  SetupOptimizer(0.004, 0.2, 0.02, 0.0, 0.5, sinkhorn=true), every group's
  learning rate times 0.05.
* ``Optimizer`` is optimizer.NewMuonAdamW + MuonAdamW.Step on a Session's
  device parameters and gradients.
"""
from __future__ import annotations

import ctypes as C
import math

import numpy as np

from ._lib import call
from .config import Config

KIND_ADAMW, KIND_MUON, KIND_SINKHORN = 0, 1, 2

# gn_opt_param (C layout)
OPT_PARAM_DTYPE = np.dtype([
    ("offset", np.int64), ("rows", np.int32), ("cols", np.int32), ("kind", np.int32),
    ("lr", np.float32), ("beta1", np.float32), ("beta2", np.float32), ("eps", np.float32),
    ("weight_decay", np.float32), ("momentum", np.float32), ("ns_steps", np.int32),
    ("muon_beta2", np.float32), ("gamma", np.float32), ("sinkhorn_steps", np.int32),
    ("tau", np.float32), ("sinkhorn_eps", np.float32)], align=True)

_f32 = np.float32


def _entry(offset, rows, cols, kind, **hyper):
    e = np.zeros((), OPT_PARAM_DTYPE)
    e["offset"], e["rows"], e["cols"], e["kind"] = offset, rows, cols, kind
    for k, v in hyper.items():
        e[k] = v
    return e


def _views(off: int, count: int, rows: int, cols: int):
    """Row-block views of a packed [count*rows, cols] weight: headWiseViews /
    expertViews (model/optimizer.go:153-181)."""
    return [(off + i * rows * cols, rows, cols) for i in range(count)]


def setup_optimizer(cfg: Config, unembedding_lr: float, embedding_lr: float, matrix_lr: float,
                    weight_decay: float, scalar_lr: float, sinkhorn: bool,
                    lr_scale: float = 1.0) -> np.ndarray:
    """Transformer.SetupOptimizer (model/optimizer.go:16-141) as a table of
    gn_opt_param entries; every group's LR is multiplied by lr_scale in
    float32 afterwards (as cmd/chat_rl does)."""
    sl = cfg.param_slices()
    D = cfg.head_dim

    def T(name):
        off, r, c = sl[name]
        return (off, r, c)

    matrices = []  # (offset, rows, cols) in matrixParameters order
    for l in range(cfg.n_layer):
        p = f"transformer.h.{l}."
        if cfg.mla:
            for n in ("mla_q_down", "mla_q_up", "mla_q_rope", "mla_kv_down", "mla_k_up",
                      "mla_v_up", "mla_k_rope"):
                matrices.append(T(p + f"attn.{n}.weight"))
            matrices += [T(p + "attn.c_proj.weight"), T(p + "mlp.c_fc.weight"),
                         T(p + "mlp.c_proj.weight")]
            if p + "mlp.c_gate.weight" in sl:
                matrices.append(T(p + "mlp.c_gate.weight"))
            if p + "attn.ve_gate.weight" in sl:
                matrices.append(T(p + "attn.ve_gate.weight"))
            continue
        if cfg.head_wise_muon:
            q, k = T(p + "attn.c_q.weight"), T(p + "attn.c_k.weight")
            matrices += _views(q[0], cfg.n_head, D, q[2])
            matrices += _views(k[0], cfg.n_kv_head, D, k[2])
        else:
            matrices += [T(p + "attn.c_q.weight"), T(p + "attn.c_k.weight")]
        matrices += [T(p + "attn.c_v.weight"), T(p + "attn.c_proj.weight"),
                     T(p + "mlp.c_fc.weight"), T(p + "mlp.c_proj.weight")]
        for n in ("mlp.c_gate.weight", "attn.ve_gate.weight", "attn.compress_logits.weight",
                  "attn.indexer_query.weight", "attn.indexer_key.weight"):
            if p + n in sl:
                matrices.append(T(p + n))
    if cfg.moe:  # router + per-expert views; the router bias is not optimized
        E, EH, C_ = cfg.n_experts, cfg.expert_hidden, cfg.n_embd
        for l in range(cfg.n_layer):
            p = f"transformer.h.{l}.moe."
            matrices.append(T(p + "router.weight"))
            matrices += _views(sl[p + "experts.gate.weight"][0], E, EH, C_)
            matrices += _views(sl[p + "experts.up.weight"][0], E, EH, C_)
            matrices += _views(sl[p + "experts.down.weight"][0], E, C_, EH)

    ve = [T(n) for n in sorted(sl) if n.startswith("value_embeds.")]
    ve.sort(key=lambda t: t[0])
    smear = [T("smear_gate.weight"), T("smear_lambda"), T("backout_lambda")]
    for l in range(cfg.n_layer):
        p = f"transformer.h.{l}.attn."
        for n in ("compress_bias", "indexer_heads"):
            if p + n in sl:
                smear.append(T(p + n))

    scale = _f32(math.pow(cfg.n_embd / 768.0, -0.5))
    groups = []  # (kind, tensors, hyper)
    if sinkhorn:
        def sk(tensors, lr):  # sinkhornGroup (model/optimizer.go:143-151)
            return (KIND_SINKHORN, tensors, dict(lr=lr, momentum=0.95, gamma=0.18,
                                                 sinkhorn_steps=11, tau=1e-3, sinkhorn_eps=1e-20))
        groups += [sk([T("lm_head.weight")], _f32(unembedding_lr) * scale),
                   sk([T("transformer.wte.weight")], _f32(embedding_lr) * scale),
                   sk(ve, _f32(embedding_lr) * scale * _f32(0.5))]
    else:
        groups += [(KIND_ADAMW, [T("lm_head.weight")],
                    dict(lr=_f32(unembedding_lr) * scale, beta1=0.8, beta2=0.96, eps=1e-10,
                         weight_decay=0.01)),
                   (KIND_ADAMW, [T("transformer.wte.weight")],
                    dict(lr=_f32(embedding_lr) * scale, beta1=0.8, beta2=0.995, eps=1e-10,
                         weight_decay=0.001)),
                   (KIND_ADAMW, ve, dict(lr=_f32(embedding_lr) * scale * _f32(0.5), beta1=0.8,
                                         beta2=0.995, eps=1e-10, weight_decay=0.01))]
    groups += [(KIND_ADAMW, [T("resid_lambdas")],
                dict(lr=_f32(scalar_lr) * _f32(0.01), beta1=0.8, beta2=0.95, eps=1e-10,
                     weight_decay=0.05)),
               (KIND_ADAMW, [T("x0_lambdas")],
                dict(lr=_f32(scalar_lr), beta1=0.96, beta2=0.95, eps=1e-10, weight_decay=0.0)),
               (KIND_ADAMW, smear, dict(lr=_f32(0.2), beta1=0.8, beta2=0.95, eps=1e-10,
                                         weight_decay=0.0))]
    by_shape: dict[tuple[int, int], list] = {}
    for t in matrices:
        by_shape.setdefault((t[1], t[2]), []).append(t)
    for shape in sorted(by_shape):
        groups.append((KIND_MUON, by_shape[shape],
                       dict(lr=_f32(matrix_lr), momentum=0.95, ns_steps=5, muon_beta2=0.9,
                            weight_decay=_f32(weight_decay))))

    entries = []
    for kind, tensors, hyper in groups:
        hyper = dict(hyper)
        hyper["lr"] = _f32(hyper["lr"]) * _f32(lr_scale)
        for off, r, c in tensors:
            entries.append(_entry(off, r, c, kind, **hyper))
    table = np.array(entries, OPT_PARAM_DTYPE)
    _check_cover(cfg, table)
    return table


def _check_cover(cfg: Config, table: np.ndarray):
    """Every parameter float is optimized exactly once, except the MoE router
    correction bias (updated by load, not by the optimizer)."""
    covered = np.zeros(cfg.param_total(), np.int8)
    for e in table:
        n = int(e["rows"]) * int(e["cols"])
        covered[e["offset"]:e["offset"] + n] += 1
    for name, (off, r, c) in cfg.param_slices().items():
        want = 0 if name.endswith("moe.router_bias") else 1
        if not (covered[off:off + r * c] == want).all():
            raise AssertionError(f"optimizer groups cover {name} wrongly")


def chat_rl_table(cfg: Config) -> np.ndarray:
    """cmd/chat_rl/main.go:68-71."""
    return setup_optimizer(cfg, 0.004, 0.2, 0.02, 0.0, 0.5, True, lr_scale=0.05)


def state_floats(table: np.ndarray) -> int:
    n = table["rows"].astype(np.int64) * table["cols"].astype(np.int64)
    side = np.maximum(table["rows"], table["cols"]).astype(np.int64)
    return int(np.where(table["kind"] == KIND_ADAMW, 2 * n,
                        np.where(table["kind"] == KIND_MUON, n + side, n)).sum())


class Optimizer:
    """optimizer.NewMuonAdamW over a Session (its device parameters)."""

    def __init__(self, session, table: np.ndarray):
        self.table = np.ascontiguousarray(table, OPT_PARAM_DTYPE)
        self._session = session
        h = C.c_void_p()
        call("gn_optimizer_create", session._h, self.table.ctypes.data_as(C.c_void_p),
             len(self.table), C.byref(h))
        self._h = h

    def step(self):
        """MuonAdamW.Step (optimizer/optimizer.go:118-137)."""
        call("gn_optimizer_step", self._h)

    def set_hyper(self, lr=None, momentum=None, weight_decay=None):
        """Per-entry LR / Momentum / WeightDecay (table order); None keeps a
        field as it is."""
        arrs = []
        for v in (lr, momentum, weight_decay):
            arrs.append(None if v is None else np.ascontiguousarray(
                np.broadcast_to(np.asarray(v, np.float32), (len(self.table),))))
        ptr = [None if a is None else a.ctypes.data_as(C.c_void_p) for a in arrs]
        call("gn_optimizer_set_hyper", self._h, ptr[0], ptr[1], ptr[2], len(self.table))
        for name, a in zip(("lr", "momentum", "weight_decay"), arrs):
            if a is not None:
                self.table[name] = a

    def state(self) -> np.ndarray:
        n = C.c_int64()
        call("gn_optimizer_state_size", self._h, C.byref(n))
        out = np.empty(n.value, np.float32)
        call("gn_optimizer_get_state", self._h, out, out.size)
        return out

    def close(self):
        if self._h:
            call("gn_optimizer_destroy", self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


# ---- Trainer.StepOptimizer's schedules (trainer/scheduler.go:10-41) ----------
def lr_multiplier(step: int, num_iterations: int, warmup_steps: int, warmdown_ratio: float,
                  final_lr_frac: float) -> float:
    """trainer/scheduler.go:10-20, in float32 as the reference computes it."""
    f = np.float32
    warmdown = int(f(num_iterations) * f(warmdown_ratio))
    if step < warmup_steps:
        return float(f(step + 1) / f(warmup_steps))
    if step <= num_iterations - warmdown:
        return 1.0
    progress = f(num_iterations - step) / f(warmdown)
    return float(progress * f(1.0) + (f(1) - progress) * f(final_lr_frac))


def muon_momentum(step: int, num_iterations: int, warmdown_ratio: float) -> float:
    """trainer/scheduler.go:24-36."""
    f = np.float32
    warmdown = int(f(num_iterations) * f(warmdown_ratio))
    start = num_iterations - warmdown
    if step < 400:
        fr = f(step) / f(400)
        return float((f(1) - fr) * f(0.85) + fr * f(0.97))
    if step >= start:
        progress = f(step - start) / f(warmdown)
        return float(f(0.97) * (f(1) - progress) + f(0.90) * progress)
    return 0.97


def weight_decay_cosine(step: int, num_iterations: int, base: float) -> float:
    """trainer/scheduler.go:39-41."""
    f = np.float32
    return float(f(base) * f(0.5) * f(1 + math.cos(math.pi * float(step) / float(num_iterations))))


def step_optimizer(opt: "Optimizer", session, initial_lr: np.ndarray, step: int,
                   num_iterations: int, warmup_steps: int, warmdown_ratio: float,
                   final_lr_frac: float, weight_decay: float):
    """Trainer.StepOptimizer (trainer/trainer.go:80-102): the LR multiplier on
    every group, the Muon momentum and cosine weight decay on Muon groups,
    the momentum and zero weight decay on Sinkhorn groups; then the step,
    UpdateRouterBias and ZeroGrad.  initial_lr: the table's LRs at creation."""
    f = np.float32
    mult = f(lr_multiplier(step, num_iterations, warmup_steps, warmdown_ratio, final_lr_frac))
    mom = f(muon_momentum(step, num_iterations, warmdown_ratio))
    wd = f(weight_decay_cosine(step, num_iterations, weight_decay))
    kind = opt.table["kind"]
    lr = (np.asarray(initial_lr, np.float32) * mult).astype(np.float32)
    momentum = np.where(kind == KIND_ADAMW, opt.table["momentum"], mom).astype(np.float32)
    decay = np.where(kind == KIND_MUON, wd,
                     np.where(kind == KIND_SINKHORN, f(0), opt.table["weight_decay"])).astype(np.float32)
    opt.set_hyper(lr, momentum, decay)
    opt.step()
    session.update_router_bias()
    session.zero_grad()

"""Model configuration for the RL-step path: gonano's ``model.Config`` and the
helpers that derive it, restated for the host side of the HIP backend.

Citations refer to the gonano source tree.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

SMEAR_GATE_CHANNELS = 24  # model/helpers.go:7
VE_GATE_CHANNELS = 12  # model/attention.go:18
VOCAB_PADDING = 64  # model/config.go:620


@dataclass
class Config:
    """model.Config (model/config.go:9-124), dense fields."""

    sequence_len: int
    vocab_size: int
    n_layer: int
    n_head: int
    n_kv_head: int
    n_embd: int
    window_pattern: str = "SSSL"
    rotary_dims: int = 0

    # -- derived quantities -------------------------------------------------
    @property
    def head_dim(self) -> int:  # model/config.go:447
        return self.n_embd // self.n_head

    @property
    def rotary_dimension(self) -> int:  # model/config.go:430-444
        if self.rotary_dims <= 0:
            return self.head_dim
        if self.rotary_dims > self.head_dim:
            raise ValueError(f"RotaryDims {self.rotary_dims} exceeds head dim {self.head_dim}")
        if self.rotary_dims % 2:
            raise ValueError(f"RotaryDims {self.rotary_dims} must be even")
        return self.rotary_dims

    @property
    def padded_vocab(self) -> int:  # model/config.go:622-624
        return ((self.vocab_size + VOCAB_PADDING - 1) // VOCAB_PADDING) * VOCAB_PADDING

    @property
    def mlp_hidden(self) -> int:  # model/mlp.go:35-37
        return 4 * self.n_embd

    def has_value_embedding(self, layer: int) -> bool:  # model/helpers.go:69-71
        return layer % 2 == (self.n_layer - 1) % 2

    def window_sizes(self) -> list[int]:
        """model/config.go:629-645; Go's integer division truncates toward zero."""
        T = self.sequence_len
        # -((-T/4)/128)*128 with truncating division equals floor(floor(T/4)/128)*128
        short = ((T // 4) // 128) * 128
        out = []
        for layer in range(self.n_layer):
            ch = self.window_pattern[layer % len(self.window_pattern)]
            out.append(T if ch in "Ll" else short)
        out[-1] = T
        return out

    def validate(self) -> None:  # model/config.go:453-466 (dense subset)
        if self.n_embd % self.n_head:
            raise ValueError(f"EmbedDim {self.n_embd} not divisible by NumHead {self.n_head}")
        if self.n_kv_head > self.n_head or self.n_head % self.n_kv_head:
            raise ValueError(f"NumKVHead {self.n_kv_head} must divide NumHead {self.n_head}")
        for ch in self.window_pattern:
            if ch not in "LSls":
                raise ValueError(f"invalid window pattern {self.window_pattern!r}")
        _ = self.rotary_dimension

    # -- parameter table (model/params.go:14-85, sorted as ParameterNames) ---
    def param_table(self) -> list[tuple[str, int, int, int]]:
        C_, D, PV = self.n_embd, self.head_dim, self.padded_vocab
        ents = [("transformer.wte.weight", PV, C_), ("lm_head.weight", PV, C_)]
        for l in range(self.n_layer):
            p = f"transformer.h.{l}."
            ents += [(p + "attn.c_q.weight", self.n_head * D, C_),
                     (p + "attn.c_k.weight", self.n_kv_head * D, C_),
                     (p + "attn.c_v.weight", self.n_kv_head * D, C_),
                     (p + "attn.c_proj.weight", C_, C_)]
            if self.has_value_embedding(l):
                ents += [(p + "attn.ve_gate.weight", self.n_kv_head, VE_GATE_CHANNELS),
                         (f"value_embeds.{l}.weight", PV, self.n_kv_head * D)]
            ents += [(p + "mlp.c_fc.weight", self.mlp_hidden, C_),
                     (p + "mlp.c_proj.weight", C_, self.mlp_hidden)]
        ents += [("resid_lambdas", self.n_layer, 1), ("x0_lambdas", self.n_layer, 1),
                 ("smear_gate.weight", 1, SMEAR_GATE_CHANNELS), ("smear_lambda", 1, 1),
                 ("backout_lambda", 1, 1)]
        ents.sort(key=lambda e: e[0].encode())
        out, off = [], 0
        for name, r, c in ents:
            out.append((name, r, c, off))
            off += r * c
        return out

    def param_total(self) -> int:
        t = self.param_table()
        return t[-1][3] + t[-1][1] * t[-1][2]

    def param_slices(self) -> dict[str, tuple[int, int, int]]:
        return {n: (off, r, c) for n, r, c, off in self.param_table()}


def config_for_depth_ratio(depth: int, vocab_size: int, aspect_ratio: int, head_dim: int,
                           seq_len: int, window_pattern: str, kv_head_ratio: int) -> Config:
    """model/config.go:575-604 (ConfigForDepthRatio)."""
    if kv_head_ratio < 1:
        raise ValueError(f"kvHeadRatio {kv_head_ratio} must be >= 1")
    base = depth * aspect_ratio
    model_dim = ((base + head_dim - 1) // head_dim) * head_dim
    heads = model_dim // head_dim
    if heads % kv_head_ratio:
        raise ValueError(f"numHeads {heads} not divisible by kvHeadRatio {kv_head_ratio}")
    rot = min(64, head_dim)  # defaultRotaryDims, model/config.go:425,585-591
    if rot % 2:
        rot -= 1
    cfg = Config(seq_len, vocab_size, depth, heads, heads // kv_head_ratio, model_dim,
                 window_pattern, rot)
    cfg.validate()
    return cfg


def dense_d2() -> Config:
    """ConfigForPreset(dense, 2, 32768, 64, 128, 512, "SSSL")."""
    return config_for_depth_ratio(2, 32768, 64, 128, 512, "SSSL", 1)


def dense_d12() -> Config:
    """depth 12, 6 query heads, 2 KV heads, vocab 65536, seq 512."""
    return config_for_depth_ratio(12, 65536, 64, 128, 512, "SSSL", 3)


def dense_d20() -> Config:
    """depth 20, 10 query heads, 2 KV heads, seq 2048."""
    return config_for_depth_ratio(20, 65536, 64, 128, 2048, "SSSL", 5)


# ---------------------------------------------------------------------------
# Weights with InitWeights' distributions (model/transformer.go:139-205).
# Go's NormFloat64 stream and its map-ordered value-embedding init are not
# reproducible outside Go, so weights are generated from numpy and handed to
# both sides as an input.
# ---------------------------------------------------------------------------
def init_weights(cfg: Config, seed: int = 0, perturb: float = 0.0,
                 perturb_seed: int = 123) -> np.ndarray:
    rng = np.random.default_rng(seed)
    total = cfg.param_total()
    w = np.zeros(total, np.float32)
    sl = cfg.param_slices()
    bound = math.sqrt(3.0) / math.sqrt(cfg.n_embd)  # uniformBound, transformer.go:18-20

    def put(name, values):
        off, r, c = sl[name]
        w[off:off + r * c] = np.asarray(values, np.float32).reshape(-1)

    def n(name):
        off, r, c = sl[name]
        return r * c

    put("transformer.wte.weight", rng.standard_normal(n("transformer.wte.weight")) * 0.8)
    put("lm_head.weight", rng.standard_normal(n("lm_head.weight")) * 0.001)
    for l in range(cfg.n_layer):
        p = f"transformer.h.{l}."
        for k in ("attn.c_q.weight", "attn.c_k.weight", "attn.c_v.weight"):
            put(p + k, rng.uniform(-bound, bound, n(p + k)))
        put(p + "mlp.c_fc.weight", rng.uniform(-0.4 * bound, 0.4 * bound, n(p + "mlp.c_fc.weight")))
        # c_proj weights stay zero (transformer.go:162,167)
    L1 = max(cfg.n_layer - 1, 1)
    put("resid_lambdas", [1.15 - 0.10 * l / L1 for l in range(cfg.n_layer)])
    put("x0_lambdas", [0.20 - 0.15 * l / L1 for l in range(cfg.n_layer)])
    put("smear_lambda", [0.0])
    put("backout_lambda", [0.2])
    put("smear_gate.weight", rng.uniform(0.0, 0.02, SMEAR_GATE_CHANNELS))
    for l in range(cfg.n_layer):
        if cfg.has_value_embedding(l):
            put(f"value_embeds.{l}.weight", rng.uniform(-bound, bound, n(f"value_embeds.{l}.weight")))
    for l in range(cfg.n_layer):
        if cfg.has_value_embedding(l):
            k = f"transformer.h.{l}.attn.ve_gate.weight"
            put(k, rng.uniform(0.0, 0.02, n(k)))
    if perturb:
        # model/gradcheck_test.go:24-30: every parameter += N(0,1)*0.1 in sorted order
        prng = np.random.default_rng(perturb_seed)
        w += (prng.standard_normal(total) * perturb).astype(np.float32)
    return w

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


DEFAULT_ROTARY_DIMS = 64  # model/config.go:425
DEFAULT_MOE_CLAMP = 10.0  # model/config.go:125
DEFAULT_MOE_BALANCE_WEIGHT = 1e-4  # model/config.go:134


@dataclass
class Config:
    """model.Config (model/config.go:9-124): the dense fields plus the latent
    preset's MLA and DeepSeekMoE fields.  MoE fields hold resolved values
    (ApplyMoEDefaults, MoEEffectiveClamp/Scale, MoEBalanceLossWeight); zeros
    keep the dense model."""

    sequence_len: int
    vocab_size: int
    n_layer: int
    n_head: int
    n_kv_head: int
    n_embd: int
    window_pattern: str = "SSSL"
    rotary_dims: int = 0
    mla_latent: int = 0          # Config.MLALatent
    mla_rope_dims: int = 0       # Config.MLARotaryDims (0: default)
    n_experts: int = 0           # Config.NumExperts
    experts_per_token: int = 0   # MoEActiveExperts()
    expert_hidden: int = 0       # MoEExpertHidden()
    shared_hidden: int = 0       # MoESharedHidden()
    moe_clamp: float = 0.0       # MoEEffectiveClamp() (negative: no clamping)
    moe_scale: float = 0.0       # MoEEffectiveScale()
    balance_weight: float = 0.0  # MoEBalanceLossWeight()
    compression_ratio: int = 0   # Config.CompressionRatio (> 1: HCA compressed layers)
    swa_window: int = 0          # Config.SWAWindowSize(): local branch of compressed layers
    sparse_topk: int = 0         # Config.SparseTopK (> 0: CSA lightning-indexer selection)
    indexer_dim: int = 0         # Config.IndexerDim (0: 64)
    indexer_heads: int = 0       # Config.IndexerHeads (0: 1)
    indexer_pool: int = 0        # Config.IndexerPool (> 1: hierarchical indexer)
    indexer_candidates: int = 0  # Config.IndexerCandidates (0: max(8*SparseTopK, 64))
    indexer_weight: float = 0.0  # Config.IndexerLossWeight (0: 1)
    reuse_pattern: str = ""      # Config.ReusePattern ("FRU": Full / Reindex / Reuse layers)
    ced: bool = False            # Config.CED (causal encoder-decoder split)
    head_wise_muon: bool = False  # Config.HeadWiseMuon (optimizer: per-head q/k views)
    router_bias_update: float = 0.0  # Config.RouterBiasUpdate as given (0: 0.001); only the
                                     # router-bias update reads it, which the RL step skips

    # -- derived quantities -------------------------------------------------
    @property
    def head_dim(self) -> int:  # model/config.go:447
        return self.n_embd // self.n_head

    @property
    def mla_rope_dimension(self) -> int:  # model/config.go:262-280
        if self.mla_rope_dims <= 0:
            width = min(self.head_dim // 2, DEFAULT_ROTARY_DIMS)
            return width - (width % 2)
        if self.mla_rope_dims > self.head_dim:
            raise ValueError(f"MLARotaryDims {self.mla_rope_dims} exceeds head dim {self.head_dim}")
        if self.mla_rope_dims % 2:
            raise ValueError(f"MLARotaryDims {self.mla_rope_dims} must be even")
        return self.mla_rope_dims

    @property
    def mla(self) -> bool:  # model/config.go:250
        return self.mla_latent > 0

    @property
    def moe(self) -> bool:  # model/config.go:138
        return self.n_experts > 0

    @property
    def compression(self) -> int:  # model/config.go:407-414
        return self.compression_ratio if self.compression_ratio > 1 else 1

    @property
    def rotary_dimension(self) -> int:  # model/config.go:430-444
        if self.mla:
            return self.mla_rope_dimension
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
    def mlp_hidden(self) -> int:  # model/mlp.go:35-37, model/block.go:23-28
        return self.shared_hidden if self.moe else 4 * self.n_embd

    # -- flash preset layer roles (model/config.go:282-402) ------------------
    @property
    def ced_split(self) -> int:
        return self.n_layer // 2 if self.ced else 0

    def _reuse_start(self, layer: int) -> int:
        split = self.ced_split
        return split if (self.ced and split > 0 and layer >= split) else 0

    def reuse_mode_at(self, layer: int) -> str:
        """'F' (owns compressor and indexer), 'R' (own indexer on the group's
        compressed KV) or 'U' (reuses both), config.go:326-344."""
        if not self.reuse_pattern:
            return "F"
        ch = self.reuse_pattern[(layer - self._reuse_start(layer)) % len(self.reuse_pattern)]
        return {"R": "R", "r": "R", "U": "U", "u": "U"}.get(ch, "F")

    def reuse_producer(self, layer: int) -> int:  # config.go:357-370
        if self.reuse_mode_at(layer) == "F":
            return layer
        for i in range(layer - 1, self._reuse_start(layer) - 1, -1):
            if self.reuse_mode_at(i) == "F":
                return i
        return layer

    @property
    def indexer_shape(self) -> tuple[int, int]:  # (dim, heads), config.go:391-402
        return (self.indexer_dim if self.indexer_dim > 0 else 64,
                self.indexer_heads if self.indexer_heads > 0 else 1)

    @property
    def indexer_budget(self) -> int:  # config.go:372-381
        if self.indexer_candidates > 0:
            return self.indexer_candidates
        return max(8 * self.sparse_topk, 64)

    def has_value_embedding(self, layer: int) -> bool:
        """model/helpers.go:69-71; never under MLA (model/transformer.go:72-78)."""
        return not self.mla and layer % 2 == (self.n_layer - 1) % 2

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
        if self.mla and self.head_dim - self.mla_rope_dimension <= 0:  # config.go:502-504
            raise ValueError("MLA content dimension must be positive")
        if self.mla and self.compression > 1:  # config.go:483-486
            raise ValueError("MLA is not supported with compression")
        if self.sparse_topk > 0 and self.compression <= 1:  # config.go:465-467
            raise ValueError("SparseTopK requires CompressionRatio > 1")
        if self.reuse_pattern:  # config.go:506-520
            if self.compression <= 1:
                raise ValueError("ReusePattern requires CompressionRatio > 1")
            if any(ch not in "FRUfru" for ch in self.reuse_pattern):
                raise ValueError(f"invalid reuse pattern {self.reuse_pattern!r}")
            if self.reuse_pattern[0] not in "Ff":
                raise ValueError(f"reuse pattern {self.reuse_pattern!r} must start with F")
        if self.ced:  # config.go:521-533
            if self.compression <= 1 or self.swa_window <= 0 or self.n_layer < 2:
                raise ValueError("CED requires compression, a local window and >= 2 layers")
            if self.reuse_pattern and self.reuse_mode_at(self.ced_split) != "F":
                raise ValueError("CED reuse pattern must start each half with F")
        if self.moe and not 0 < self.experts_per_token <= self.n_experts:  # config.go:535-541
            raise ValueError(f"NumExpertsPerToken {self.experts_per_token} must be in "
                             f"[1, NumExperts={self.n_experts}]")

    # -- parameter table (model/params.go:14-85, sorted as ParameterNames) ---
    def param_table(self) -> list[tuple[str, int, int, int]]:
        C_, D, PV = self.n_embd, self.head_dim, self.padded_vocab
        ents = [("transformer.wte.weight", PV, C_), ("lm_head.weight", PV, C_)]
        Hq, Hkv, F = self.n_head, self.n_kv_head, self.mlp_hidden
        for l in range(self.n_layer):
            p = f"transformer.h.{l}."
            if self.mla:  # model/params.go:19-27, model/mla.go:41-58
                lat, rd = self.mla_latent, self.mla_rope_dimension
                cd = D - rd
                ents += [(p + "attn.mla_q_down.weight", lat, C_),
                         (p + "attn.mla_q_up.weight", Hq * cd, lat),
                         (p + "attn.mla_q_rope.weight", Hq * rd, C_),
                         (p + "attn.mla_kv_down.weight", lat, C_),
                         (p + "attn.mla_k_up.weight", Hkv * cd, lat),
                         (p + "attn.mla_v_up.weight", Hkv * D, lat),
                         (p + "attn.mla_k_rope.weight", Hkv * rd, C_)]
            else:
                ents += [(p + "attn.c_q.weight", Hq * D, C_),
                         (p + "attn.c_k.weight", Hkv * D, C_),
                         (p + "attn.c_v.weight", Hkv * D, C_)]
            ents += [(p + "attn.c_proj.weight", C_, C_)]
            if self.compression > 1:  # model/params.go:43-51, attention.go:210-226
                mode = self.reuse_mode_at(l)
                if mode == "F":
                    ents += [(p + "attn.compress_logits.weight", D, C_),
                             (p + "attn.compress_bias", self.compression, D)]
                if self.sparse_topk > 0 and mode != "U":
                    idim, ih = self.indexer_shape
                    ents += [(p + "attn.indexer_query.weight", ih * idim, C_),
                             (p + "attn.indexer_key.weight", ih * idim, D),
                             (p + "attn.indexer_heads", ih, 1)]
            if self.has_value_embedding(l):
                ents += [(p + "attn.ve_gate.weight", Hkv, VE_GATE_CHANNELS),
                         (f"value_embeds.{l}.weight", PV, Hkv * D)]
            ents += [(p + "mlp.c_fc.weight", F, C_), (p + "mlp.c_proj.weight", C_, F)]
            if self.moe:  # model/params.go:53-63; packed [E, H, C] / [E, C, H]
                E, EH = self.n_experts, self.expert_hidden
                ents += [(p + "mlp.c_gate.weight", F, C_),
                         (p + "moe.router.weight", E, C_),
                         (p + "moe.router_bias", E, 1),
                         (p + "moe.experts.gate.weight", E * EH, C_),
                         (p + "moe.experts.up.weight", E * EH, C_),
                         (p + "moe.experts.down.weight", E * C_, EH)]
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
    """The benchmark's d2 workload: ConfigForPreset(dense, 2, 32768, 64, 128, 512, "SSSL")."""
    return config_for_depth_ratio(2, 32768, 64, 128, 512, "SSSL", 1)


def dense_d12() -> Config:
    """The benchmark's d12 workload: depth 12, 6 query heads, 2 KV heads, vocab 65536, seq 512."""
    return config_for_depth_ratio(12, 65536, 64, 128, 512, "SSSL", 3)


def dense_d20() -> Config:
    """The benchmark's d20 workload: depth 20, 10 query heads, 2 KV heads, seq 2048."""
    return config_for_depth_ratio(20, 65536, 64, 128, 2048, "SSSL", 5)


def moe_experts_for_depth(depth: int) -> int:
    """model/config.go:609-615: max(2*depth, 8) routed experts."""
    return max(2 * depth, 8)


def apply_latent_preset(cfg: Config, mla_latent: int = 0, n_experts: int = 0,
                        experts_per_token: int = 0, expert_hidden: int = 0,
                        shared_hidden: int = 0, moe_scale: float = 0.0,
                        balance_weight: float = 0.0) -> Config:
    """Config.ApplyPreset(PresetLatent) (model/preset.go:120-152) followed by
    ApplyMoEDefaults (model/config.go:210-227), with the effective clamp,
    scale and balance weight resolved (config.go:152-188).  Fields already
    set by the caller are respected, as the preset does."""
    if cfg.n_kv_head == cfg.n_head and cfg.n_head % 2 == 0:  # applyDefaultGroupedQuery
        cfg.n_kv_head = cfg.n_head // 2
    cfg.mla_latent = mla_latent if mla_latent > 0 else cfg.n_embd // 2
    cfg.head_wise_muon = False
    return enable_moe(cfg, n_experts, experts_per_token, expert_hidden, shared_hidden, moe_scale,
                      balance_weight)


def enable_moe(cfg: Config, n_experts: int = 0, experts_per_token: int = 0,
               expert_hidden: int = 0, shared_hidden: int = 0, moe_scale: float = 0.0,
               balance_weight: float = 0.0, moe_clamp: float = 0.0) -> Config:
    """Config.enableMoE (model/preset.go:142-152) and ApplyMoEDefaults
    (model/config.go:210-227) with the effective clamp, scale and balance
    weight resolved (config.go:152-188): the DeepSeekMoE feed-forward of the
    latent and flash presets.  As the reference: a zero clamp is the default
    10 and a negative one disables clamping (MoEEffectiveClamp and the
    clamp > 0 tests of kernels/scalar/elementwise.go:105-126); a zero scale
    is 1; a zero balance weight is 1e-4 and a negative one disables the
    loss."""
    cfg.n_experts = n_experts if n_experts > 0 else moe_experts_for_depth(cfg.n_layer)
    k = experts_per_token if experts_per_token > 0 else 2
    cfg.experts_per_token = min(k, cfg.n_experts)
    cfg.expert_hidden = expert_hidden if expert_hidden > 0 else cfg.n_embd
    cfg.shared_hidden = shared_hidden if shared_hidden > 0 else cfg.expert_hidden
    cfg.moe_clamp = float(moe_clamp) if moe_clamp != 0 else DEFAULT_MOE_CLAMP
    cfg.moe_scale = float(moe_scale) if moe_scale != 0 else 1.0
    if balance_weight < 0:
        cfg.balance_weight = 0.0
    else:
        cfg.balance_weight = balance_weight if balance_weight > 0 else DEFAULT_MOE_BALANCE_WEIGHT
    cfg.validate()
    return cfg


def apply_flash_preset(cfg: Config, sparse_topk: int = 0, swa_window: int = 0,
                       n_experts: int = 0, experts_per_token: int = 0, expert_hidden: int = 0,
                       shared_hidden: int = 0, balance_weight: float = 0.0) -> Config:
    """Config.ApplyPreset(PresetFlash) (model/preset.go:93-118) with the
    MoE defaults resolved: compression ratio 4, SparseTopK 8, IndexerPool 8,
    ReusePattern "FRU", SWAWindow 128 and CED (with >= 2 layers) unless the
    caller set them, then the DeepSeekMoE feed-forward."""
    if cfg.n_kv_head == cfg.n_head and cfg.n_head % 2 == 0:  # applyDefaultGroupedQuery
        cfg.n_kv_head = cfg.n_head // 2
    if cfg.compression <= 1:
        cfg.compression_ratio = 4
    cfg.sparse_topk = sparse_topk if sparse_topk > 0 else (cfg.sparse_topk or 8)
    if cfg.indexer_pool <= 1:
        cfg.indexer_pool = 8
    if not cfg.reuse_pattern:
        cfg.reuse_pattern = "FRU"
    if swa_window > 0:
        cfg.swa_window = swa_window
    elif cfg.swa_window <= 0:
        cfg.swa_window = 128
    if cfg.n_layer >= 2:
        cfg.ced = True
    cfg.head_wise_muon = True
    return enable_moe(cfg, n_experts, experts_per_token, expert_hidden, shared_hidden, 0.0,
                      balance_weight)


def flash_d12() -> Config:
    """The benchmark's flash d12 workload: flash preset depth 12 (d_model 768, 6 query heads,
    one KV head), compression 4, top-16 sparse selection (pool 8, 128
    candidates, indexer 64 x 1 head), SWA window 512, FRU reuse, CED split at
    layer 6, DeepSeekMoE 1 shared + 16 routed experts of hidden 768, top-2;
    SequenceLen 16384 so 8192-token prompts + 512 new tokens fit."""
    cfg = config_for_depth_ratio(12, 65536, 64, 128, 16384, "SSSL", 1)
    cfg.n_kv_head = 1
    return apply_flash_preset(cfg, sparse_topk=16, swa_window=512, n_experts=16)


def latent_d12() -> Config:
    """The benchmark's latent d12 workload: latent preset depth 12 (d_model 768, 6 query heads,
    3 KV heads by the preset's grouped-query default), absorbed MLA with
    latent 256 (one MLALatent serves both the query and the KV latent, so
    the benchmark's separate q latent of 384 cannot be expressed), rope 64,
    DeepSeekMoE 1 shared + 16 routed experts of hidden 512, top-2."""
    cfg = config_for_depth_ratio(12, 65536, 64, 128, 512, "SSSL", 1)
    return apply_latent_preset(cfg, mla_latent=256, n_experts=16, experts_per_token=2,
                               expert_hidden=512)


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
        if cfg.mla:
            keys = ("attn.mla_q_down.weight", "attn.mla_q_up.weight", "attn.mla_q_rope.weight",
                    "attn.mla_kv_down.weight", "attn.mla_k_up.weight", "attn.mla_v_up.weight",
                    "attn.mla_k_rope.weight")
        else:
            keys = ("attn.c_q.weight", "attn.c_k.weight", "attn.c_v.weight")
        for k in keys:
            put(p + k, rng.uniform(-bound, bound, n(p + k)))
        put(p + "mlp.c_fc.weight", rng.uniform(-0.4 * bound, 0.4 * bound, n(p + "mlp.c_fc.weight")))
        if cfg.compression > 1 and cfg.reuse_mode_at(l) == "F":  # transformer.go:196-199
            k = p + "attn.compress_logits.weight"
            put(k, rng.uniform(-bound, bound, n(k)))
        if cfg.compression > 1 and cfg.sparse_topk > 0 and cfg.reuse_mode_at(l) != "U":
            for k in ("attn.indexer_query.weight", "attn.indexer_key.weight"):  # :200-204
                put(p + k, rng.uniform(-bound, bound, n(p + k)))
            put(p + "attn.indexer_heads", np.ones(n(p + "attn.indexer_heads")))
        if cfg.moe:  # transformer.go:163-174
            put(p + "mlp.c_gate.weight",
                rng.uniform(-0.4 * bound, 0.4 * bound, n(p + "mlp.c_gate.weight")))
            for k in ("moe.experts.gate.weight", "moe.experts.up.weight"):
                put(p + k, rng.uniform(-0.4 * bound, 0.4 * bound, n(p + k)))
            put(p + "moe.router.weight", rng.standard_normal(n(p + "moe.router.weight")) * 0.02)
        # c_proj, expert down weights and the router bias stay zero
        # (transformer.go:162,167,172-173)
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

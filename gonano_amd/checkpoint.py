"""The `.gn` checkpoint format (model/checkpoint/checkpoint.go) on the host:
the file either side of the RL step, so a session can start from a trained
gonano model and hand its parameters back.

Layout (checkpoint.go:36-82): the 8-byte magic ``GONANO\\x00\\x01``, a
little-endian uint32 length, that many bytes of JSON metadata (``step``,
``model_config`` with model.Config's JSON names, ``params``: name and
shape of every tensor in sorted-name order, optional ``val_bpb`` /
``user_config`` / ``loop_state`` / ``dataloader_state``), then every
tensor's float32 values little-endian in the same order.  Sorted-name
order is also the session's flat parameter order (model/params.go:77-113),
so a model's flat vector is the payload itself once the names match.
"""
from __future__ import annotations

import json
import os
import re

import numpy as np

from . import config as G
from .config import Config

MAGIC = b"GONANO\x00\x01"  # checkpoint.go:20


class CheckpointError(ValueError):
    pass


def save(path: str, meta: dict, params: dict[str, np.ndarray]) -> None:
    """checkpoint.Save (checkpoint.go:36-82): params sorted by name, their
    names and shapes written into meta["params"]."""
    names = sorted(params)
    meta = dict(meta)
    meta["params"] = [{"name": n, "shape": list(np.shape(params[n]))} for n in names]
    blob = json.dumps(meta, separators=(",", ":")).encode()
    with open(path, "wb") as f:
        f.write(MAGIC)
        f.write(len(blob).to_bytes(4, "little"))
        f.write(blob)
        for n in names:
            f.write(np.ascontiguousarray(params[n], "<f4").tobytes())


def load(path: str) -> tuple[dict, dict[str, np.ndarray]]:
    """checkpoint.Load (checkpoint.go:84-121), with its three errors:
    invalid magic, truncated metadata, truncated params."""
    with open(path, "rb") as f:
        data = f.read()
    if len(data) < len(MAGIC) + 4 or data[:len(MAGIC)] != MAGIC:
        raise CheckpointError(f"checkpoint: invalid magic in {path}")
    pos = len(MAGIC)
    n = int.from_bytes(data[pos:pos + 4], "little")
    pos += 4
    if pos + n > len(data):
        raise CheckpointError(f"checkpoint: truncated metadata in {path}")
    meta = json.loads(data[pos:pos + n])
    pos += n
    params = {}
    for pm in meta.get("params", []):
        shape = tuple(int(d) for d in pm["shape"])
        count = int(np.prod(shape, dtype=np.int64)) if shape else 1
        need = 4 * count
        if pos + need > len(data):
            raise CheckpointError(f"checkpoint: truncated params in {path}")
        params[pm["name"]] = np.frombuffer(data, "<f4", count, pos).astype(np.float32).reshape(shape)
        pos += need
    return meta, params


# model.Config's JSON names (model/config.go:10-123)
MODEL_CONFIG_KEYS = frozenset((
    "sequence_len", "vocab_size", "n_layer", "n_head", "n_kv_head", "n_embd", "window_pattern",
    "rotary_dims", "compression_ratio", "sparse_top_k", "indexer_dim", "indexer_heads",
    "indexer_loss_weight", "indexer_pool", "indexer_candidates", "reuse_pattern", "swa_window",
    "ced", "head_wise_muon", "query_compression_dim", "kv_latent_dim", "mla_latent",
    "mla_rotary_dims", "num_experts", "num_experts_per_token", "expert_hidden_dim",
    "shared_expert_hidden_dim", "moe_clamp", "moe_scale", "router_bias_update",
    "moe_balance_weight"))
# fields of model.Config this backend does not build (the low-rank query
# and KV-latent projections of config.go:68-79): a checkpoint that sets them
# is refused rather than loaded as a different model
UNSUPPORTED_KEYS = ("query_compression_dim", "kv_latent_dim")


def config_from_meta(meta: dict) -> Config:
    """The resolved host Config of meta["model_config"] (model.Config JSON
    names, model/config.go:10-123), with the preset defaults that
    NewTransformer resolves (MoE, indexer) filled in.  Keys model.Config
    does not have, and the fields this backend does not build, raise
    CheckpointError."""
    mc = meta["model_config"]
    unknown = sorted(set(mc) - MODEL_CONFIG_KEYS)
    if unknown:
        raise CheckpointError(f"checkpoint: unknown model_config keys {unknown}")
    for k in UNSUPPORTED_KEYS:
        if mc.get(k, 0):
            raise CheckpointError(f"checkpoint: model_config {k} is not supported by this backend")
    cfg = Config(sequence_len=mc["sequence_len"], vocab_size=mc["vocab_size"],
                 n_layer=mc["n_layer"], n_head=mc["n_head"], n_kv_head=mc["n_kv_head"],
                 n_embd=mc["n_embd"], window_pattern=mc.get("window_pattern", "L"),
                 rotary_dims=mc.get("rotary_dims", 0), mla_latent=mc.get("mla_latent", 0),
                 mla_rope_dims=mc.get("mla_rotary_dims", 0),
                 compression_ratio=mc.get("compression_ratio", 0),
                 swa_window=mc.get("swa_window", 0), sparse_topk=mc.get("sparse_top_k", 0),
                 indexer_dim=mc.get("indexer_dim", 0), indexer_heads=mc.get("indexer_heads", 0),
                 indexer_pool=mc.get("indexer_pool", 0),
                 indexer_candidates=mc.get("indexer_candidates", 0),
                 indexer_weight=mc.get("indexer_loss_weight", 0.0),
                 reuse_pattern=mc.get("reuse_pattern", ""), ced=bool(mc.get("ced", False)),
                 head_wise_muon=bool(mc.get("head_wise_muon", False)),
                 router_bias_update=float(mc.get("router_bias_update", 0.0)))
    if mc.get("num_experts", 0) > 0:
        G.enable_moe(cfg, mc["num_experts"], mc.get("num_experts_per_token", 0),
                     mc.get("expert_hidden_dim", 0), mc.get("shared_expert_hidden_dim", 0),
                     mc.get("moe_scale", 0.0), mc.get("moe_balance_weight", 0.0),
                     mc.get("moe_clamp", 0.0))
    cfg.validate()
    return cfg


def meta_for(cfg: Config, step: int = 0, **extra) -> dict:
    """Metadata whose model_config reproduces cfg as model.Config JSON
    (omitempty): resolved values are written explicitly, which model.Config
    keeps as they are, except where zero would read back as a default -- a
    disabled balance loss is written as -1 (MoEBalanceLossWeight: negative
    disables it)."""
    mc = {"sequence_len": cfg.sequence_len, "vocab_size": cfg.vocab_size,
          "n_layer": cfg.n_layer, "n_head": cfg.n_head, "n_kv_head": cfg.n_kv_head,
          "n_embd": cfg.n_embd, "window_pattern": cfg.window_pattern}
    opt = {"rotary_dims": cfg.rotary_dims, "mla_latent": cfg.mla_latent,
           "mla_rotary_dims": cfg.mla_rope_dims, "compression_ratio": cfg.compression_ratio,
           "swa_window": cfg.swa_window, "sparse_top_k": cfg.sparse_topk,
           "indexer_dim": cfg.indexer_dim, "indexer_heads": cfg.indexer_heads,
           "indexer_pool": cfg.indexer_pool, "indexer_candidates": cfg.indexer_candidates,
           "indexer_loss_weight": cfg.indexer_weight, "reuse_pattern": cfg.reuse_pattern,
           "ced": cfg.ced, "head_wise_muon": cfg.head_wise_muon,
           "router_bias_update": cfg.router_bias_update}
    if cfg.moe:
        opt.update({"num_experts": cfg.n_experts, "num_experts_per_token": cfg.experts_per_token,
                    "expert_hidden_dim": cfg.expert_hidden,
                    "shared_expert_hidden_dim": cfg.shared_hidden, "moe_clamp": cfg.moe_clamp,
                    "moe_scale": cfg.moe_scale,
                    "moe_balance_weight": cfg.balance_weight if cfg.balance_weight > 0 else -1.0})
    mc.update({k: v for k, v in opt.items() if v})  # omitempty
    meta = {"step": step, "model_config": mc}
    meta.update(extra)
    return meta


def flat_from_params(cfg: Config, params: dict[str, np.ndarray], base: np.ndarray | None = None,
                     strict: bool = False) -> np.ndarray:
    """LoadModel (checkpoint.go:146-155) into the session's flat vector: the
    model's own initial weights (`base`, default init_weights(cfg)), then
    every tensor of the file whose name the model has copied over it with Go's
    copy (the shorter length wins); names the model lacks are ignored and
    parameters the file lacks keep their initial values.  strict=True
    instead requires every parameter with its exact size (CheckpointError
    otherwise), for callers that want a file of another architecture
    refused rather than partly loaded."""
    table = cfg.param_table()
    if strict:
        for name, rows, cols, _ in table:
            if name not in params:
                raise CheckpointError(f"checkpoint: missing parameter {name}")
            n = np.asarray(params[name]).size
            if n != rows * cols:
                raise CheckpointError(f"checkpoint: {name} has {n} values, want {rows}x{cols}")
    out = np.array(G.init_weights(cfg) if base is None else base, np.float32, copy=True)
    if out.size != cfg.param_total():
        raise CheckpointError("checkpoint: base weights do not match the config")
    for name, rows, cols, off in table:
        if name in params:
            a = np.asarray(params[name], np.float32).ravel()
            n = min(a.size, rows * cols)
            out[off:off + n] = a[:n]
    return out


def params_from_flat(cfg: Config, flat: np.ndarray) -> dict[str, np.ndarray]:
    return {name: flat[off:off + r * c].reshape(_shape(r, c))
            for name, r, c, off in cfg.param_table()}


def _shape(rows: int, cols: int) -> tuple[int, ...]:
    # vectors and scalars are [n] tensors in the reference (model/params.go)
    return (rows,) if cols == 1 else (rows, cols)


def find_last_step(directory: str) -> int:
    """FindLastStep (checkpoint.go:144-172)."""
    pat = re.compile(r"model_(\d+)\.gn$")
    steps = [int(m.group(1)) for e in os.listdir(directory) if (m := pat.search(e))]
    if not steps:
        raise CheckpointError(f"checkpoint: no checkpoints in {directory}")
    return max(steps)


def model_path(directory: str, step: int) -> str:
    """ModelPath (checkpoint.go:178-181)."""
    return os.path.join(directory, f"model_{step:06d}.gn")

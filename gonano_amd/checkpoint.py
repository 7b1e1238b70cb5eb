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


def config_from_meta(meta: dict) -> Config:
    """The resolved host Config of meta["model_config"] (model.Config JSON
    names, model/config.go:10-123), with the preset defaults that
    NewTransformer resolves (MoE, indexer) filled in."""
    mc = meta["model_config"]
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
                 head_wise_muon=bool(mc.get("head_wise_muon", False)))
    if mc.get("num_experts", 0) > 0:
        G.enable_moe(cfg, mc["num_experts"], mc.get("num_experts_per_token", 0),
                     mc.get("expert_hidden_dim", 0), mc.get("shared_expert_hidden_dim", 0),
                     mc.get("moe_scale", 0.0), mc.get("moe_balance_weight", 0.0))
        if mc.get("moe_clamp", 0.0) > 0:
            cfg.moe_clamp = float(mc["moe_clamp"])
    cfg.validate()
    return cfg


def meta_for(cfg: Config, step: int = 0, **extra) -> dict:
    """Metadata whose model_config reproduces cfg (resolved values written
    explicitly; model.Config keeps explicit values as they are)."""
    mc = {"sequence_len": cfg.sequence_len, "vocab_size": cfg.vocab_size,
          "n_layer": cfg.n_layer, "n_head": cfg.n_head, "n_kv_head": cfg.n_kv_head,
          "n_embd": cfg.n_embd, "window_pattern": cfg.window_pattern}
    opt = {"rotary_dims": cfg.rotary_dims, "mla_latent": cfg.mla_latent,
           "mla_rotary_dims": cfg.mla_rope_dims, "compression_ratio": cfg.compression_ratio,
           "swa_window": cfg.swa_window, "sparse_top_k": cfg.sparse_topk,
           "indexer_dim": cfg.indexer_dim, "indexer_heads": cfg.indexer_heads,
           "indexer_pool": cfg.indexer_pool, "indexer_candidates": cfg.indexer_candidates,
           "indexer_loss_weight": cfg.indexer_weight, "reuse_pattern": cfg.reuse_pattern,
           "ced": cfg.ced, "head_wise_muon": cfg.head_wise_muon}
    if cfg.moe:
        opt.update({"num_experts": cfg.n_experts, "num_experts_per_token": cfg.experts_per_token,
                    "expert_hidden_dim": cfg.expert_hidden,
                    "shared_expert_hidden_dim": cfg.shared_hidden, "moe_clamp": cfg.moe_clamp,
                    "moe_scale": cfg.moe_scale, "moe_balance_weight": cfg.balance_weight})
    mc.update({k: v for k, v in opt.items() if v})  # omitempty
    meta = {"step": step, "model_config": mc}
    meta.update(extra)
    return meta


def flat_from_params(cfg: Config, params: dict[str, np.ndarray]) -> np.ndarray:
    """LoadModel (checkpoint.go:130-141) into the session's flat vector:
    every parameter of cfg must be present with its shape (a file from a
    different architecture is rejected rather than partly copied)."""
    out = np.empty(cfg.param_total(), np.float32)
    for name, rows, cols, off in cfg.param_table():
        if name not in params:
            raise CheckpointError(f"checkpoint: missing parameter {name}")
        a = np.asarray(params[name], np.float32)
        if a.size != rows * cols:
            raise CheckpointError(f"checkpoint: {name} has {a.size} values, want {rows}x{cols}")
        out[off:off + rows * cols] = a.ravel()
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

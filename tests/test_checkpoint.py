"""The `.gn` checkpoint reader/writer (gonano_amd/checkpoint.py) against the
format checkpoint.go fixes: a file assembled byte by byte from the layout
(magic, little-endian length, JSON, little-endian float32 payload in
sorted-name order) loads to its values; Save writes exactly that layout;
round trips for the dense, latent and flash parameter tables; and the
reference's rejections (model/checkpoint/checkpoint_test.go:12-232:
roundtrip, LoadModel, FindLastStep, non-checkpoint files)."""
import json
import os
import struct

import numpy as np
import pytest

from gonano_amd import checkpoint as CK
from gonano_amd import config as G


def test_load_hand_assembled_file(tmp_path):
    meta = {"step": 7, "model_config": {"sequence_len": 64, "vocab_size": 10, "n_layer": 1,
                                        "n_head": 1, "n_kv_head": 1, "n_embd": 4,
                                        "window_pattern": "L"},
            "params": [{"name": "a", "shape": [2, 3]}, {"name": "b", "shape": [2]}]}
    blob = json.dumps(meta).encode()
    vals = [1.5, -2.0, 3.25, 0.0, 1e-3, -7.0, 42.0, -0.5]
    raw = b"GONANO\x00\x01" + struct.pack("<I", len(blob)) + blob + struct.pack("<8f", *vals)
    path = tmp_path / "x.gn"
    path.write_bytes(raw)
    m, p = CK.load(str(path))
    assert m["step"] == 7 and list(p) == ["a", "b"]
    np.testing.assert_array_equal(p["a"], np.array(vals[:6], np.float32).reshape(2, 3))
    np.testing.assert_array_equal(p["b"], np.array(vals[6:], np.float32))


def test_save_writes_the_layout(tmp_path):
    params = {"z": np.array([1, 2], np.float32), "a": np.array([[3, 4, 5]], np.float32)}
    path = tmp_path / "y.gn"
    CK.save(str(path), {"step": 3}, params)
    raw = path.read_bytes()
    assert raw[:8] == b"GONANO\x00\x01"
    n = struct.unpack("<I", raw[8:12])[0]
    meta = json.loads(raw[12:12 + n])
    assert meta["step"] == 3
    assert meta["params"] == [{"name": "a", "shape": [1, 3]}, {"name": "z", "shape": [2]}]
    assert struct.unpack("<5f", raw[12 + n:]) == (3, 4, 5, 1, 2)


@pytest.mark.parametrize("factory", ["dense_d2", "latent_d12", "flash_d12"])
def test_roundtrip_model(tmp_path, factory):  # checkpoint_test.go:12-57, 90-130, 197-232
    cfg = getattr(G, factory)()
    if factory != "dense_d2":  # keep the file small: fewer layers, smaller vocab
        cfg.n_layer, cfg.vocab_size = 2, 512
        cfg.validate()
    w = G.init_weights(cfg, seed=1, perturb=0.1)
    path = CK.model_path(str(tmp_path), 12)
    CK.save(path, CK.meta_for(cfg, step=12, val_bpb=1.25), CK.params_from_flat(cfg, w))
    meta, params = CK.load(path)
    assert meta["step"] == 12 and meta["val_bpb"] == 1.25
    cfg2 = CK.config_from_meta(meta)
    assert cfg2 == cfg  # the whole resolved Config, not only its parameter table
    np.testing.assert_array_equal(CK.flat_from_params(cfg2, params), w)


@pytest.mark.parametrize("clamp,balance,scale,bias", [(-1.0, -1.0, 0.5, 0.002), (0.0, 0.0, 0.0, 0.0),
                                                      (7.5, 3e-4, -2.0, 0.0)])
def test_moe_config_semantics_roundtrip(tmp_path, clamp, balance, scale, bias):
    """model.Config's MoE fields keep their meaning through a file
    (model/config.go:104-123, 152-188): a negative clamp disables clamping, a
    negative balance weight disables the loss (written back as -1, not left
    out, which would read as the 1e-4 default), zeros take the defaults, a
    negative scale is kept, and router_bias_update survives."""
    meta = {"step": 0, "model_config": {
        "sequence_len": 64, "vocab_size": 256, "n_layer": 2, "n_head": 2, "n_kv_head": 1,
        "n_embd": 128, "window_pattern": "L", "num_experts": 4, "num_experts_per_token": 2,
        "moe_clamp": clamp, "moe_balance_weight": balance, "moe_scale": scale,
        "router_bias_update": bias}}
    cfg = CK.config_from_meta(meta)
    assert cfg.moe_clamp == (clamp if clamp != 0 else 10.0)
    assert cfg.balance_weight == (0.0 if balance < 0 else balance if balance > 0 else 1e-4)
    assert cfg.moe_scale == (scale if scale != 0 else 1.0)
    assert cfg.router_bias_update == bias
    path = str(tmp_path / "moe.gn")
    CK.save(path, CK.meta_for(cfg), CK.params_from_flat(cfg, G.init_weights(cfg, seed=2)))
    meta2, _ = CK.load(path)
    assert CK.config_from_meta(meta2) == cfg
    if balance < 0:
        assert meta2["model_config"]["moe_balance_weight"] < 0


def test_model_config_rejections():
    base = {"sequence_len": 64, "vocab_size": 256, "n_layer": 1, "n_head": 1, "n_kv_head": 1,
            "n_embd": 128}
    with pytest.raises(CK.CheckpointError, match="unknown model_config keys"):
        CK.config_from_meta({"model_config": dict(base, n_embdd=3)})
    for key in ("query_compression_dim", "kv_latent_dim"):
        with pytest.raises(CK.CheckpointError, match="not supported"):
            CK.config_from_meta({"model_config": dict(base, **{key: 32})})
    assert CK.config_from_meta({"model_config": dict(base, kv_latent_dim=0)}).n_embd == 128


def test_load_rejects_non_checkpoint(tmp_path):  # checkpoint_test.go:185-195
    bad = tmp_path / "not.gn"
    bad.write_bytes(b"hello world, not a checkpoint")
    with pytest.raises(CK.CheckpointError, match="invalid magic"):
        CK.load(str(bad))
    blob = json.dumps({"params": [{"name": "a", "shape": [4]}]}).encode()
    (tmp_path / "m.gn").write_bytes(b"GONANO\x00\x01" + struct.pack("<I", len(blob) + 9) + blob)
    with pytest.raises(CK.CheckpointError, match="truncated metadata"):
        CK.load(str(tmp_path / "m.gn"))
    (tmp_path / "p.gn").write_bytes(b"GONANO\x00\x01" + struct.pack("<I", len(blob)) + blob +
                                    struct.pack("<3f", 1, 2, 3))
    with pytest.raises(CK.CheckpointError, match="truncated params"):
        CK.load(str(tmp_path / "p.gn"))


def test_flat_follows_load_model():
    """LoadModel (checkpoint.go:146-155): the model's initial weights, then
    each tensor the file has copied over with Go's copy (the shorter length
    wins); names the model lacks are ignored, missing parameters keep their
    initial values.  strict=True refuses such a file instead."""
    cfg = G.dense_d2()
    w = G.init_weights(cfg, seed=0, perturb=0.1)
    base = G.init_weights(cfg, seed=9)
    params = CK.params_from_flat(cfg, w)
    del params["lm_head.weight"]
    params["not.a.parameter"] = np.ones(3, np.float32)
    params["resid_lambdas"] = np.array([5.0], np.float32)  # shorter than the model's
    got = CK.flat_from_params(cfg, params, base=base)
    sl = cfg.param_slices()
    for name, r, c, off in cfg.param_table():
        seg = got[off:off + r * c]
        if name == "lm_head.weight":
            np.testing.assert_array_equal(seg, base[off:off + r * c])
        elif name == "resid_lambdas":
            assert seg[0] == 5.0
            np.testing.assert_array_equal(seg[1:], base[off + 1:off + r * c])
        else:
            np.testing.assert_array_equal(seg, w[off:off + r * c])
    assert sl["lm_head.weight"][0] >= 0
    with pytest.raises(CK.CheckpointError, match="missing parameter"):
        CK.flat_from_params(cfg, params, strict=True)
    params["lm_head.weight"] = w[:10]
    with pytest.raises(CK.CheckpointError, match="values, want"):
        CK.flat_from_params(cfg, params, strict=True)


def test_find_last_step(tmp_path):  # checkpoint_test.go:169-183
    for s in (5, 120, 17):
        open(CK.model_path(str(tmp_path), s), "wb").close()
    (tmp_path / "model_999.txt").write_text("x")
    assert CK.find_last_step(str(tmp_path)) == 120
    assert os.path.basename(CK.model_path(str(tmp_path), 120)) == "model_000120.gn"
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(CK.CheckpointError, match="no checkpoints"):
        CK.find_last_step(str(empty))

"""A `.gn` checkpoint (model/checkpoint/checkpoint.go:36-155) into a device
session: the file's model_config resolves to the session's config, its
tensors (LoadModel) become the session's parameters, and the session's
forward logits and policy-gradient gradients equal the oracle's on the
weights that were saved; the session's parameters written back through a
file reload bit for bit."""
import numpy as np
import pytest

from conftest import assert_close, rel_err
from gonano_amd import checkpoint as CK
from gonano_amd import config as G

pytestmark = pytest.mark.gpu


def _configs():
    dense = G.Config(sequence_len=512, vocab_size=2048, n_layer=2, n_head=2, n_kv_head=1,
                     n_embd=256, window_pattern="SSSL", rotary_dims=64)
    latent = G.config_for_depth_ratio(4, 2048, 64, 128, 512, "SSSL", 1)
    latent.n_layer = 2
    G.apply_latent_preset(latent, mla_latent=128, n_experts=4, experts_per_token=2,
                          expert_hidden=256)
    return [("dense", dense, 0.1), ("latent", latent, 0.05)]


@pytest.mark.parametrize("name,cfg,perturb", _configs(), ids=["dense", "latent"])
def test_checkpoint_into_session_matches_oracle(tmp_path, orc, name, cfg, perturb):
    from gonano_amd.session import Session
    w = G.init_weights(cfg, seed=17, perturb=perturb)
    path = CK.model_path(str(tmp_path), 42)
    CK.save(path, CK.meta_for(cfg, step=42), CK.params_from_flat(cfg, w))
    meta, params = CK.load(path)
    assert meta["step"] == 42 and CK.find_last_step(str(tmp_path)) == 42
    cfg2 = CK.config_from_meta(meta)
    assert cfg2 == cfg
    flat = CK.flat_from_params(cfg2, params, strict=True)
    rng = np.random.default_rng(3)
    ids = rng.integers(0, cfg.vocab_size, (2, 96)).astype(np.int32)
    targets = rng.integers(0, cfg.vocab_size, (2, 96)).astype(np.int32)
    targets[:, :30] = -1
    adv = np.array([0.4, -0.4], np.float32)
    with Session(cfg2) as s:
        s.set_params(flat)
        logits = s.forward(ids)
        s.zero_grad()
        loss, nll = s.policy_gradient_step(ids, targets, adv, 97.0)
        grads = s.grads()
        back = s.get_params()
    m = orc.OracleModel(orc.ModelShape.from_config(cfg), w)
    want = m.forward(ids)
    assert rel_err(logits, want) < 1e-4
    assert_close(logits, want, 1e-3, 1e-4, "logits")
    wl, wnll, wg = m.pg_step(ids, targets, adv, 97.0)
    assert abs(loss - wl) <= 1e-4 * max(abs(wl), 1e-3)
    assert rel_err(grads, wg) < 1e-4
    # the device parameters, saved again, reload unchanged
    path2 = CK.model_path(str(tmp_path), 43)
    CK.save(path2, CK.meta_for(cfg2, step=43), CK.params_from_flat(cfg2, back))
    _, params2 = CK.load(path2)
    assert np.array_equal(CK.flat_from_params(cfg2, params2, strict=True), w)

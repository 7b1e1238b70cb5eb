"""The policy-gradient step in micro-batches of sequences (the path a batch
takes when its saved activations exceed the device budget) equals the
oracle's single PolicyGradientStep (trainer/rl.go:14-60) over the whole
batch: the loss, NLL and gradients are sums over sequences, and the MoE
balance loss (model/moe.go:290-313) averages over every sequence of the
batch, not of the micro-batch.  GN_PG_MICRO_BATCH caps the micro-batch
size; 1 and 2 split a batch of 3 into three and two passes."""
import os

import numpy as np
import pytest

from conftest import rel_err
from gonano_amd import config as G
from test_gpu_csa import csa_cfg
from test_gpu_latent import latent_small_cfg
from test_gpu_session import _compare_grads, small_cfg

pytestmark = pytest.mark.gpu

CFGS = {
    "dense": (small_cfg, 0.1),
    "latent_moe": (latent_small_cfg, 0.05),
    "flash_hier_fru": (lambda: csa_cfg("hier_fru"), 0.1),
}


@pytest.mark.parametrize("name", list(CFGS))
def test_micro_batched_pg_step_matches_oracle(name, orc):
    from gonano_amd.session import Session
    make, perturb = CFGS[name]
    cfg = make()
    w = G.init_weights(cfg, seed=31, perturb=perturb)
    rng = np.random.default_rng(32)
    B, T = 3, 97
    inputs = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets[:, :20] = -1
    targets[2, 80:] = -1
    adv = np.array([0.75, -0.5, -0.25], np.float32)
    wl, wnll, wg = orc.OracleModel(orc.ModelShape.from_config(cfg), w).pg_step(
        inputs, targets, adv, float(T + 1))
    old = os.environ.get("GN_PG_MICRO_BATCH")
    try:
        with Session(cfg) as s:
            s.set_params(w)
            s.zero_grad()
            whole = s.policy_gradient_step(inputs, targets, adv, float(T + 1))
            aux_whole = s.aux_loss()
            for mb in (1, 2):
                os.environ["GN_PG_MICRO_BATCH"] = str(mb)
                s.zero_grad()
                loss, nll = s.policy_gradient_step(inputs, targets, adv, float(T + 1))
                grads = s.grads()
                assert abs(loss - wl) <= 1e-4 * max(abs(wl), 1e-3), (mb, loss, wl)
                assert abs(loss - whole[0]) <= 1e-5 * max(abs(wl), 1e-3), mb
                assert rel_err(nll, wnll) < 1e-4
                assert rel_err(nll, whole[1]) < 1e-6, mb
                _compare_grads(cfg, grads, wg)
                if cfg.moe:
                    assert aux_whole > 0
                    assert abs(s.aux_loss() - aux_whole) <= 1e-6 * aux_whole, mb
                del os.environ["GN_PG_MICRO_BATCH"]
    finally:
        if old is None:
            os.environ.pop("GN_PG_MICRO_BATCH", None)
        else:
            os.environ["GN_PG_MICRO_BATCH"] = old

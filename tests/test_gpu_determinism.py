"""Run-to-run determinism on the device: the same work in two fresh sessions
gives bitwise-equal results, and a rollout replayed from the captured
decode graph equals the one launched kernel by kernel.

Every product runs on hand-written kernels whose sums have a fixed order
(split-K partials added in float64 in split order, no atomics), the MoE
routing places tokens by counting, and the decode attention, sampler and
norms reduce in a fixed order, so nothing in these paths depends on timing.
(The one exception in the library is the sparse compressed-attention
backward, whose compressed K/V gradients are scattered with float atomics;
it is not exercised here.)
"""
import dataclasses

import numpy as np
import pytest

from gonano_amd import config as G

pytestmark = pytest.mark.gpu


def _dense_v65536():
    # the d12 width at the benchmark's vocabulary, two layers
    return dataclasses.replace(G.dense_d12(), n_layer=2, vocab_size=65536)


def _latent():
    cfg = G.config_for_depth_ratio(12, 4096, 64, 128, 512, "SSSL", 1)
    cfg.n_layer = 2
    return G.apply_latent_preset(cfg, mla_latent=256, n_experts=16, experts_per_token=2,
                                 expert_hidden=512)


def _pg(cfg, w, B, T, prompt_len, seed=3):
    from gonano_amd.session import Session
    rng = np.random.default_rng(seed)
    inputs = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets[:, :prompt_len] = -1
    adv = np.linspace(-0.5, 0.5, B).astype(np.float32)
    with Session(cfg) as s:
        s.set_params(w)
        s.zero_grad()
        loss, nll = s.policy_gradient_step(inputs, targets, adv, float(T + 1))
        return loss, nll, s.grads(), s.aux_loss()


@pytest.mark.parametrize("wide", [False, True], ids=["default", "wide_engine_everywhere"])
def test_pg_step_bitwise_repeatable_dense(monkeypatch, wide):
    """The policy-gradient step (4 x 512 tokens, V = 65,536) in two fresh
    sessions: loss, NLL and every gradient bitwise equal, with the default
    engine choice and with every product the wide-tile engine can take sent
    there (GN_GEMM_WIDE_MIN=1: its split-K weight gradients included)."""
    if wide:
        monkeypatch.setenv("GN_GEMM_WIDE_MIN", "1")
    cfg = _dense_v65536()
    w = G.init_weights(cfg, seed=5, perturb=0.1)
    a = _pg(cfg, w, 4, 512, 384)
    b = _pg(cfg, w, 4, 512, 384)
    assert a[0] == b[0]
    assert np.array_equal(a[1], b[1])
    assert np.array_equal(a[2], b[2])


def test_pg_step_bitwise_repeatable_latent_moe():
    """The same for MLA + DeepSeekMoE (16 experts, top-2): routing, the
    expert-grouped products and the balance loss repeat bit for bit."""
    cfg = _latent()
    w = G.init_weights(cfg, seed=6, perturb=0.02)
    a = _pg(cfg, w, 4, 256, 128)
    b = _pg(cfg, w, 4, 256, 128)
    assert a[0] == b[0] and a[3] == b[3]
    assert np.array_equal(a[1], b[1])
    assert np.array_equal(a[2], b[2])


def test_rollout_graph_equals_eager_and_repeats():
    """256 rows (16 prompts x 16 samples) at V = 65,536, so the rollout's
    lm_head runs on the wide-tile engine and the MLP products on the
    slim-tile engine: the graph-replayed rollout equals the eagerly
    launched one token for token, and a second session repeats it."""
    from gonano_amd.session import Session
    cfg = _dense_v65536()
    w = G.init_weights(cfg, seed=7, perturb=0.1)
    prompts = np.random.default_rng(8).integers(0, cfg.vocab_size, (16, 96)).astype(np.int32)
    seeds = np.arange(16, dtype=np.uint64) + 40
    out = []
    for graph in (True, False, True):
        with Session(cfg) as s:
            s.set_params(w)
            s.set_decode_graph(graph)
            rows = s.generate_batch(prompts, 16, 8, 1.0, 50, seeds)
        out.append([np.asarray(r) for r in rows])
    for other in out[1:]:
        assert len(other) == len(out[0])
        for x, y in zip(out[0], other):
            assert np.array_equal(x, y)

"""Parity of the flash preset's sparse compressed attention on the GPU with the
oracle on identical inputs: Transformer.Forward logits and
PolicyGradientStep's loss, NLL and every parameter gradient -- the
indexer's (trained by its distillation alone), the compressor's, and the
shared projections' -- for the lightning-indexer selection (flat and
hierarchical), Full / Reindex / Reuse cross-layer reuse (dense and sparse)
and the causal encoder-decoder split (model/indexer.go,
model/compress_attention.go, model/share.go, model/transformer.go:363-449).

Floating-point bars as the dense tests: 1e-4 normwise relative per tensor
plus kerneltest.Close(1e-3, 1e-4) element-wise.  The selection is integer
work decided by float scores; on these seeded inputs the GPU's selection
agrees with the oracle's (a near-tie flip would show as an outlier far
beyond the float tolerance).

The CED case perturbs InitWeights by N(0, 0.05) (the others by 0.1): the
decoder's compressor reads the unnormalized encoder hidden state, and at 0.1
the oracle's own float32 build is already 1.4e-4 normwise from its float64
build on this step's gradient (fwd 1.2e-5); at 0.05 that is 3.2e-5."""
import numpy as np
import pytest

from conftest import assert_close, rel_err
from gonano_amd import config as G
from test_gpu_session import _compare_grads
from tf_check import teacher_forced_group

pytestmark = pytest.mark.gpu

CASES = {
    # flat top-4 with a two-head indexer
    "flat": dict(sparse_topk=4, indexer_dim=32, indexer_heads=2),
    # hierarchical (groups of 2, 8 candidates) with Full / Reindex / Reuse
    "hier_fru": dict(sparse_topk=3, indexer_pool=2, indexer_candidates=8, indexer_dim=16,
                     reuse_pattern="FRU"),
    # dense compressed attention with reuse
    "dense_fu": dict(reuse_pattern="FU"),
    # CED (layers 0-1 encoder, 2-3 decoder) with per-half reuse and selection
    "ced": dict(sparse_topk=3, indexer_pool=2, indexer_candidates=6, indexer_dim=16,
                reuse_pattern="FR", ced=True, n_layer=4),
}


def csa_cfg(case):
    kw = dict(CASES[case])
    n_layer = kw.pop("n_layer", 3)
    cfg = G.Config(sequence_len=512, vocab_size=4096, n_layer=n_layer, n_head=2, n_kv_head=1,
                   n_embd=256, window_pattern="SSSL", rotary_dims=64, compression_ratio=4,
                   swa_window=64, **kw)
    cfg.validate()
    return cfg


def oracle(orc, cfg, w):
    return orc.OracleModel(orc.ModelShape.from_config(cfg), w)


@pytest.fixture(scope="module", params=list(CASES))
def csa(request):
    from gonano_amd.session import Session
    cfg = csa_cfg(request.param)
    w = G.init_weights(cfg, seed=41, perturb=0.05 if cfg.ced else 0.1)
    s = Session(cfg)
    s.set_params(w)
    yield request.param, cfg, w, s
    s.close()


def test_csa_param_roundtrip(csa):
    _, cfg, w, s = csa
    assert s.param_total == cfg.param_total()
    assert [(n, r, c, o) for n, r, c, o in s.param_table()] == cfg.param_table()
    assert np.array_equal(s.get_params(), w)


def test_csa_forward_matches_oracle(csa, orc):
    _, cfg, w, s = csa
    ids = np.random.default_rng(1).integers(0, cfg.vocab_size, (2, 203)).astype(np.int32)
    got = s.forward(ids)
    want = oracle(orc, cfg, w).forward(ids)
    assert rel_err(got, want) < 1e-4
    assert_close(got, want, 1e-3, 1e-4, "logits")


def test_csa_policy_gradient_step_matches_oracle(csa, orc):
    case, cfg, w, s = csa
    rng = np.random.default_rng(2)
    B, T = 3, 162
    inputs = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets[:, :40] = -1
    adv = np.array([0.5, -0.25, -0.25], np.float32)
    s.zero_grad()
    loss, nll = s.policy_gradient_step(inputs, targets, adv, float(T + 1))
    grads = s.grads()
    wl, wnll, wg = oracle(orc, cfg, w).pg_step(inputs, targets, adv, float(T + 1))
    assert abs(loss - wl) <= 1e-4 * max(abs(wl), 1e-3)
    assert rel_err(nll, wnll) < 1e-4
    _compare_grads(cfg, grads, wg)
    for name, r, c, off in cfg.param_table():
        if "indexer" in name or "compress" in name:
            assert np.any(grads[off:off + r * c]), name


def _teacher_forced(orc, cfg, w, prompts, rows, S, N, seeds):
    """Every sampled token of every row against the oracle's draw from the
    group stream given the same fed columns (tf_check.teacher_forced_group),
    so a near-tie flip between the engines' logits cannot change later
    columns of the comparison."""
    m = oracle(orc, cfg, w)
    checked = 0
    for g in range(prompts.shape[0]):
        checked += teacher_forced_group(orc, m, prompts[g], rows[g * S:(g + 1) * S],
                                        int(seeds[g]), N, 1.0, 50)
    assert checked > 0


def test_csa_rollouts_match_oracle(csa, orc):
    """Engine.GenerateBatchWith end to end (engine.go:112-369): the prefill
    (PrefillCED's bounded replay under CED), PrefillFrom, and every decode
    step's compression, indexer keys, selection and attention; every sampled
    token equals the oracle's draw by teacher forcing."""
    _, cfg, w, s = csa
    G_, P, S, N = 2, 37, 3, 20
    prompts = np.random.default_rng(4).integers(0, cfg.vocab_size, (G_, P)).astype(np.int32)
    seeds = np.array([7, 1000], np.uint64)
    got = s.generate_batch(prompts, S, N, 1.0, 50, seeds)
    _teacher_forced(orc, cfg, w, prompts, got, S, N, seeds)


def test_csa_decode_graph_matches_eager(csa):
    _, cfg, w, s = csa
    prompts = np.random.default_rng(5).integers(0, cfg.vocab_size, (3, 17)).astype(np.int32)
    seeds = np.array([3, 77, 901], np.uint64)
    try:
        s.set_decode_graph(False)
        eager = s.generate_batch(prompts, 2, 26, 1.0, 50, seeds)
        s.set_decode_graph(True)
        for _ in range(2):
            got = s.generate_batch(prompts, 2, 26, 1.0, 50, seeds)
            for a, b in zip(got, eager):
                assert np.array_equal(a, b)
            s.forward(prompts[:, :5])  # eager work between replays
    finally:
        s.set_decode_graph(True)


def test_csa_long_rollout_matches_oracle(orc):
    """A 300-token prompt and 180 decode steps of the hierarchical Full /
    Reindex / Reuse model: up to 119 compressed blocks per row, pools of 2,
    selections published and reused across layers while the local window
    slides."""
    from gonano_amd.session import Session
    cfg = csa_cfg("hier_fru")
    w = G.init_weights(cfg, seed=8, perturb=0.1)
    prompts = np.random.default_rng(9).integers(0, cfg.vocab_size, (1, 300)).astype(np.int32)
    seeds = np.array([5], np.uint64)
    with Session(cfg) as s:
        s.set_params(w)
        got = s.generate_batch(prompts, 2, 180, 1.0, 50, seeds)
    _teacher_forced(orc, cfg, w, prompts, got, 2, 180, seeds)


def test_ced_bounded_replay_rollout_matches_oracle(orc):
    """A 150-token prompt under a 64-token window: PrefillCED replays only
    the last 64 tokens through the decoder (its first replayed row unmixed
    by the smear), then decodes 40 steps."""
    from gonano_amd.session import Session
    cfg = csa_cfg("ced")
    w = G.init_weights(cfg, seed=12, perturb=0.05)
    prompts = np.random.default_rng(13).integers(0, cfg.vocab_size, (2, 150)).astype(np.int32)
    seeds = np.array([21, 22], np.uint64)
    with Session(cfg) as s:
        s.set_params(w)
        got = s.generate_batch(prompts, 2, 40, 1.0, 50, seeds)
    _teacher_forced(orc, cfg, w, prompts, got, 2, 40, seeds)


@pytest.mark.parametrize("case", ["flat", "hier_fru", "ced"])
def test_csa_select_kernels_agree(case, monkeypatch):
    """The two selection kernels (one wave per row; one block of 8 waves per
    row, chosen for decode-size row counts) rank by the same strict order,
    so forward logits (prefill-size selections) and rollouts (decode-size
    selections) are bitwise the same with either forced."""
    from gonano_amd.session import Session
    cfg = csa_cfg(case)
    w = G.init_weights(cfg, seed=41, perturb=0.05 if cfg.ced else 0.1)
    rng = np.random.default_rng(17)
    ids = rng.integers(0, cfg.vocab_size, (2, 150)).astype(np.int32)
    prompts = rng.integers(0, cfg.vocab_size, (2, 90)).astype(np.int32)
    seeds = np.array([5, 6], np.uint64)
    out = {}
    for mode in ("wave", "block"):
        monkeypatch.setenv("GN_CSA_SELECT", mode)
        with Session(cfg) as s:
            s.set_params(w)
            out[mode] = (s.forward(ids), s.generate_batch(prompts, 3, 40, 1.0, 50, seeds))
    assert np.array_equal(out["wave"][0], out["block"][0])
    for a, b in zip(out["wave"][1], out["block"][1]):
        assert np.array_equal(a, b)

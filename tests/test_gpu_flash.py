"""Parity of compressed attention (HCA: channel compressor, block-causal
attention over compressed keys, sliding-window local branch merged by
log-sum-exp; model/compress.go, model/compress_attention.go) on the GPU with
the oracle on identical inputs: Transformer.Forward logits (ragged last
blocks, with and without the local branch), PolicyGradientStep's NLL, loss
and every parameter gradient (the compressor's weight and bias included),
rollouts by teacher forcing (decode compresses each completed block into the
compressed cache, the prompt's tail logits wait in the ring), decode graphs
against eager launches, and one RL step with the DeepSeekMoE feed-forward
of the flash preset.

Floating-point bars as the dense tests: 1e-4 normwise relative per tensor
plus kerneltest.Close(1e-3, 1e-4) element-wise;
sampled ids are compared exactly.

The test with the DeepSeekMoE feed-forward perturbs InitWeights by N(0, 0.05)
(the others by 0.1, as the dense tests): on that RL step at 0.1 the oracle's
own float32 build is already 8.6e-5 normwise from its float64 build on the
gradient (6.5e-5 with compression; 1.7e-5 for compression alone), which
leaves no room to test a 1e-4 bar."""
import numpy as np
import pytest

from conftest import assert_close, rel_err
from gonano_amd import config as G
from test_gpu_session import _compare_grads

pytestmark = pytest.mark.gpu


def flash_small_cfg(swa=64, ratio=4, moe=False):
    # the flash family (D=128, GQA, partial RoPE, compression ratio 4, local
    # window) at a size the float64-accumulating oracle finishes in seconds
    cfg = G.Config(sequence_len=512, vocab_size=4096, n_layer=3, n_head=2, n_kv_head=1,
                   n_embd=256, window_pattern="SSSL", rotary_dims=64,
                   compression_ratio=ratio, swa_window=swa)
    if moe:
        cfg = G.enable_moe(cfg, n_experts=4, experts_per_token=2, expert_hidden=64,
                          shared_hidden=96, balance_weight=1e-2)
    return cfg


def oracle(orc, cfg, w, dtype=np.float32):
    return orc.OracleModel(orc.ModelShape.from_config(cfg), w, dtype)


@pytest.fixture(scope="module", params=[64, 0], ids=["swa64", "noswa"])
def flash(request):
    from gonano_amd.session import Session
    cfg = flash_small_cfg(swa=request.param)
    w = G.init_weights(cfg, seed=31, perturb=0.1)
    s = Session(cfg)
    s.set_params(w)
    yield cfg, w, s
    s.close()


def test_flash_param_roundtrip(flash):
    cfg, w, s = flash
    assert s.param_total == cfg.param_total()
    assert [(n, r, c, o) for n, r, c, o in s.param_table()] == cfg.param_table()
    assert any(n.endswith("attn.compress_bias") for n, *_ in s.param_table())
    assert np.array_equal(s.get_params(), w)


@pytest.mark.parametrize("T", [200, 3])  # a ragged last block; a sequence inside block 0
def test_flash_forward_matches_oracle(flash, orc, T):
    cfg, w, s = flash
    ids = np.random.default_rng(1).integers(0, cfg.vocab_size, (2, T)).astype(np.int32)
    got = s.forward(ids)
    want = oracle(orc, cfg, w).forward(ids)
    assert rel_err(got, want) < 1e-4
    assert_close(got, want, 1e-3, 1e-4, "logits")


@pytest.mark.parametrize("batch_splits", [None, "2"])
def test_flash_policy_gradient_step_matches_oracle(flash, orc, monkeypatch, batch_splits):
    """batch_splits "2": the indexer gradient's per-sequence products, one
    batched launch per head, split K in two (GN_GEMM_BATCH_SPLITS) and sum
    the partials of every sequence in one reduction launch."""
    if batch_splits:
        monkeypatch.setenv("GN_GEMM_BATCH_SPLITS", batch_splits)
    cfg, w, s = flash
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
    assert_close(nll, wnll, 1e-3, 1e-4, "nll")
    _compare_grads(cfg, grads, wg)
    for name, r, c, off in cfg.param_table():
        if "compress" in name:  # the compressor trains
            assert np.any(grads[off:off + r * c]), name


def test_flash_generate_teacher_forced(flash, orc):
    cfg, w, s = flash
    G_, P, S, N = 2, 21, 4, 24  # a prompt tail of one row; blocks complete while decoding
    prompts = np.random.default_rng(4).integers(0, cfg.vocab_size, (G_, P)).astype(np.int32)
    seeds = np.array([7, 1000], np.uint64)
    rows = s.generate_batch(prompts, S, N, 1.0, 50, seeds)
    m = oracle(orc, cfg, w)
    for g in range(G_):
        rng = orc.GoRNG(int(seeds[g]))
        group = rows[g * S:(g + 1) * S]
        for r in group:
            assert (r[:P] == prompts[g]).all()
        for t in range(N):
            live = [i for i in range(S) if len(group[i]) > P + t]
            if not live:
                break
            ctx = np.stack([np.concatenate([r[:P + t], np.zeros(max(0, P + t - len(r)), np.int32)])
                            for r in group])[:, :P + t]
            z = m.forward(ctx)[:, -1, :] if t > 0 else np.repeat(m.forward(prompts[g:g + 1])[:, -1, :], S, 0)
            want = orc.sample_next_token(z.astype(np.float32), rng, 1.0, 50)
            for i in live:
                assert group[i][P + t] == want[i], (g, i, t)


@pytest.mark.parametrize("P", [500, 3])
def test_flash_decode_long(orc, P):
    """A 500-token prompt and 540 decode steps with a 300-key window: the
    last steps attend to 259 compressed blocks (two decode splits) and 301
    raw keys (two more), all merged in one combine; a 3-token prompt starts
    inside block 0, where a query without a window sees nothing.  Teacher
    forcing on the last columns."""
    from gonano_amd.session import Session
    cfg = flash_small_cfg(swa=300 if P == 500 else 0)
    cfg.n_layer = 2
    w = G.init_weights(cfg, seed=5, perturb=0.1)
    S, N = 2, 540 if P == 500 else 12
    prompt = np.random.default_rng(6).integers(0, cfg.vocab_size, (1, P)).astype(np.int32)
    with Session(cfg) as s:
        s.set_params(w)
        rows = s.generate_batch(prompt, S, N, 1.0, 50, np.array([11], np.uint64))
    m = oracle(orc, cfg, w)
    rng = orc.GoRNG(11)
    first = max(N - 3, 0)
    rng.advance(S * cfg.vocab_size * first)
    for t in range(first, N):
        live = [i for i in range(S) if len(rows[i]) > P + t]
        if not live:
            break
        ctx = np.stack([np.concatenate([r[:P + t], np.zeros(max(0, P + t - len(r)), np.int32)])
                        for r in rows])[:, :P + t]
        z = m.forward(ctx)[:, -1, :]
        want = orc.sample_next_token(z.astype(np.float32), rng, 1.0, 50)
        for i in live:
            assert rows[i][P + t] == want[i], (i, t)


def test_flash_decode_graph_matches_eager(flash):
    cfg, w, s = flash
    prompts = np.random.default_rng(5).integers(0, cfg.vocab_size, (3, 17)).astype(np.int32)
    seeds = np.array([3, 77, 901], np.uint64)
    try:
        s.set_decode_graph(False)
        eager = s.generate_batch(prompts, 4, 30, 1.0, 50, seeds)
        s.set_decode_graph(True)
        for _ in range(2):
            got = s.generate_batch(prompts, 4, 30, 1.0, 50, seeds)
            for a, b in zip(got, eager):
                assert np.array_equal(a, b)
            s.forward(prompts[:, :5])  # eager work between replays
    finally:
        s.set_decode_graph(True)


def test_flash_rl_step_with_moe_matches_oracle(orc):
    """One RL step of a compressed model with the flash preset's DeepSeekMoE
    feed-forward: the PG step on the GPU's rollouts equals the oracle's on
    the same tokens."""
    from gonano_amd.session import Session
    cfg = flash_small_cfg(moe=True)
    cfg.vocab_size = 8192
    w = G.init_weights(cfg, seed=0, perturb=0.05)
    prompts = np.random.default_rng(1).integers(0, cfg.vocab_size, (2, 32)).astype(np.int32)
    rewards = (np.random.default_rng(2).random(16) < 0.3).astype(np.float32)
    seeds = np.arange(2, dtype=np.uint64)
    with Session(cfg) as s:
        s.set_params(w)
        s.zero_grad()
        out = s.rl_step(prompts, 8, 24, 1.0, 50, seeds, rewards)
        grads = s.grads()
        aux = s.aux_loss()
    rows, maxlen = out["rows"], out["max_len"]
    inputs = np.stack([np.concatenate([r, np.full(maxlen - len(r), 260, np.int32)])[:-1] for r in rows])
    targets = np.stack([np.concatenate([r, np.full(maxlen - len(r), 260, np.int32)])[1:] for r in rows])
    targets[:, :32] = -1
    m = oracle(orc, cfg, w)
    wl, _, wg = m.pg_step(inputs, targets, out["adv"], float(maxlen))
    assert abs(out["loss"] - wl) <= 1e-4 * max(abs(wl), 1e-3)
    assert abs(aux - m.aux_loss()) <= 1e-6 * abs(m.aux_loss())
    _compare_grads(cfg, grads, wg)

"""Parity of the device-resident RL step with the oracle on identical inputs:
Transformer.Forward logits, the top-k Gumbel sampler (bit-exact given the
same logits and stream), rollouts checked by teacher forcing (the oracle
re-samples every GPU column from its own logits of the GPU prefix with the
same Go stream), and PolicyGradientStep's NLL, loss and every parameter
gradient.

Tolerance for floating point: 1e-4 relative, measured
per tensor as ||got-want||_2 / ||want||_2, plus an element-wise
kerneltest.Close(rel 1e-3, abs 1e-4) guard against localized errors.  The
element-wise bar is looser because the oracle accumulates in float64 and the
MFMA GEMMs in float32: on the perturbed test models the oracle's own float32
build already sits 4e-5 (absolute) from its float64 build on some logits."""
import numpy as np
import pytest

from conftest import assert_close, rel_err
from gonano_amd import config as G

pytestmark = pytest.mark.gpu


def shape_of(cfg):
    from oracle.oracle import ModelShape
    return ModelShape(cfg.sequence_len, cfg.vocab_size, cfg.n_layer, cfg.n_head, cfg.n_kv_head,
                      cfg.n_embd, cfg.rotary_dims, cfg.window_pattern)


def small_cfg():
    # d12's shape family (D=128, GQA, partial RoPE, SSSL windows of 128) at a
    # size the float64-accumulating oracle finishes in seconds
    return G.Config(sequence_len=512, vocab_size=4096, n_layer=3, n_head=2, n_kv_head=1,
                    n_embd=256, window_pattern="SSSL", rotary_dims=64)


@pytest.fixture(scope="module")
def small():
    from gonano_amd.session import Session
    cfg = small_cfg()
    w = G.init_weights(cfg, seed=11, perturb=0.1)
    s = Session(cfg)
    s.set_params(w)
    yield cfg, w, s
    s.close()


def test_param_roundtrip(small):
    cfg, w, s = small
    assert s.param_total == cfg.param_total()
    assert [(n, r, c, o) for n, r, c, o in s.param_table()] == cfg.param_table()
    assert np.array_equal(s.get_params(), w)


def test_forward_matches_oracle(small, orc):
    cfg, w, s = small
    ids = np.random.default_rng(1).integers(0, cfg.vocab_size, (2, 200)).astype(np.int32)
    got = s.forward(ids)
    want = orc.OracleModel(shape_of(cfg), w).forward(ids)
    assert rel_err(got, want) < 1e-4
    assert_close(got, want, 1e-3, 1e-4, "logits")


def _compare_grads(cfg, got, want, tol=1e-4, scalar_tol=5e-4):
    """The whole gradient vector and every matrix parameter: normwise
    relative error below tol (1e-4).

    The per-layer lambdas and the smear scalars (fewer than 64 entries) are
    each ONE dot product over every token and channel of the end-of-chain
    gradient; their conditioning (~3 on these models) amplifies the float32
    error the GPU carries there (~4e-5, against ~1.5e-5 for the oracle's own
    float32 build, which accumulates in float64), so they are held to
    scalar_tol.  A tensor whose exact gradient is (near) zero by symmetry --
    backout_lambda when the backout layer is the last one, whose output only
    feeds a scale-invariant RMSNorm -- holds roundoff on both sides and
    passes when its absolute error is below 1e-5 of the largest gradient
    entry of the model."""
    assert rel_err(got, want) < tol
    floor = 1e-5 * float(np.abs(want).max())
    worst = []
    for name, r, c, off in cfg.param_table():
        g, wv = got[off:off + r * c], want[off:off + r * c]
        d = float(np.abs(g - wv).max())
        if d <= floor:
            continue
        e = rel_err(g, wv)
        worst.append((e, name))
        assert e < (tol if r * c >= 64 else scalar_tol), (name, e, d, floor)
        assert d <= 1e-3 * np.abs(wv).max() + floor, name
    return max(worst) if worst else (0.0, "")


def test_policy_gradient_step_matches_oracle(small, orc):
    cfg, w, s = small
    rng = np.random.default_rng(2)
    B, T = 3, 160
    inputs = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets[:, :40] = -1
    adv = np.array([0.5, -0.25, -0.25], np.float32)
    s.zero_grad()
    loss, nll = s.policy_gradient_step(inputs, targets, adv, float(T + 1))
    grads = s.grads()
    wl, wnll, wg = orc.OracleModel(shape_of(cfg), w).pg_step(inputs, targets, adv, float(T + 1))
    assert abs(loss - wl) <= 1e-4 * max(abs(wl), 1e-3)
    assert rel_err(nll, wnll) < 1e-4
    assert_close(nll, wnll, 1e-3, 1e-4, "nll")
    _compare_grads(cfg, grads, wg)
    # gradients accumulate across calls (Tensor.Grad semantics)
    s.policy_gradient_step(inputs, targets, adv, float(T + 1))
    assert rel_err(s.grads(), 2 * grads) < 1e-6


@pytest.mark.parametrize("V", [12340, 33000, 50260, 50257])
def test_pg_step_partial_vocab_rows(orc, V):
    """Vocabularies that are not a multiple of 4096: the register loss
    kernel's partial-row variants (4, 8 and 16 float4 per thread, padding
    masked) and the streaming kernel (V % 4 != 0); NLL, loss and every
    gradient against the oracle.  (50,257 is GPT-2's vocabulary.)"""
    from gonano_amd.session import Session
    cfg = G.Config(sequence_len=256, vocab_size=V, n_layer=1, n_head=2, n_kv_head=1, n_embd=256,
                   window_pattern="L", rotary_dims=64)
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    rng = np.random.default_rng(V)
    inputs = rng.integers(0, V, (2, 96)).astype(np.int32)
    targets = rng.integers(0, V, (2, 96)).astype(np.int32)
    targets[:, :20] = -1
    targets[1, 50] = V - 1  # the last entry of the padded group
    adv = np.array([0.7, -0.3], np.float32)
    with Session(cfg) as s:
        s.set_params(w)
        s.zero_grad()
        loss, nll = s.policy_gradient_step(inputs, targets, adv, 97.0)
        grads = s.grads()
    wl, wnll, wg = orc.OracleModel(shape_of(cfg), w).pg_step(inputs, targets, adv, 97.0)
    assert abs(loss - wl) <= 1e-4 * max(abs(wl), 1e-3)
    assert_close(nll, wnll, 1e-3, 1e-4, "nll")
    _compare_grads(cfg, grads, wg)


def test_sampler_bit_exact(orc):
    from gonano_amd.backend import sample_next_token
    rng = np.random.default_rng(3)
    # the row held in registers (V <= 65,536, V % 4 == 0) with 1, 2 and 4
    # group maxima per thread (k up to 1024), the two-pass path (V > 65,536,
    # or V % 4 != 0), argmax, no mask, and small rows mostly -inf (fewer
    # finite entries than k: every entry is a candidate)
    for V, rows, T, k in [(4096, 64, 1.0, 50), (65536, 8, 1.0, 50), (32768, 16, 0.8, 50),
                          (1000, 9, 1.0, 0), (300, 5, 1.0, 300), (777, 7, 0.0, 50), (5000, 4, 1.3, 1),
                          (8192, 6, 1.0, 300), (8192, 6, 1.0, 600), (65536, 3, 1.0, 1000),
                          (70004, 3, 1.0, 50), (1001, 5, 1.0, 50), (128, 3, 1.0, 50)]:
        z = (rng.standard_normal((rows, V)) * 2).astype(np.float32)
        z[:, ::97] = z[:, :1]  # ties, including at the threshold
        z = np.round(z * 64) / 64  # many exact duplicates
        z = z.astype(np.float32)
        if V == 128:
            z[:, :120] = -np.inf
        for seed in (0, 12345):
            g = orc.GoRNG(seed)
            state = np.array(g.hi_lo, np.uint64)
            got = sample_next_token(z, state, T, k)
            want = orc.sample_next_token(z, g, T, k)
            assert (got == want).all(), (V, T, k, seed, np.nonzero(got != want))
            assert tuple(int(x) for x in state) == g.hi_lo


def test_generate_teacher_forced(small, orc):
    cfg, w, s = small
    G_, P, S, N = 2, 20, 4, 24
    prompts = np.random.default_rng(4).integers(0, cfg.vocab_size, (G_, P)).astype(np.int32)
    seeds = np.array([7, 1000], np.uint64)
    rows = s.generate_batch(prompts, S, N, 1.0, 50, seeds)
    assert len(rows) == G_ * S
    m = orc.OracleModel(shape_of(cfg), w)
    for g in range(G_):
        rng = orc.GoRNG(int(seeds[g]))
        group = rows[g * S:(g + 1) * S]
        for r in group:
            assert (r[:P] == prompts[g]).all()
            assert 260 not in r[P:] and 256 not in r[P:]
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


def test_softcap_non_decreasing_over_all_floats():
    """The decode sampler picks its top-k candidates on the raw lm_head
    products and softcaps only those, which equals softcapping every logit
    first because the device softcap is non-decreasing over all floats:
    checked exhaustively, every neighbouring pair of the 2^32 bit patterns
    but NaNs."""
    from gonano_amd.backend import softcap_order_violations
    assert softcap_order_violations() == 0


def test_generate_saturated_softcap_teacher_forced(orc):
    """lm_head scaled by 1e9: nearly every logit softcaps to exactly +-15, so
    the sampler's selection on raw products cannot prove its bound (softcap
    is flat across it) and every row takes the exact radix select over the
    softcapped row, with thousands of tied logits kept; the tokens still
    match the oracle's.  (At this scale no product falls in the band where
    float32 and float64 tanh round to different sides of 15.)"""
    from gonano_amd.session import Session
    cfg = small_cfg()
    w = G.init_weights(cfg, seed=11, perturb=0.1).copy()
    (name, r, c, off), = [e for e in cfg.param_table() if e[0] == "lm_head.weight"]
    w[off:off + r * c] *= 1e9
    G_, P, S, N = 2, 20, 4, 6
    prompts = np.random.default_rng(5).integers(0, cfg.vocab_size, (G_, P)).astype(np.int32)
    seeds = np.array([3, 99], np.uint64)
    with Session(cfg) as s:
        s.set_params(w)
        rows = s.generate_batch(prompts, S, N, 1.0, 50, seeds)
    m = orc.OracleModel(shape_of(cfg), w)
    checked = 0
    for g in range(G_):
        rng = orc.GoRNG(int(seeds[g]))
        group = rows[g * S:(g + 1) * S]
        for t in range(N):
            live = [i for i in range(S) if len(group[i]) > P + t]
            if not live:
                break
            ctx = np.stack([np.concatenate([r[:P + t], np.zeros(max(0, P + t - len(r)), np.int32)])
                            for r in group])[:, :P + t]
            z = m.forward(ctx)[:, -1, :] if t > 0 else np.repeat(m.forward(prompts[g:g + 1])[:, -1, :], S, 0)
            z = z.astype(np.float32)
            assert (np.abs(z) == 15.0).mean() > 0.9
            want = orc.sample_next_token(z, rng, 1.0, 50)
            for i in live:
                assert group[i][P + t] == want[i], (g, i, t)
                checked += 1
    assert checked >= G_ * S


def test_decode_graph_replays_match_eager(small):
    """Rollouts replayed from the captured decode graph equal the eager ones
    token for token, across repeated calls (a fresh capture per call, with
    eager work and synchronizations between the replays) and for a shorter
    second call."""
    cfg, w, s = small
    prompts = np.random.default_rng(5).integers(0, cfg.vocab_size, (3, 17)).astype(np.int32)
    seeds = np.array([3, 77, 901], np.uint64)
    try:
        s.set_decode_graph(False)
        eager = s.generate_batch(prompts, 4, 30, 1.0, 50, seeds)
        eager_short = s.generate_batch(prompts, 4, 9, 0.7, 20, seeds)
        s.set_decode_graph(True)
        for _ in range(2):
            got = s.generate_batch(prompts, 4, 30, 1.0, 50, seeds)
            assert len(got) == len(eager)
            for a, b in zip(got, eager):
                assert np.array_equal(a, b)
            s.forward(prompts[:, :5])  # eager work between replays
            got = s.generate_batch(prompts, 4, 9, 0.7, 20, seeds)
            for a, b in zip(got, eager_short):
                assert np.array_equal(a, b)
    finally:
        s.set_decode_graph(True)


def test_rl_step_d2_matches_oracle(orc):
    """The benchmark's d2 workload: dense depth 2, 4 prompts x 8 samples, 24 new
    tokens, T=1.0, top-k 50, Bernoulli(0.3) rewards; the PG step on the
    GPU's rollouts is compared with the oracle's on the same tokens."""
    from gonano_amd.session import Session
    cfg = G.dense_d2()
    w = G.init_weights(cfg, seed=0, perturb=0.1)
    prompts = np.random.default_rng(1).integers(0, cfg.vocab_size, (4, 32)).astype(np.int32)
    rewards = (np.random.default_rng(2).random(32) < 0.3).astype(np.float32)
    seeds = np.arange(4, dtype=np.uint64)  # step*1000 + g at step 0
    with Session(cfg) as s:
        s.set_params(w)
        s.zero_grad()
        out = s.rl_step(prompts, 8, 24, 1.0, 50, seeds, rewards)
        grads = s.grads()
    lens = out["lens"]
    assert out["max_len"] == lens.max()
    rows = out["rows"]
    maxlen = out["max_len"]
    inputs = np.stack([np.concatenate([r, np.full(maxlen - len(r), 260, np.int32)])[:-1] for r in rows])
    targets = np.stack([np.concatenate([r, np.full(maxlen - len(r), 260, np.int32)])[1:] for r in rows])
    targets[:, :32] = -1
    adv = rewards - rewards.reshape(4, 8).mean(1).repeat(8)
    assert_close(out["adv"], adv, 1e-6, 1e-7, "advantages")
    m = orc.OracleModel(shape_of(cfg), w)
    wl, wnll, wg = m.pg_step(inputs, targets, out["adv"], float(maxlen))
    m64 = orc.OracleModel(shape_of(cfg), w.astype(np.float64), dtype=np.float64)
    _, _, wg64 = m64.pg_step(inputs, targets, out["adv"], float(maxlen))
    for name, r, c, off in cfg.param_table():
        sl = slice(off, off + r * c)
        print(f"{name:40s} gpu-f32 {rel_err(grads[sl], wg[sl]):.2e}  gpu-f64 "
              f"{rel_err(grads[sl], wg64[sl]):.2e}  f32-f64 {rel_err(wg[sl], wg64[sl]):.2e}")
        if r * c < 64:
            print("   gpu", grads[sl], "\n   f32", wg[sl], "\n   f64", wg64[sl])
    assert abs(out["loss"] - wl) <= 1e-4 * max(abs(wl), 1e-3)
    _compare_grads(cfg, grads, wg)
    # teacher-forced check of the first group's first columns
    rng = orc.GoRNG(0)
    group = rows[:8]
    for t in range(4):
        ctx = np.stack([r[:32 + t] for r in group])
        z = m.forward(ctx)[:, -1, :]
        want = orc.sample_next_token(z, rng, 1.0, 50)
        for i in range(8):
            if len(group[i]) > 32 + t:
                assert group[i][32 + t] == want[i]

"""Parity at the benchmark's shapes.

The other GPU tests use narrow models (C = 256, two query heads) that the
oracle finishes quickly; the kernel paths the benchmark workloads select
depend on width, head counts, row counts and context lengths, so these
tests run those exact widths -- d12 (C 768, 6:2 heads, F 3072), d20 (C 1280,
10:2 heads), latent d12 (MLA latent 256 over 6:3 heads, 16 experts of 512)
and flash d12 (6:1 heads, ratio 4, top-16 of 128 candidates, SWA 512, FRU,
CED, 16 experts of 768) -- with the row counts of their rollouts (256, 512,
256, 64) and prompts long enough to reach the multi-split decode attention
and the hierarchical selection, at a depth and vocabulary the oracle handles
in seconds; plus the full d12 model (12 layers, V = 65536).  The paths
checked include decode attention at GQA ratios 3, 5 and 6 with one or two
key splits and the combine, with the q/k/v post-processing fused into it
(plain windows) or launched apart, the 32 x 96 decode GEMM tiles with
deferred split-K sums (M = 256, N a multiple of 96), MLA decode at 6:3
heads, the sparse decode at 6:1, and the policy-gradient loss over several
logits chunks (GN_LOGITS_CHUNK) with the rows without a target left out of
the lm_head products.

Rollouts are checked by teacher forcing (tests/tf_check.py: every sampled
token of every checked group equals the oracle's draw from the group stream
given the same prefix, bit-exact); logits at the 1e-4 normwise bar of the
other GPU tests.  The policy-gradient step is compared with the oracle's
float32 build, which takes the same discrete decisions (expert routing,
block selection) as the GPU, at 1e-4 or at twice the oracle's own float32
error (float32 build against float64 build) where that is larger.

MLA has no QK-norm, so its attention logits grow with the width and the
weight perturbation: the latent and flash tests perturb InitWeights by
N(0, 0.02) at C = 768 (the narrow tests' 0.05 at C = 256).  At 0.05 and
C = 768 the problem is ill-conditioned: the oracle's float32 build is 3.7e-5
from its float64 build on the latent gradient and a float32-accumulating
implementation (the GPU, like the reference's SIMD backend) 2e-4; at 0.02
both are below 1e-5."""
import dataclasses
import os

import numpy as np
import pytest

from conftest import assert_close, rel_err
from gonano_amd import config as G
from tf_check import teacher_forced_group

pytestmark = pytest.mark.gpu


def with_depth(cfg, layers, vocab):
    return dataclasses.replace(cfg, n_layer=layers, vocab_size=vocab)


def d12_width():
    return with_depth(G.dense_d12(), 2, 4096)


def d20_width():
    return with_depth(G.dense_d20(), 2, 4096)


def latent_width():
    cfg = G.config_for_depth_ratio(12, 4096, 64, 128, 512, "SSSL", 1)
    cfg.n_layer = 2
    return G.apply_latent_preset(cfg, mla_latent=256, n_experts=16, experts_per_token=2,
                                 expert_hidden=512)


def flash_width():
    cfg = G.config_for_depth_ratio(12, 4096, 64, 128, 2048, "SSSL", 1)
    cfg.n_kv_head = 1
    cfg.n_layer = 6
    return G.apply_flash_preset(cfg, sparse_topk=16, swa_window=512, n_experts=16)


def _model(orc, cfg, w):
    return orc.OracleModel(orc.ModelShape.from_config(cfg), w)


def _rollout_check(orc, cfg, w, G_, S, P, N, temperature, groups, seed0=1000):
    from gonano_amd.session import Session
    prompts = np.random.default_rng(cfg.n_embd + P).integers(0, cfg.vocab_size, (G_, P)).astype(np.int32)
    seeds = (seed0 + np.arange(G_)).astype(np.uint64)
    with Session(cfg) as s:
        s.set_params(w)
        rows = s.generate_batch(prompts, S, N, temperature, 50, seeds)
    assert len(rows) == G_ * S
    m = _model(orc, cfg, w)
    checked = 0
    for g in groups:
        checked += teacher_forced_group(orc, m, prompts[g], rows[g * S:(g + 1) * S], seeds[g], N,
                                        temperature, 50)
    assert checked >= len(groups) * S * min(N, 4)
    return checked


def report(line):
    """One line of the parity report: printed (pytest -s / -rA show it) and
    appended to $GN_PARITY_REPORT when that is set."""
    print(line)
    path = os.environ.get("GN_PARITY_REPORT")
    if path:
        with open(path, "a") as f:
            f.write(line + "\n")


def _bar(e32, tol):
    """The accuracy bar of one quantity: tol (the north-star 1e-4), or twice
    the oracle's own float32 error (its float32 build against its float64
    build) where the float32 arithmetic itself is further than that from the
    exact result -- an ill-conditioned tensor, which no float32
    implementation can be held closer to than its own rounding."""
    return max(tol, 2.0 * e32)


def _compare_grads(cfg, got, w32, w64, tol=1e-4, scalar_tol=5e-4):
    """Every parameter's gradient against the oracle's float32 build (which
    takes the same discrete decisions -- expert routing, block selection --
    as the GPU): normwise within _bar(float32-vs-float64 error, tol) --
    scalar_tol for the per-layer lambdas and smear scalars (single dot
    products over every token and channel) -- and element-wise within 1e-3 of
    the tensor's largest entry.  Tensors whose gradient is roundoff on both
    sides pass below 1e-5 of the largest entry of the model."""
    floor = 1e-5 * float(np.abs(w32).max())
    rows, bad = [], []
    for name, r, c, off in cfg.param_table():
        g, a, b = got[off:off + r * c], w32[off:off + r * c], w64[off:off + r * c]
        d = float(np.abs(g - a).max())
        e, e32 = rel_err(g, a), rel_err(a, b)
        base = tol if r * c >= 64 else scalar_tol
        bar = _bar(e32, base)
        rows.append((e, e32, bar, base, name))
        if d <= floor:
            continue
        if e >= bar or d > 1e-3 * np.abs(a).max() + floor:
            bad.append((name, e, e32, d))
    e_all, e32_all = rel_err(got, w32), rel_err(w32, w64)
    report(f"all gradients: gpu-f32 {e_all:.2e}  f32-f64 {e32_all:.2e}  bar "
           f"{_bar(e32_all, tol):.1e}{' (widened)' if _bar(e32_all, tol) > tol else ''}")
    for e, e32, bar, base, n in rows:
        report(f"  {n:45s} gpu-f32 {e:.2e}  f32-f64 {e32:.2e}  bar {bar:.1e}"
               f"{' (widened)' if bar > base else ''}")
    worst = "\n".join(f"  {n:45s} gpu-f32 {e:.2e}  f32-f64 {e32:.2e}" for e, e32, _, _, n in
                      sorted(rows, reverse=True)[:8])
    assert e_all < _bar(e32_all, tol), worst
    assert not bad, f"{bad}\n{worst}"


def _pg_check(orc, cfg, w, B, T, prompt_len, chunk, monkeypatch, seed=7, timing=False):
    """PolicyGradientStep on random sequences whose first prompt_len targets
    are ignored (the chat_rl masking); the logits run in chunks of `chunk`
    rows, so several chunks and a partial last one are exercised.  Loss, NLL
    and gradients are compared with the oracle's float32 build within the
    1e-4 bar, or twice the oracle's own float32 error (its float64 build
    runs too) where that is larger."""
    from gonano_amd.session import Session
    rng = np.random.default_rng(seed)
    inputs = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets[:, :prompt_len] = -1
    adv = np.linspace(-0.5, 0.5, B).astype(np.float32) + 0.1
    monkeypatch.setenv("GN_LOGITS_CHUNK", str(chunk))
    with Session(cfg) as s:
        s.set_params(w)
        s.set_timing(timing)
        s.zero_grad()
        loss, nll = s.policy_gradient_step(inputs, targets, adv, float(T + 1))
        grads = s.grads()
        aux = s.aux_loss()
        t = s.timing() if timing else None
    monkeypatch.delenv("GN_LOGITS_CHUNK")
    m32 = _model(orc, cfg, w)
    l32, n32, g32 = m32.pg_step(inputs, targets, adv, float(T + 1))
    m64 = orc.OracleModel(orc.ModelShape.from_config(cfg), w.astype(np.float64), dtype=np.float64)
    l64, n64, g64 = m64.pg_step(inputs, targets, adv, float(T + 1))
    import inspect
    report(f"== {inspect.stack()[1].function}: V {cfg.vocab_size}, {B} x {T} tokens, "
           f"{B * (T - prompt_len)} target rows, logits chunk {chunk}")
    lbar = max(1e-4 * max(abs(l32), 1e-3), 2 * abs(l32 - l64))
    report(f"loss: gpu {loss:.9g} f32 {l32:.9g} f64 {l64:.9g}  |gpu-f32| {abs(loss - l32):.2e} "
           f"bar {lbar:.1e}")
    e_n, e32_n = rel_err(nll, n32), rel_err(n32, n64)
    report(f"nll: gpu-f32 {e_n:.2e}  f32-f64 {e32_n:.2e}  bar {_bar(e32_n, 1e-4):.1e}")
    assert abs(loss - l32) <= lbar, (loss, l32, l64)
    assert np.all(nll[:, :prompt_len] == 0)
    assert e_n < _bar(e32_n, 1e-4), (e_n, e32_n)
    assert_close(nll, n32, 1e-3, 1e-4, "nll")
    if cfg.moe:
        assert abs(aux - m32.aux_loss()) <= 1e-6 * max(abs(m32.aux_loss()), 1e-9)
    _compare_grads(cfg, grads, g32, g64)
    return t


# ---- dense d12 width (the benchmark's d12 workload at 2 layers, V 4096) -----
@pytest.fixture(scope="module")
def d12w():
    cfg = d12_width()
    assert (cfg.n_embd, cfg.n_head, cfg.n_kv_head, cfg.mlp_hidden) == (768, 6, 2, 3072)
    assert cfg.window_sizes() == [128, 512]
    return cfg, G.init_weights(cfg, seed=12, perturb=0.1)


def test_d12_width_rollout_teacher_forced(orc, d12w):
    """256 rows (16 groups x 16), 260-token prompts: the full-context layer
    attends 260..267 keys and the windowed layer 129, each in one split (256
    rows x 2 KV heads fill the CUs without splitting the keys); the attention
    kernel does the q/k/v post-processing itself (VE gate on the full layer,
    RoPE, QK-norm, the new key/value written to the cache); the decode MLP
    and output projections take the 32 x 96 tiles at M = 256."""
    cfg, w = d12w
    _rollout_check(orc, cfg, w, 16, 16, 260, 8, 1.0, groups=(0, 7, 15))


def test_d12_width_split_combine_rollout(orc, d12w):
    """32 rows (2 groups x 16) with 300-token prompts: 64 (row, kv-head)
    blocks leave the keys in splits of at most 256, so the full-context
    layer's 301..306 keys take two splits and the combine kernel (the dense
    multi-split path; the benchmark's 256 and 512 rows run one split)."""
    cfg, w = d12w
    _rollout_check(orc, cfg, w, 2, 16, 300, 6, 1.0, groups=(0, 1))


def test_d12_width_pg_step_chunked(orc, d12w, monkeypatch):
    cfg, w = d12w
    _pg_check(orc, cfg, w, B=3, T=300, prompt_len=150, chunk=128, monkeypatch=monkeypatch)


def test_d12_width_pg_step_wide_engine(orc, d12w, monkeypatch):
    """The policy-gradient step with every product the 256 x 256-tile engine
    can take routed there at any grid size (GN_GEMM_WIDE_MIN=1; the
    benchmark's 130,816-token products take it by size): 4 x 512 tokens
    make every M, N >= 256 and every K a multiple of 64, so the instances
    run are the forward products (plain qkv, residual-add wo, ReLU^2 fc
    with the saved pre-activation, the proj product as split-K partials
    with the residual add in the reduction), the input gradients (plain,
    ReLU^2 backward, split-K partials), the weight gradients (split-K
    partials over the tokens), and the lm_head forward, input gradient
    (split over the vocabulary) and weight gradient (accumulated) over two
    256-row logits chunks."""
    cfg, w = d12w
    monkeypatch.setenv("GN_GEMM_WIDE_MIN", "1")
    t = _pg_check(orc, cfg, w, B=4, T=512, prompt_len=384, chunk=256, monkeypatch=monkeypatch,
                  timing=True)
    monkeypatch.delenv("GN_GEMM_WIDE_MIN")
    # every product of the step ran on the wide engine
    assert t["gemm_wide_launches"] == t["gemm_launches"], t


def test_d12_width_pg_step_tile_engine(orc, d12w, monkeypatch):
    """The same 4 x 512-token step with the wide engine switched off
    (GN_GEMM_WIDE=0): the large products run on gemm_kernel, whose 128 x 128
    tiles take the epilogues through LDS (store, residual add, ReLU^2 with
    the saved pre-activation, ReLU^2 backward) and whose long-K products
    split K into float64-summed partials."""
    cfg, w = d12w
    monkeypatch.setenv("GN_GEMM_WIDE", "0")
    t = _pg_check(orc, cfg, w, B=4, T=512, prompt_len=384, chunk=256, monkeypatch=monkeypatch,
                  timing=True)
    monkeypatch.delenv("GN_GEMM_WIDE")
    assert t["gemm_wide_launches"] == 0, t


def test_d12_width_pg_step_wide_engine_ragged_k(orc, d12w, monkeypatch):
    """As above with 4 x 500 tokens: the weight gradients' K (2000 tokens) is
    not a multiple of 64, so the engine runs K in [0, 1984) as its splits
    and the last 16 tokens as one more split on gemm_kernel, summed with the
    others by the reduction (the flash and d20 workloads' token counts,
    16 x 8703 and B x 1535, take this path)."""
    cfg, w = d12w
    monkeypatch.setenv("GN_GEMM_WIDE_MIN", "1")
    t = _pg_check(orc, cfg, w, B=4, T=500, prompt_len=372, chunk=256, monkeypatch=monkeypatch,
                  timing=True)
    monkeypatch.delenv("GN_GEMM_WIDE_MIN")
    assert t["gemm_wide_launches"] == t["gemm_launches"], t


def test_d12_width_graph_equals_eager(d12w):
    """The captured decode graph at the d12 width replays the eager steps
    token for token (two replays, eager work between them)."""
    from gonano_amd.session import Session
    cfg, w = d12w
    prompts = np.random.default_rng(9).integers(0, cfg.vocab_size, (16, 260)).astype(np.int32)
    seeds = np.arange(16, dtype=np.uint64)
    with Session(cfg) as s:
        s.set_params(w)
        s.set_decode_graph(False)
        eager = s.generate_batch(prompts, 16, 10, 1.0, 50, seeds)
        s.set_decode_graph(True)
        for _ in range(2):
            got = s.generate_batch(prompts, 16, 10, 1.0, 50, seeds)
            assert all(np.array_equal(a, b) for a, b in zip(got, eager))
            s.forward(prompts[:2, :8])


def test_d12_width_fused_qkv_post_equals_separate(d12w, monkeypatch):
    """The q/k/v post-processing inside the decode attention kernel (the
    default) and the separate qkv_post launch (GN_FUSE_QKV_POST=0) give the
    same rollouts token for token: the same arithmetic in the same order,
    the new key and value written to the cache and used from the block's own
    copy on the step they are made."""
    from gonano_amd.session import Session
    cfg, w = d12w
    prompts = np.random.default_rng(4).integers(0, cfg.vocab_size, (16, 260)).astype(np.int32)
    seeds = np.arange(100, 116, dtype=np.uint64)
    out = {}
    for fuse in ("0", "1"):
        monkeypatch.setenv("GN_FUSE_QKV_POST", fuse)
        with Session(cfg) as s:
            s.set_params(w)
            out[fuse] = s.generate_batch(prompts, 16, 12, 1.0, 50, seeds)
    monkeypatch.delenv("GN_FUSE_QKV_POST")
    assert len(out["0"]) == len(out["1"]) == 256
    assert all(np.array_equal(a, b) for a, b in zip(out["0"], out["1"]))


# ---- d12 width at the benchmark's vocabulary (V = 65536) --------------------
@pytest.fixture(scope="module")
def d12v():
    cfg = with_depth(G.dense_d12(), 2, 65536)
    return cfg, G.init_weights(cfg, seed=65, perturb=0.1)


def test_d12_vocab_pg_step_chunked(orc, d12v, monkeypatch):
    """The policy-gradient step at the benchmark's vocabulary: V = 65536 runs
    the loss kernel's 16-register instance over whole 4096-wide tiles
    (pg_loss_rows_reg_kernel<16, true>, the instance d12 and d20 run).
    2 x 256 tokens, the first 128 of each without a target: 256 target rows
    in three logits chunks (96, 96, 64)."""
    cfg, w = d12v
    _pg_check(orc, cfg, w, B=2, T=256, prompt_len=128, chunk=96, monkeypatch=monkeypatch)


def test_d12_vocab_pg_step_wide_engine(orc, d12v, monkeypatch):
    """The same vocabulary with 256-row logits chunks and every product the
    256 x 256-tile engine can take routed there (GN_GEMM_WIDE_MIN=1): the
    lm_head forward, its input gradient (K = 65536, split) and weight
    gradient at the benchmark's V."""
    cfg, w = d12v
    monkeypatch.setenv("GN_GEMM_WIDE_MIN", "1")
    t = _pg_check(orc, cfg, w, B=2, T=384, prompt_len=128, chunk=256, monkeypatch=monkeypatch,
                  timing=True)
    monkeypatch.delenv("GN_GEMM_WIDE_MIN")
    assert t["gemm_wide_launches"] == t["gemm_launches"], t


# ---- the full d12 model (the benchmark's d12 workload) ----------------------
@pytest.fixture(scope="module")
def d12full():
    cfg = G.dense_d12()
    return cfg, G.init_weights(cfg, seed=0, perturb=0.1)


def test_d12_forward_logits(orc, d12full):
    """12 layers, V = 65536: Transformer.Forward logits of a short batch."""
    from gonano_amd.session import Session
    cfg, w = d12full
    ids = np.random.default_rng(1).integers(0, cfg.vocab_size, (2, 96)).astype(np.int32)
    with Session(cfg) as s:
        s.set_params(w)
        got = s.forward(ids)
    want = _model(orc, cfg, w).forward(ids)
    assert rel_err(got, want) < 1e-4
    assert_close(got, want, 1e-3, 1e-4, "logits")


def test_d12_rollout_teacher_forced(orc, d12full):
    """The benchmark's rollout shape (16 x 16 rows, 256-token prompts, the
    12-layer model, V = 65536 through the lm_head and the sampler) for its
    first columns."""
    cfg, w = d12full
    _rollout_check(orc, cfg, w, 16, 16, 256, 4, 1.0, groups=(5,))


# ---- dense d20 width (the benchmark's d20 workload at 2 layers, V 4096) -----
@pytest.fixture(scope="module")
def d20w():
    cfg = d20_width()
    assert (cfg.n_embd, cfg.n_head, cfg.n_kv_head) == (1280, 10, 2)
    assert cfg.window_sizes() == [512, 2048]
    return cfg, G.init_weights(cfg, seed=20, perturb=0.1)


def test_d20_width_rollout_teacher_forced(orc, d20w):
    """512 rows (32 x 16), 520-token prompts, T = 0.8: GQA ratio 5, every
    window in one split of up to 528 keys (the 512-token window admits 513);
    the decode projections at M = 512 take the 32 x 80 / 32 x 112 tiles with
    deferred split sums or run whole on gemm_kernel."""
    cfg, w = d20w
    _rollout_check(orc, cfg, w, 32, 16, 520, 6, 0.8, groups=(0, 31))


def test_d20_width_pg_step_chunked(orc, d20w, monkeypatch):
    cfg, w = d20w
    _pg_check(orc, cfg, w, B=1, T=540, prompt_len=520, chunk=8, monkeypatch=monkeypatch)


# ---- latent d12 width (the benchmark's latent d12 workload at 2 layers, V 4096) ---
@pytest.fixture(scope="module")
def latw():
    cfg = latent_width()
    assert (cfg.n_embd, cfg.n_head, cfg.n_kv_head, cfg.mla_latent) == (768, 6, 3, 256)
    assert (cfg.n_experts, cfg.experts_per_token, cfg.expert_hidden) == (16, 2, 512)
    return cfg, G.init_weights(cfg, seed=31, perturb=0.02)


def test_latent_width_rollout_teacher_forced(orc, latw):
    cfg, w = latw
    _rollout_check(orc, cfg, w, 16, 16, 260, 8, 1.0, groups=(0, 15))


def test_latent_width_pg_step_chunked(orc, latw, monkeypatch):
    cfg, w = latw
    _pg_check(orc, cfg, w, B=2, T=300, prompt_len=150, chunk=100, monkeypatch=monkeypatch)


def _wide_launches(cfg, w, B, T, prompt_len, env, monkeypatch, seed=7):
    """gemm_wide_launches of one policy-gradient step under env (no oracle)."""
    from gonano_amd.session import Session
    rng = np.random.default_rng(seed)
    inputs = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    targets[:, :prompt_len] = -1
    for k, v in env.items():
        monkeypatch.setenv(k, v)
    with Session(cfg) as s:
        s.set_params(w)
        s.set_timing(True)
        s.zero_grad()
        s.policy_gradient_step(inputs, targets, np.full(B, 0.3, np.float32), float(T + 1))
        t = s.timing()
    for k in env:
        monkeypatch.delenv(k)
    return t["gemm_wide_launches"], t["gemm_launches"]


@pytest.mark.parametrize("parts", ["1", "3"])
def test_latent_width_pg_step_wide_grouped_k(orc, latw, monkeypatch, parts):
    """The routed experts' weight gradients (GEMM_GROUP_K: one reduction
    over each expert's rows) on the 256 x 256-tile engine, each expert's
    rows cut into `parts` ranges (GN_GEMM_WIDE_PARTS; the benchmark's
    16,000-row experts take 8 by the round-filling rule) whose partials
    gemm_reduce_kernel sums into the gradient.  600 tokens give ~75 rows per
    expert: every range ends inside a tile pair (rows past it read as
    zeros), and at 3 parts some experts' last range is empty.  Against the
    oracle as the other policy-gradient checks; the launch count against
    GN_GEMM_WIDE_GROUPED_K=0 shows the three weight gradients of each layer
    (down, gate, up) moved."""
    cfg, w = latw
    monkeypatch.setenv("GN_GEMM_WIDE_MIN", "1")
    monkeypatch.setenv("GN_GEMM_WIDE_PARTS", parts)
    _pg_check(orc, cfg, w, B=2, T=300, prompt_len=150, chunk=100, monkeypatch=monkeypatch)
    monkeypatch.delenv("GN_GEMM_WIDE_PARTS")
    monkeypatch.delenv("GN_GEMM_WIDE_MIN")
    env = {"GN_GEMM_WIDE_MIN": "1", "GN_GEMM_WIDE_PARTS": parts, "GN_LOGITS_CHUNK": "100"}
    on, n_on = _wide_launches(cfg, w, 2, 300, 150, env, monkeypatch)
    off, n_off = _wide_launches(cfg, w, 2, 300, 150, {**env, "GN_GEMM_WIDE_GROUPED_K": "0"},
                                monkeypatch)
    report(f"wide launches {on} (grouped K off: {off}) of {n_on}")
    assert n_on == n_off and on - off == 3 * cfg.n_layer, (on, off, n_on)


# ---- flash d12 width (the benchmark's flash d12 workload at 6 layers, V 4096) ---
@pytest.fixture(scope="module")
def flashw():
    cfg = flash_width()
    assert (cfg.n_embd, cfg.n_head, cfg.n_kv_head, cfg.compression_ratio) == (768, 6, 1, 4)
    assert (cfg.sparse_topk, cfg.swa_window, cfg.indexer_pool, cfg.indexer_budget) == (16, 512, 8, 128)
    assert cfg.ced and cfg.reuse_pattern == "FRU" and cfg.expert_hidden == 768
    return cfg, G.init_weights(cfg, seed=41, perturb=0.02)


def test_flash_width_rollout_teacher_forced(orc, flashw):
    """64 rows (4 x 16), 600-token prompts: 150 compressed blocks exceed the
    128-candidate budget (hierarchical selection over pools of 8), the
    512-key window is shorter than the prompt (CED's bounded replay), and
    decode attention runs the 6:1 group over the selection and the window."""
    cfg, w = flashw
    _rollout_check(orc, cfg, w, 4, 16, 600, 8, 1.0, groups=(0, 3))


def test_flash_width_pg_step_chunked(orc, flashw, monkeypatch):
    cfg, w = flashw
    _pg_check(orc, cfg, w, B=1, T=560, prompt_len=300, chunk=96, monkeypatch=monkeypatch)


def test_flash_width_pg_step_wide_grouped_k(orc, flashw, monkeypatch):
    """As the latent case at the flash width (experts of 768: 3 x 3 tiles
    per expert), 2 parts per expert's rows."""
    cfg, w = flashw
    monkeypatch.setenv("GN_GEMM_WIDE_MIN", "1")
    monkeypatch.setenv("GN_GEMM_WIDE_PARTS", "2")
    _pg_check(orc, cfg, w, B=1, T=560, prompt_len=300, chunk=96, monkeypatch=monkeypatch)
    monkeypatch.delenv("GN_GEMM_WIDE_PARTS")
    monkeypatch.delenv("GN_GEMM_WIDE_MIN")

"""Pins the oracle's model, RNG and sampler without running the reference:

* the backward by central finite differences on the float64 build
  (model/gradcheck_test.go:14-110 harness, perturbed weights);
* decode == prefill and batched == sequential (model/smear_test.go:30-82);
* engine == recompute under greedy decoding (inference/inference_test.go:306-440);
* Go's PCG stream against numpy's independent PCG64 (LCG transition and
  jump-ahead) and PCG64DXSM (output permutation);
* the top-k threshold against a sort, and sampler properties
  (inference/inference_test.go:11-30);
* the RoPE known answers (model/model_test.go:196-311) on the oracle's own
  rotation and its table's frequencies.
"""
import math

import numpy as np
import pytest

from conftest import assert_close, rel_err
from gonano_amd import config as G


def shape_of(cfg):
    from oracle.oracle import ModelShape
    return ModelShape(cfg.sequence_len, cfg.vocab_size, cfg.n_layer, cfg.n_head, cfg.n_kv_head,
                      cfg.n_embd, cfg.rotary_dims, cfg.window_pattern)


def tiny_cfg(**kw):
    base = dict(sequence_len=16, vocab_size=16, n_layer=2, n_head=2, n_kv_head=2, n_embd=32,
                window_pattern="L", rotary_dims=0)
    base.update(kw)
    return G.Config(**base)


# --------------------------------------------------------------------- RNG --
GO_MUL = 0x2360ED051FC65DA44385DF649FCCF645
GO_INC = (6364136223846793005 << 64) | 1442695040888963407


def test_go_pcg_stream_pinned_by_numpy(orc):
    seed = 12345
    rng = orc.GoRNG(seed)
    hi, lo = rng.hi_lo
    assert hi == seed and lo == seed ^ 0x9E3779B97F4A7C15
    pcg = np.random.PCG64()
    pcg.state = {"bit_generator": "PCG64", "state": {"state": (hi << 64) | lo, "inc": GO_INC},
                 "has_uint32": 0, "uinteger": 0}
    for _ in range(200):
        pcg.random_raw()  # 128-bit LCG step with Go's multiplier and increment
        s = pcg.state["state"]["state"]
        dx = np.random.PCG64DXSM()
        dx.state = {"bit_generator": "PCG64DXSM", "state": {"state": s, "inc": 1},
                    "has_uint32": 0, "uinteger": 0}
        want = int(dx.random_raw())  # DXSM of the pre-iterated state
        assert rng.uint64() == want
        assert rng.hi_lo == (s >> 64, s & ((1 << 64) - 1))


def test_go_pcg_jump_ahead_pinned_by_numpy(orc):
    for n in (1, 7, 65536, 123456789, 2 ** 40 + 3):
        rng = orc.GoRNG(77)
        hi, lo = rng.hi_lo
        pcg = np.random.PCG64()
        pcg.state = {"bit_generator": "PCG64", "state": {"state": (hi << 64) | lo, "inc": GO_INC},
                     "has_uint32": 0, "uinteger": 0}
        pcg.advance(n)
        rng.advance(n)
        s = pcg.state["state"]["state"]
        assert rng.hi_lo == (s >> 64, s & ((1 << 64) - 1))
    # stepping one at a time equals one jump
    a, b = orc.GoRNG(9), orc.GoRNG(9)
    for _ in range(1000):
        a.uint64()
    b.advance(1000)
    assert a.hi_lo == b.hi_lo


def test_float32_mapping(orc):
    """Rand.Float32 takes the low 24 bits of Uint32 = Uint64>>32 (Go's
    math/rand/v2 source; not cross-checked against a Go run here)."""
    a, b = orc.GoRNG(5), orc.GoRNG(5)
    for _ in range(100):
        x = a.uint64()
        assert b.float32() == np.float32(((x >> 32) & 0xFFFFFF) / 2 ** 24)


def test_gumbel_transform(orc):
    L = orc.lib()
    for u in (0.5, 1e-7, 0.999999, 2 ** -24):
        assert L.orc_gumbel_from_uniform(u) == np.float32(-math.log(-math.log(np.float32(u))))
    # u <= 0 becomes 1e-12 (tensors/random.go:69-71)
    assert L.orc_gumbel_from_uniform(0.0) == np.float32(-math.log(-math.log(np.float32(1e-12))))


# ----------------------------------------------------------------- sampler --
def test_kth_largest_with_ties(orc):
    rng = np.random.default_rng(0)
    for trial in range(50):
        n = int(rng.integers(5, 300))
        k = int(rng.integers(1, n))
        v = rng.integers(-5, 5, n).astype(np.float32) if trial % 2 else rng.standard_normal(n).astype(np.float32)
        assert orc.lib().orc_kth_largest(v, n, k) == np.sort(v)[::-1][k - 1]


def test_sampler_properties(orc):  # inference/inference_test.go:11-30
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((64, 500)).astype(np.float32)
    g = orc.GoRNG(3)
    greedy = orc.sample_next_token(logits, g, 0.0, 50)
    assert (greedy == logits.argmax(1)).all()
    assert g.hi_lo == orc.GoRNG(3).hi_lo  # T <= 0 consumes no randomness
    top1 = orc.sample_next_token(logits, orc.GoRNG(4), 1.0, 1)
    assert (top1 == logits.argmax(1)).all()
    s = orc.sample_next_token(logits, orc.GoRNG(5), 1.0, 50)
    thr = np.sort(logits, 1)[:, -50]
    assert (logits[np.arange(64), s] >= thr).all()
    dominant = np.zeros((1, 100), np.float32)
    dominant[0, 7] = 6.0
    g = orc.GoRNG(6)
    picks = [orc.sample_next_token(dominant, g, 1.0, 0)[0] for _ in range(300)]
    assert np.bincount(picks).argmax() == 7


def test_sampler_stream_positions(orc):
    """Every row consumes exactly V draws (masked entries included), so row r
    of a batch uses draws [r*V, (r+1)*V) of the stream."""
    rng = np.random.default_rng(2)
    V = 257
    logits = rng.standard_normal((5, V)).astype(np.float32)
    batched = orc.sample_next_token(logits, orc.GoRNG(11), 1.0, 13)
    for r in range(5):
        g = orc.GoRNG(11)
        g.advance(r * V)
        assert orc.sample_next_token(logits[r:r + 1], g, 1.0, 13)[0] == batched[r]
    g = orc.GoRNG(11)
    orc.sample_next_token(logits, g, 1.0, 13)
    h = orc.GoRNG(11)
    h.advance(5 * V)
    assert g.hi_lo == h.hi_lo


# ------------------------------------------------------------------- model --
def test_rope_known_answers(orc):
    """The oracle's RoPE (the function its model rotates with) against the
    reference's known answers: a quarter turn of [3, 4] at position 1 gives
    [4, -3] (model/model_test.go:196-211); with D = 4 and R = 2 the leading
    channels stay and the trailing pair turns, [10, 20, 3, 4] -> [10, 20, 4,
    -3] (:283-300).  Then its table: rotation preserves each head's norm
    (:302-311); the angle of column j at position p is p * 100000^(-2j/R)
    (rotary.go:10,16-30: base 100000, frequencies over the rotary width, not
    the head width), read back through atan2, which a wrong base, a
    transposed table or a half-split at the wrong offset fails."""
    cos_row, sin_row = np.array([0.0], np.float32), np.array([1.0], np.float32)
    got = orc.apply_rotary(np.array([[3.0, 4.0]], np.float32), cos_row, sin_row)
    assert got.tolist() == [[4.0, -3.0]]
    got = orc.apply_rotary(np.array([[10.0, 20.0, 3.0, 4.0]], np.float32), cos_row, sin_row)
    assert got.tolist() == [[10.0, 20.0, 4.0, -3.0]]
    # two heads: each rotates on its own trailing pair
    got = orc.apply_rotary(np.array([[1, 2, 3, 4], [5, 6, 7, 8]], np.float32), cos_row, sin_row)
    assert got.tolist() == [[1, 2, 4, -3], [5, 6, 8, -7]]
    # norm preservation with the real table (R = D = 8, 32 positions)
    c, sn = orc.rotary_table(32, 8)
    x = np.random.default_rng(3).standard_normal((2, 8)).astype(np.float32)
    for p in range(32):
        y = orc.apply_rotary(x, c[p], sn[p])
        assert np.allclose(np.linalg.norm(y, axis=1), np.linalg.norm(x, axis=1), rtol=1e-6)
    # the frequencies: partial RoPE over R = 64 of a 128-wide head
    c, sn = orc.rotary_table(8, 64)
    assert c.shape == (8, 32)
    assert np.all(c[0] == 1) and np.all(sn[0] == 0)
    ang = np.arctan2(sn[1].astype(np.float64), c[1].astype(np.float64))
    want = 100000.0 ** (-2.0 * np.arange(32) / 64.0)
    assert np.allclose(ang, want, rtol=1e-6, atol=1e-7)
    assert abs(ang[0] - 1.0) < 1e-7 and abs(ang[16] - 100000.0 ** -0.5) < 1e-9
    # a position's angles are that multiple of position 1's (mod 2 pi)
    ang5 = np.arctan2(sn[5].astype(np.float64), c[5].astype(np.float64))
    assert np.allclose(np.cos(ang5), np.cos(5 * want), atol=1e-6)
    # rotation by p then by q equals rotation by p + q (rotations compose)
    big_c, big_s = orc.rotary_table(16, 8)
    y = orc.apply_rotary(orc.apply_rotary(x, big_c[3], big_s[3]), big_c[4], big_s[4])
    assert np.allclose(y, orc.apply_rotary(x, big_c[7], big_s[7]), atol=1e-5)
    # the config side: R defaults to the head width and must be even and <= D
    cfg = tiny_cfg()
    assert cfg.rotary_dimension == 16
    assert G.Config(16, 16, 1, 4, 4, 32, "L", 4).rotary_dimension == 4
    with pytest.raises(ValueError):
        _ = G.Config(16, 16, 1, 4, 4, 32, "L", 10).rotary_dimension
    with pytest.raises(ValueError):
        _ = G.Config(16, 16, 1, 4, 4, 32, "L", 3).rotary_dimension


def test_window_sizes():
    assert G.dense_d12().window_sizes() == [128, 128, 128, 512] * 3
    assert G.dense_d2().window_sizes() == [128, 512]
    assert G.Config(256, 16, 2, 1, 1, 128, "SSSL", 64).window_sizes() == [0, 256]
    assert G.dense_d20().window_sizes()[:4] == [512, 512, 512, 2048]


@pytest.mark.parametrize("kw", [dict(), dict(n_head=4, n_kv_head=2, rotary_dims=4, n_layer=3)])
def test_decode_equals_prefill(orc, kw):
    cfg = tiny_cfg(**kw)
    w = G.init_weights(cfg, seed=1, perturb=0.1)
    m = orc.OracleModel(shape_of(cfg), w)
    ids = np.random.default_rng(4).integers(0, cfg.vocab_size, (2, 9)).astype(np.int32)
    full = m.forward(ids)
    assert_close(m.forward_decode(ids, 1), full, 1e-4, 1e-5, "token-by-token decode")
    assert_close(m.forward_decode(ids, 4), full, 1e-4, 1e-5, "chunked decode")
    # batched == sequential
    for b in range(2):
        assert_close(m.forward(ids[b:b + 1])[0], full[b], 1e-5, 1e-6, "row")


def _fd_check(orc, cfg, loss_fn, n_elem=3, seed=7):
    w = G.init_weights(cfg, seed=1, perturb=0.1).astype(np.float64)
    m = orc.OracleModel(shape_of(cfg), w, dtype=np.float64)
    base, grads = loss_fn(m)
    rng = np.random.default_rng(seed)
    # directional derivative over every parameter
    d = rng.standard_normal(w.size)
    d /= np.linalg.norm(d)
    eps = 1e-5
    lp = loss_fn(orc.OracleModel(shape_of(cfg), w + eps * d, dtype=np.float64), False)[0]
    lm = loss_fn(orc.OracleModel(shape_of(cfg), w - eps * d, dtype=np.float64), False)[0]
    num = (lp - lm) / (2 * eps)
    ana = float(grads @ d)
    assert abs(num - ana) <= 1e-6 * max(1.0, abs(ana)), (num, ana)
    # a few elements of every tensor
    for name, r, c, off in cfg.param_table():
        for j in rng.choice(r * c, size=min(n_elem, r * c), replace=False):
            e = np.zeros_like(w)
            e[off + j] = eps
            lp = loss_fn(orc.OracleModel(shape_of(cfg), w + e, dtype=np.float64), False)[0]
            lm = loss_fn(orc.OracleModel(shape_of(cfg), w - e, dtype=np.float64), False)[0]
            num = (lp - lm) / (2 * eps)
            assert abs(num - grads[off + j]) <= 1e-6 * max(1e-2, abs(num)) + 1e-9, \
                (name, j, num, grads[off + j])


@pytest.mark.parametrize("kw", [dict(), dict(n_head=4, n_kv_head=2, rotary_dims=4, n_layer=3)])
def test_ce_backward_finite_differences(orc, kw):
    cfg = tiny_cfg(**kw)
    ids = np.array([[1, 5, 2, 8, 3, 7]], np.int32)  # gradcheck_test.go:87-91
    tg = np.array([[5, 2, 8, 3, 7, 4]], np.int32)

    def loss_fn(m, want=True):
        return m.ce_loss(ids, tg, want)

    _fd_check(orc, cfg, loss_fn)


def test_pg_backward_finite_differences(orc):
    cfg = tiny_cfg(n_head=4, n_kv_head=1, rotary_dims=8, n_layer=2, vocab_size=24)
    rng = np.random.default_rng(8)
    ids = rng.integers(0, 24, (3, 7)).astype(np.int32)
    tg = rng.integers(0, 24, (3, 7)).astype(np.int32)
    tg[:, :3] = -1
    adv = np.array([0.7, -0.2, -0.5], np.float32)

    def loss_fn(m, want=True):
        loss, nll, g = m.pg_step(ids, tg, adv, 8.0)
        return loss, g

    _fd_check(orc, cfg, loss_fn, n_elem=2)


def test_pg_loss_closed_form(orc):
    """loss = sum_valid nll*adv/norm, nll = lse - z_t (trainer/rl.go:25-35)."""
    cfg = tiny_cfg(vocab_size=20)
    w = G.init_weights(cfg, seed=2, perturb=0.1)
    m = orc.OracleModel(shape_of(cfg), w, dtype=np.float64)
    rng = np.random.default_rng(9)
    ids = rng.integers(0, 20, (2, 6)).astype(np.int32)
    tg = rng.integers(0, 20, (2, 6)).astype(np.int32)
    tg[0, :2] = -1
    adv = np.array([0.25, -0.25], np.float32)
    loss, nll, _ = m.pg_step(ids, tg, adv, 6.0)
    z = m.forward(ids).astype(np.float64)
    lse = np.log(np.exp(z).sum(-1))
    want_nll = np.where(tg >= 0, lse - np.take_along_axis(z, np.maximum(tg, 0)[..., None], -1)[..., 0], 0)
    assert_close(nll, want_nll, 1e-12, 1e-12)
    assert abs(loss - (want_nll * adv[:, None].astype(np.float64) / 6.0).sum()) < 1e-12


def test_engine_matches_recompute_greedy(orc):
    """inference/inference_test.go:306-440: greedy KV-cache decoding
    reproduces a no-cache recompute token for token."""
    cfg = tiny_cfg(vocab_size=300, sequence_len=64, n_head=4, n_kv_head=2, rotary_dims=4)
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    m = orc.OracleModel(shape_of(cfg), w)
    prompt = np.array([1, 7, 3, 9, 2], np.int32)
    rows = m.generate_batch(prompt, 3, 12, 0.0, 0, 0)
    for r in rows:
        assert (r[:5] == prompt).all()
        full = m.forward(r[None, :].astype(np.int32))[0]
        for t in range(5, len(r)):
            assert full[t - 1].argmax() == r[t]


def test_generate_uses_group_stream(orc):
    """Sampled columns equal SampleNextToken on the engine's own logits with
    the stream advanced by S*V per column (inference/engine.go:238-256)."""
    cfg = tiny_cfg(vocab_size=300, sequence_len=64)
    w = G.init_weights(cfg, seed=4, perturb=0.1)
    m = orc.OracleModel(shape_of(cfg), w)
    prompt = np.array([4, 4, 8], np.int32)
    S, N, seed = 4, 6, 17
    rows = m.generate_batch(prompt, S, N, 1.0, 50, seed)
    g = orc.GoRNG(seed)
    ids = np.stack([np.concatenate([r, np.zeros(3 + N - len(r), np.int32)]) for r in rows])
    for t in range(N):
        z = m.forward(ids[:, :3 + t])[:, -1, :]
        want = orc.sample_next_token(z, g, 1.0, 50)
        live = [s for s in range(S) if len(rows[s]) > 3 + t]
        for s in live:
            assert rows[s][3 + t] == want[s]


def test_advantages_and_padding(orc):
    """cmd/chat_rl/main.go:139-180 closed form on a tiny model."""
    cfg = tiny_cfg(vocab_size=300, sequence_len=64)
    w = G.init_weights(cfg, seed=5, perturb=0.1)
    m = orc.OracleModel(shape_of(cfg), w)
    prompts = np.array([[1, 2, 3], [4, 5, 6]], np.int32)
    rewards = np.array([1, 0, 0, 1, 1, 1], np.float32)
    out = m.rl_step(prompts, 3, 5, 1.0, 50, np.array([0, 1], np.uint64), rewards)
    assert_close(out["adv"], [2 / 3, -1 / 3, -1 / 3, 0, 0, 0], 1e-6, 1e-7)
    maxlen = max(len(r) for r in out["rows"])
    assert out["max_len"] == maxlen
    for b, r in enumerate(out["rows"]):
        padded = np.concatenate([r, np.full(maxlen - len(r), 260, np.int32)])
        assert (out["inputs"][b] == padded[:-1]).all()
        tg = padded[1:].copy()
        tg[:3] = -1
        assert (out["targets"][b] == tg).all()


@pytest.mark.parametrize("temperature,top_k", [(1.0, 50), (0.7, 5)])
def test_decode_forced_reproduces_generate(orc, temperature, top_k):
    """The teacher-forced checker is itself pinned: sampling every step of a
    group from orc_decode_forced's logits (the rows' own columns fed) with
    the group stream reproduces the oracle's own generate_batch rows, and its
    step logits equal the full forward's at the same positions (decode ==
    prefill)."""
    from tf_check import teacher_forced_group
    cfg = G.Config(sequence_len=512, vocab_size=300, n_layer=2, n_head=2, n_kv_head=1,
                   n_embd=64, window_pattern="SSSL", rotary_dims=32)
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    m = orc.OracleModel(shape_of(cfg), w)
    prompt = np.random.default_rng(4).integers(0, 256, 20).astype(np.int32)
    rows = m.generate_batch(prompt, 6, 12, temperature, top_k, 99)
    assert teacher_forced_group(orc, m, prompt, rows, 99, 12, temperature, top_k) > 30
    # a wrong stream position is caught
    with pytest.raises(AssertionError):
        teacher_forced_group(orc, m, prompt, rows, 98, 12, temperature, top_k)
    full = [r for r in rows if len(r) == 32]
    if full:
        cols = np.stack([r[20:31] for r in full], 1)
        z = m.decode_forced(prompt, cols)
        ref = m.forward(np.stack(full)[:, :31])
        for i in range(len(full)):
            assert rel_err(z[:, i, :], ref[i, 19:31, :]) < 1e-5

"""Pins the oracle's compressed attention (HCA: ChannelCompressor + block-causal
attention over compressed keys + sliding-window local branch merged by
log-sum-exp) without running the reference:

* the compressor's known answer (model/compress_test.go:10-26) and two
  special cases the softmax fixes: a shift of one block's logits changes
  nothing, and one dominant logit per channel selects that row's value;
* the branch merge equals one attention over the concatenated keys
  (model/swa_test.go:14-136), forward, against a float64 numpy attention;
* the model backward by central finite differences on the float64 build,
  with and without the local branch (model/swa_test.go:138-140), every
  parameter including the compressor's;
* decode against the compressed cache == the training forward, token by
  token and chunked, across several blocks and the window;
* the block rule: without a local branch a position sees only blocks that
  ended before its own block, so perturbing an earlier token of the same
  block (beyond the smear gate's previous-token reach) leaves its logits
  unchanged, while perturbing a token of the previous block does not;
* the local branch participates (model/swa_test.go:203-260).
"""
import numpy as np
import pytest

from gonano_amd import config as G


def flash_cfg(swa=3, ratio=2, seq=16, vocab=16, n_layer=2, kv=2, head=2, embd=32, window="L"):
    # tinySWAModel's configuration (model/swa_test.go:120-136)
    return G.Config(sequence_len=seq, vocab_size=vocab, n_layer=n_layer, n_head=head,
                    n_kv_head=kv, n_embd=embd, window_pattern=window,
                    compression_ratio=ratio, swa_window=swa)


def oracle_model(orc, cfg, w, dtype=np.float32):
    return orc.OracleModel(orc.ModelShape.from_config(cfg), w, dtype)


def compress(orc, logits, value, ratio):
    T, D = value.shape
    blocks = -(-T // ratio)
    comp = np.zeros((blocks, D), np.float32)
    probs = np.zeros((blocks, ratio, D), np.float32)
    orc.lib().orc_channel_compress(T, D, ratio, np.ascontiguousarray(logits, np.float32),
                                 np.ascontiguousarray(value, np.float32), comp, probs)
    return comp, probs


def test_compressor_means_blocks(orc):
    # zero logits: complete blocks are means, a trailing partial block keeps its row
    comp, _ = compress(orc, np.zeros((3, 1)), np.array([[2.0], [4.0], [6.0]]), 2)
    assert comp.ravel().tolist() == [3.0, 6.0]


def test_compressor_softmax_special_cases(orc):
    rng = np.random.default_rng(0)
    T, D, r = 11, 6, 4
    logits = rng.standard_normal((T, D)).astype(np.float32)
    value = rng.standard_normal((T, D)).astype(np.float32)
    base, probs = compress(orc, logits, value, r)
    assert base.shape == (3, D)
    # probabilities of each block and channel sum to one over the block's rows
    assert np.allclose(probs.sum(1), 1, atol=1e-6)
    # a per-channel shift of one block's logits is invisible to the softmax
    shifted = logits.copy()
    shifted[4:8] += rng.standard_normal(D).astype(np.float32) * 3
    got, _ = compress(orc, shifted, value, r)
    assert np.allclose(got, base, atol=1e-5)
    # a dominant logit selects its row's value, channel by channel
    pick = rng.integers(0, r, D)
    dom = logits.copy()
    for d in range(D):
        dom[4 + pick[d], d] = 200.0
    got, _ = compress(orc, dom, value, r)
    assert np.array_equal(got[1], value[4 + pick, np.arange(D)])


def _attn64(q, k, v):
    s = q.astype(np.float64) @ k.astype(np.float64).T / np.sqrt(q.shape[1])
    m = s.max(1, keepdims=True)
    p = np.exp(s - m)
    z = p.sum(1, keepdims=True)
    return (p / z) @ v.astype(np.float64), (m + np.log(z)).ravel()


def test_merge_equals_concatenated_attention(orc):
    rng = np.random.default_rng(7)
    Q, D, ka, kb = 5, 8, 6, 4
    q = rng.standard_normal((Q, D))
    k = rng.standard_normal((ka + kb, D))
    v = rng.standard_normal((ka + kb, D))
    oa, la = _attn64(q, k[:ka], v[:ka])
    ob, lb = _attn64(q, k[ka:], v[ka:])
    want_o, want_l = _attn64(q, k, v)
    out = np.zeros((Q, D), np.float32)
    lse = np.zeros(Q, np.float32)
    f = lambda a: np.ascontiguousarray(a, np.float32)
    orc.lib().orc_merge_attention_rows(out, lse, f(oa), f(la), f(ob), f(lb), Q, D)
    assert np.abs(out - want_o).max() < 1e-6 * max(1, np.abs(want_o).max()) * 10
    assert np.abs(lse - want_l).max() < 1e-5
    # an empty branch (log-sum-exp -inf, as a query before the first complete
    # block has) leaves the other one unchanged
    orc.lib().orc_merge_attention_rows(out, lse, f(np.zeros_like(oa)), f(np.full(Q, -np.inf)),
                                     f(ob), f(lb), Q, D)
    assert np.array_equal(out, f(ob)) and np.array_equal(lse, f(lb))


@pytest.mark.parametrize("swa,ratio,kv", [(3, 2, 2), (0, 2, 2), (6, 4, 1)])
def test_flash_gradients_match_finite_differences(orc, swa, ratio, kv):
    cfg = flash_cfg(swa=swa, ratio=ratio, kv=kv, head=2 if kv == 2 else 4)
    w = G.init_weights(cfg, seed=7, perturb=0.1).astype(np.float64)
    sh = orc.ModelShape.from_config(cfg)
    rng = np.random.default_rng(1)
    ids = rng.integers(0, cfg.vocab_size, (2, 13)).astype(np.int32)  # ragged last block
    tg = rng.integers(0, cfg.vocab_size, (2, 13)).astype(np.int32)
    tg[:, :2] = -1
    _, g = orc.OracleModel(sh, w, np.float64).ce_loss(ids, tg)

    def total(wv):
        return orc.OracleModel(sh, wv, np.float64).ce_loss(ids, tg, want_grads=False)[0]

    eps = 1e-6
    d = rng.standard_normal(w.size)
    fd = (total(w + eps * d) - total(w - eps * d)) / (2 * eps)
    an = float(g @ d)
    assert abs(fd - an) <= 1e-6 * abs(an), (fd, an)
    tab = orc.param_table(sh)
    assert any(n.endswith("attn.compress_logits.weight") for n, *_ in tab)
    for name, r, c, off in tab:
        for i in off + rng.integers(0, r * c, 2):
            e = np.zeros_like(w)
            e[i] = 1
            fdv = (total(w + eps * e) - total(w - eps * e)) / (2 * eps)
            assert abs(fdv - g[i]) <= 1e-7 + 1e-5 * abs(g[i]), (name, int(i - off), fdv, g[i])


@pytest.mark.parametrize("swa", [6, 0])
@pytest.mark.parametrize("chunk", [1, 5])
def test_compressed_decode_matches_training_forward(orc, swa, chunk):
    cfg = flash_cfg(swa=swa, ratio=4, seq=64, vocab=40, kv=2, head=4, embd=64, window="SL")
    cfg.rotary_dims = 8
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    m = oracle_model(orc, cfg, w)
    ids = np.random.default_rng(0).integers(0, cfg.vocab_size, (2, 23)).astype(np.int32)
    full = m.forward(ids)
    dec = m.forward_decode(ids, chunk)
    assert np.abs(full - dec).max() <= 2e-6 * np.abs(full).max()


def test_block_rule_without_local_branch(orc):
    cfg = flash_cfg(swa=0, ratio=4, seq=32, vocab=24, n_layer=1)
    w = G.init_weights(cfg, seed=11, perturb=0.2).astype(np.float64)
    m = oracle_model(orc, cfg, w, np.float64)
    ids = np.random.default_rng(3).integers(0, cfg.vocab_size, (1, 12)).astype(np.int32)
    base = m.forward(ids)
    same = ids.copy()
    same[0, 8] = (same[0, 8] + 1) % cfg.vocab_size  # block 2, earlier than position 10
    a = m.forward(same)
    assert np.array_equal(a[0, 10], base[0, 10]) and np.array_equal(a[0, 11], base[0, 11])
    assert np.abs(a[0, 8] - base[0, 8]).max() > 0  # its own position still changes
    prev = ids.copy()
    prev[0, 5] = (prev[0, 5] + 1) % cfg.vocab_size  # block 1: compressed into block 2's keys
    b = m.forward(prev)
    assert np.abs(b[0, 10] - base[0, 10]).max() > 1e-9
    # same block, two positions later (one later sees it through the smear
    # gate's previous-token mix, transformer.go:268-275): not visible
    assert np.array_equal(b[0, 7], base[0, 7])


def test_local_branch_is_active(orc):
    base = flash_cfg(swa=0)
    with_swa = flash_cfg(swa=3)
    w = G.init_weights(base, seed=42, perturb=0.1)
    assert w.size == with_swa.param_total()  # the local branch has no parameters
    ids = np.array([[1, 5, 2, 8]], np.int32)
    a = oracle_model(orc, base, w).forward(ids)
    b = oracle_model(orc, with_swa, w).forward(ids)
    assert not np.array_equal(a, b)

"""Pins the oracle's sparse compressed attention (CSA: lightning-indexer
scores, hierarchical top-k selection, attention over the selected compressed
blocks, the indexer's distillation gradient) and cross-layer reuse (FRU:
Full / Reindex / Reuse layers sharing a group's compressed KV, candidate pool
and selection) without running the reference:

* the selection's known answers from model/indexer_test.go (tie-breaking,
  causality, block-max coarse stage, pool restriction), top-k against an
  independent stable sort with many ties, and its invariants (unbounded
  budget == flat selection, pool bounded by the budget, fine selection
  within the pool reproduces the selection);
* a closed form: with top-k at least the number of allowed blocks the sparse
  layer attends every allowed block, so the model equals the dense
  compressed model with the same weights;
* the backward by central finite differences on the float64 build of CE +
  the distillation objective with the targets held constant (the reference's
  gradient treats them as constants, compress_attention.go:133-147), for
  flat and hierarchical indexers, with and without reuse;
* decode against the caches == the training forward, token by token and
  chunked (compressed blocks, cached indexer keys, Reindex layers' own key
  caches, published pools and selections).
"""
import numpy as np
import pytest

from gonano_amd import config as G


def lib(orc):
    return orc.lib()


def topk(orc, v, k):
    v = np.ascontiguousarray(v, np.float32)
    out = np.zeros(max(len(v), 1), np.int32)
    n = lib(orc).orc_indexer_topk(v, len(v), k, out)
    return out[:n].tolist()


def select_rows(orc, scores, offset, ratio, k, pool, budget):
    scores = np.ascontiguousarray(scores, np.float32)
    T, blocks = scores.shape
    gpt = max(1, -(-budget // max(pool, 1)))
    ccap = gpt * max(pool, 1)
    sel = np.zeros((T, max(k, 1)), np.int32)
    nsel = np.zeros(T, np.int32)
    cand = np.zeros((T, ccap), np.int32)
    ncand = np.zeros(T, np.int32)
    lib(orc).orc_select_rows(scores, T, blocks, offset, ratio, k, pool, budget, max(k, 1), ccap,
                             sel, nsel, cand.ctypes.data, ncand.ctypes.data)
    return ([sel[t, :nsel[t]].tolist() for t in range(T)],
            [cand[t, :ncand[t]].tolist() for t in range(T)])


def test_topk_matches_stable_sort_with_ties(orc):
    rng = np.random.default_rng(2024)
    for n in (0, 1, 2, 5, 16, 64, 257, 1000):
        v = np.trunc(rng.standard_normal(n) * 4).astype(np.float32)  # many ties
        order = np.argsort(-v, kind="stable").tolist()
        for k in (-1, 0, 1, 3, n // 2, n, n + 5):
            assert topk(orc, v, k) == order[:max(k, 0)], (n, k)
    assert topk(orc, [5, 5, 5, 1, 2], 2) == [0, 1]  # indexer_test.go:318-325


def test_select_blocks_causality_and_ties(orc):
    # indexer_test.go:413-435: 5 tokens, 4 blocks, ratio 2, top-2
    scores = np.array([[1, 2, 3, 4], [5, 1, 2, 3], [1, 1, 9, 1], [1, 1, 1, 8], [7, 7, 7, 7]])
    sel, _ = select_rows(orc, scores, 0, 2, 2, 1, 1000)
    assert sel[0] == [] and sel[1] == []
    assert sel[2] == [0] and sel[3] == [0]
    assert sel[4] == [0, 1]


def test_block_max_coarse_stage(orc):
    # indexer_test.go:351-365: row {4,0,3,3}, super-blocks of 2 -> maxima
    # [4, 3]: the first group wins although the second has the higher mean
    sel, pool = select_rows(orc, [[4, 0, 3, 3]], 4, 1, 1, 2, 2)
    assert pool[0] == [0, 1] and sel[0] == [0]


def test_restrict_to_pool(orc):
    # indexer_test.go:367-396
    scores = np.array([[1, 2, 3, 4], [5, 6, 7, 8]], np.float32)
    target = np.array([[0.1, 0.2, 0.3, 0.4], [0.25, 0.25, 0.25, 0.25]], np.float32)
    pool = np.array([[1, 3], [0, 2]], np.int32)
    lib(orc).orc_restrict_to_pool(scores, target, 2, 4, pool, np.array([2, 2], np.int32), 2)
    assert np.isneginf(scores[0, [0, 2]]).all() and (target[0, [0, 2]] == 0).all()
    assert abs(target[0, 1] - 1 / 3) < 1e-6 and abs(target[0, 3] - 2 / 3) < 1e-6
    assert scores[0, 1] == 2 and scores[0, 3] == 4
    assert np.isneginf(scores[1, [1, 3]]).all() and scores[1, 0] == 5 and scores[1, 2] == 7


def _scores(orc, rng, T, blocks, H=2, dim=3):
    iq = rng.standard_normal((T, H * dim)).astype(np.float32)
    ik = rng.standard_normal((blocks, H * dim)).astype(np.float32)
    w = rng.standard_normal(H).astype(np.float32)
    out = np.zeros((T, blocks), np.float32)
    lib(orc).orc_indexer_scores_rows(iq, ik, w, T, blocks, H, dim, out)
    # IndexerScores restated independently: sum_h w_h ReLU(q_h . k_h)
    dots = np.einsum("thd,shd->tsh", iq.reshape(T, H, dim).astype(np.float64),
                     ik.reshape(blocks, H, dim).astype(np.float64))
    want = (np.maximum(dots, 0) * w.astype(np.float64)).sum(-1)
    assert np.abs(out - want).max() < 1e-5 * max(1, np.abs(want).max())
    return iq, ik, w, out


def test_hierarchical_equals_flat_when_unbounded(orc):
    rng = np.random.default_rng(7)
    _, _, _, sc = _scores(orc, rng, 12, 6)
    flat, _ = select_rows(orc, sc, 0, 2, 2, 1, 1000)
    for pool in (1, 2, 3):
        hier, cand = select_rows(orc, sc, 0, 2, 2, pool, 1000)
        assert hier == flat
        for t, c in enumerate(cand):  # every allowed block is a candidate
            assert sorted(c) == list(range(min(t // 2, 6)))


def test_pool_bounded_by_budget_and_causal(orc):
    rng = np.random.default_rng(9)
    _, _, _, sc = _scores(orc, rng, 6 * 1 + 200, 64)
    sel, pool = select_rows(orc, sc, 0, 2, 4, 4, 8)
    for t, (s, c) in enumerate(zip(sel, pool)):
        allowed = min(t // 2, 64)
        assert len(c) <= 8 and all(0 <= b < allowed for b in c)
        assert set(s) <= set(c) and len(s) == min(4, len(c))


def test_fine_select_within_pool_reproduces_selection(orc):
    # indexer_test.go:183-210 (SelectWithinPool == the fine stage)
    rng = np.random.default_rng(3)
    T, blocks, H, dim = 40, 19, 2, 3
    iq, ik, w, sc = _scores(orc, rng, T, blocks, H, dim)
    sel, pool = select_rows(orc, sc, 0, 2, 2, 2, 3)
    for t in range(T):
        c = np.array(pool[t] or [0], np.int32)
        out = np.zeros(2, np.int32)
        n = np.zeros(1, np.int32)
        lib(orc).orc_fine_select(np.ascontiguousarray(iq[t]), ik, w, H, dim, c, len(pool[t]), 2,
                                 min(t // 2, blocks), out, n)
        assert out[:n[0]].tolist() == sel[t]


def csa_cfg(topk=2, pool=1, budget=0, reuse="", swa=3, ratio=2, n_layer=2, kv=2, head=2,
            seq=32, vocab=24, embd=32, heads=1, dim=8):
    return G.Config(sequence_len=seq, vocab_size=vocab, n_layer=n_layer, n_head=head,
                    n_kv_head=kv, n_embd=embd, window_pattern="L", compression_ratio=ratio,
                    swa_window=swa, sparse_topk=topk, indexer_pool=pool,
                    indexer_candidates=budget, reuse_pattern=reuse, indexer_heads=heads,
                    indexer_dim=dim)


def test_param_table_roles(orc):
    cfg = csa_cfg(reuse="FRU", n_layer=3, pool=2, budget=4)
    tab = orc.param_table(orc.ModelShape.from_config(cfg))
    assert [tuple(t) for t in tab] == [tuple(t) for t in cfg.param_table()]
    names = {t[0] for t in tab}
    assert "transformer.h.0.attn.compress_logits.weight" in names       # F: compressor
    assert "transformer.h.0.attn.indexer_query.weight" in names         # F: indexer
    assert "transformer.h.1.attn.compress_logits.weight" not in names   # R: no compressor
    assert "transformer.h.1.attn.indexer_key.weight" in names           # R: own indexer
    assert not any(n.startswith("transformer.h.2.attn.indexer") for n in names)  # U: neither
    assert [cfg.reuse_producer(l) for l in range(3)] == [0, 0, 0]


def test_full_topk_equals_dense_compressed(orc):
    """top-k >= every row's allowed block count: the sparse layers attend
    every allowed block, so the logits equal the dense compressed model's
    (same shared weights; softmax over the same set in another order)."""
    sparse = csa_cfg(topk=64)
    dense = csa_cfg(topk=0)
    ws = G.init_weights(sparse, seed=5, perturb=0.1)
    wd = np.zeros(dense.param_total(), np.float32)
    ss, sd = sparse.param_slices(), dense.param_slices()
    for name, (off, r, c) in sd.items():
        o2 = ss[name][0]
        wd[off:off + r * c] = ws[o2:o2 + r * c]
    ids = np.random.default_rng(1).integers(0, sparse.vocab_size, (2, 21)).astype(np.int32)
    a = orc.OracleModel(orc.ModelShape.from_config(sparse), ws.astype(np.float64), np.float64).forward(ids)
    b = orc.OracleModel(orc.ModelShape.from_config(dense), wd.astype(np.float64), np.float64).forward(ids)
    assert np.abs(a - b).max() < 1e-12 * max(1, np.abs(b).max())
    # and a top-1 selection really drops blocks
    one = csa_cfg(topk=1)
    c = orc.OracleModel(orc.ModelShape.from_config(one), ws.astype(np.float64), np.float64).forward(ids)
    assert np.abs(c - b).max() > 1e-6


FD_CASES = {
    "flat": dict(topk=2, pool=1),
    "hier_fru": dict(topk=2, pool=2, budget=4, reuse="FRU", n_layer=3),
    "dense_fu": dict(topk=0, reuse="FU", n_layer=3),
    "hier_noswa_gqa": dict(topk=3, pool=2, budget=4, swa=0, kv=1, head=2, heads=2, dim=4),
}


@pytest.mark.parametrize("case", list(FD_CASES))
def test_csa_gradients_match_finite_differences(orc, case):
    cfg = csa_cfg(**FD_CASES[case])
    w = G.init_weights(cfg, seed=7, perturb=0.1).astype(np.float64)
    sh = orc.ModelShape.from_config(cfg)
    rng = np.random.default_rng(1)
    ids = rng.integers(0, cfg.vocab_size, (2, 13)).astype(np.int32)
    tg = rng.integers(0, cfg.vocab_size, (2, 13)).astype(np.int32)
    tg[:, :2] = -1
    m = orc.OracleModel(sh, w, np.float64)
    m.freeze_targets(1)  # record the distillation targets at w
    _, g = m.ce_loss(ids, tg)
    m.freeze_targets(2)

    def total(wv):
        m.set_params(wv)
        loss, _ = m.ce_loss(ids, tg, want_grads=False)
        return loss + m.distill_loss()

    eps = 1e-6
    d = rng.standard_normal(w.size)
    fd = (total(w + eps * d) - total(w - eps * d)) / (2 * eps)
    an = float(g @ d)
    assert abs(fd - an) <= 1e-6 * abs(an), (fd, an)
    tab = orc.param_table(sh)
    for name, r, c, off in tab:
        if "indexer" in name:  # trained by the distillation alone
            assert np.any(g[off:off + r * c]), name
        for i in off + rng.integers(0, r * c, 2):
            e = np.zeros_like(w)
            e[i] = 1
            fdv = (total(w + eps * e) - total(w - eps * e)) / (2 * eps)
            assert abs(fdv - g[i]) <= 1e-7 + 1e-5 * abs(g[i]), (name, int(i - off), fdv, g[i])


DECODE_CASES = {
    "flat": dict(topk=3, pool=1, ratio=4, swa=6),
    "hier_fru": dict(topk=2, pool=2, budget=4, reuse="FRU", n_layer=3, ratio=2, swa=5),
    "hier_noswa": dict(topk=2, pool=3, budget=6, reuse="FR", n_layer=3, ratio=2, swa=0),
    "dense_fu": dict(topk=0, reuse="FU", n_layer=3, ratio=3, swa=4),
}


@pytest.mark.parametrize("chunk", [1, 5])
@pytest.mark.parametrize("case", list(DECODE_CASES))
def test_csa_decode_matches_training_forward(orc, case, chunk):
    cfg = csa_cfg(seq=64, vocab=40, embd=64, head=4, **DECODE_CASES[case])
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    m = orc.OracleModel(orc.ModelShape.from_config(cfg), w)
    ids = np.random.default_rng(0).integers(0, cfg.vocab_size, (2, 37)).astype(np.int32)
    full = m.forward(ids)
    dec = m.forward_decode(ids, chunk)
    assert np.abs(full - dec).max() <= 2e-6 * np.abs(full).max()


# ---- CED: causal encoder-decoder split (model/transformer.go:363-449) -------
def ced_cfg(**kw):
    # cedBaseConfig (model/ced_test.go:12-17): four layers split 2 + 2
    base = dict(topk=0, ratio=2, swa=3, n_layer=4, kv=2, head=2, seq=16, vocab=16, embd=32, dim=4)
    base.update(kw)
    cfg = csa_cfg(**base)
    cfg.ced = True
    cfg.validate()
    return cfg


def test_ced_roles(orc):
    cfg = ced_cfg(reuse="FR", topk=2)
    assert cfg.ced_split == 2
    # the reuse pattern restarts at the split: each half starts with a Full layer
    assert [cfg.reuse_mode_at(l) for l in range(4)] == ["F", "R", "F", "R"]
    assert [cfg.reuse_producer(l) for l in range(4)] == [0, 0, 2, 2]
    tab = orc.param_table(orc.ModelShape.from_config(cfg))
    assert [tuple(t) for t in tab] == [tuple(t) for t in cfg.param_table()]


CED_FD = {
    "dense": dict(),
    "reindex": dict(reuse="FR", topk=2, pool=2, budget=4),
    "fru_sparse": dict(reuse="FRU", topk=2, n_layer=6, swa=4),
}


@pytest.mark.parametrize("case", list(CED_FD))
def test_ced_gradients_match_finite_differences(orc, case):
    """ced_test.go:117-125: the backward through the split, including the
    decoder's global-KV gradient injected into the encoder output."""
    cfg = ced_cfg(**CED_FD[case])
    w = G.init_weights(cfg, seed=11, perturb=0.1).astype(np.float64)
    sh = orc.ModelShape.from_config(cfg)
    rng = np.random.default_rng(4)
    ids = rng.integers(0, cfg.vocab_size, (2, 11)).astype(np.int32)
    tg = rng.integers(0, cfg.vocab_size, (2, 11)).astype(np.int32)
    tg[:, :2] = -1
    m = orc.OracleModel(sh, w, np.float64)
    m.freeze_targets(1)
    _, g = m.ce_loss(ids, tg)
    m.freeze_targets(2)

    def total(wv):
        m.set_params(wv)
        loss, _ = m.ce_loss(ids, tg, want_grads=False)
        return loss + m.distill_loss()

    eps = 1e-6
    d = rng.standard_normal(w.size)
    fd = (total(w + eps * d) - total(w - eps * d)) / (2 * eps)
    an = float(g @ d)
    assert abs(fd - an) <= 1e-6 * abs(an), (fd, an)
    tab = orc.param_table(sh)
    for name, r, c, off in tab:
        for i in off + rng.integers(0, r * c, 2):
            e = np.zeros_like(w)
            e[i] = 1
            fdv = (total(w + eps * e) - total(w - eps * e)) / (2 * eps)
            assert abs(fdv - g[i]) <= 1e-7 + 1e-5 * abs(g[i]), (name, int(i - off), fdv, g[i])
    # ced_test.go:284-300: the last encoder layer receives the decoder's gradient
    split = cfg.ced_split
    off, r, c = cfg.param_slices()[f"transformer.h.{split - 1}.mlp.c_proj.weight"]
    assert np.any(g[off:off + r * c])


@pytest.mark.parametrize("chunk", [1, 3])
@pytest.mark.parametrize("case", ["dense", "fru_sparse"])
def test_ced_decode_matches_training_forward(orc, case, chunk):
    cfg = ced_cfg(seq=64, vocab=40, embd=64, head=4, **CED_FD[case])
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    m = orc.OracleModel(orc.ModelShape.from_config(cfg), w)
    ids = np.random.default_rng(0).integers(0, cfg.vocab_size, (2, 29)).astype(np.int32)
    full = m.forward(ids)
    dec = m.forward_decode(ids, chunk)
    assert np.abs(full - dec).max() <= 2e-6 * np.abs(full).max()


@pytest.mark.parametrize("topk", [0, 2])
def test_ced_prefill_matches_full_when_window_covers_prompt(orc, topk):
    """ced_test.go:193-235: with the window covering the prompt the replay
    starts at position 0, so PrefillCED's last logits equal the full
    forward's; a shorter window truncates the replay and changes them."""
    cfg = ced_cfg(swa=16, topk=topk)
    w = G.init_weights(cfg, seed=42, perturb=0.1).astype(np.float64)
    prompt = np.array([1, 5, 2, 8, 3, 7], np.int32)
    m = orc.OracleModel(orc.ModelShape.from_config(cfg), w, np.float64)
    full = m.forward(prompt[None])[0, -1]
    ced = m.prefill_ced(prompt)
    assert np.abs(full - ced).max() <= 1e-12 * max(1, np.abs(full).max())
    short = ced_cfg(swa=3, topk=topk)
    m2 = orc.OracleModel(orc.ModelShape.from_config(short), w, np.float64)
    assert np.abs(m2.prefill_ced(prompt) - m2.forward(prompt[None])[0, -1]).max() > 1e-6

"""Pins the oracle's latent preset (absorbed MLA + DeepSeekMoE) without running
the reference:

* the backward by central finite differences of CE + balance loss on the
  float64 build, every parameter except the router bias, whose effect is
  piecewise constant (model/moe_test.go:261-362, model/mla_test.go:190-233);
* absorbed MLA decode against the latent cache == the non-absorbed training
  forward, token by token and chunked (model/mla_test.go:279-317,
  model/moe_test.go:221-259), across a sliding window;
* the balance loss of a uniform router equals its weight
  (model/moe_test.go:530-554) and matches its definition on a skewed router
  (model/moe_test.go:585-640);
* a closed form of the routed combine: with every expert equal to the
  shared expert and a zero router, the block equals a dense block whose
  shared-expert output is scaled by 1 + K/E;
* a router with one dominant expert selects it for every token
  (model/moe_test.go:158-190).
"""
import numpy as np
import pytest

from gonano_amd import config as G


def latent_cfg(seq=64, kv=2, n_layer=2, window="SL", balance=0.0):
    cfg = G.Config(sequence_len=seq, vocab_size=48, n_layer=n_layer, n_head=4, n_kv_head=kv,
                   n_embd=64, window_pattern=window)
    return G.apply_latent_preset(cfg, mla_latent=32, n_experts=4, experts_per_token=2,
                                 expert_hidden=16, shared_hidden=24, balance_weight=balance)


def oracle_model(orc, cfg, w, dtype=np.float32):
    return orc.OracleModel(orc.ModelShape.from_config(cfg), w, dtype)


def test_param_table_matches_host_config(orc):
    cfg = latent_cfg()
    tab = orc.param_table(orc.ModelShape.from_config(cfg))
    assert [tuple(t) for t in tab] == [tuple(t) for t in cfg.param_table()]
    names = [t[0] for t in tab]
    assert "transformer.h.0.attn.mla_kv_down.weight" in names
    assert "transformer.h.1.moe.experts.down.weight" in names
    assert not any(n.startswith("value_embeds") for n in names)  # no VE under MLA


def test_latent_d12_shapes():
    cfg = G.latent_d12()
    assert (cfg.n_head, cfg.n_kv_head, cfg.head_dim, cfg.mla_rope_dimension) == (6, 3, 128, 64)
    assert (cfg.mla_latent, cfg.n_experts, cfg.experts_per_token, cfg.expert_hidden,
            cfg.shared_hidden) == (256, 16, 2, 512, 512)
    assert cfg.moe_clamp == 10.0 and cfg.moe_scale == 1.0 and cfg.balance_weight == 1e-4


@pytest.mark.parametrize("chunk", [1, 5])
def test_absorbed_decode_matches_training_forward(orc, chunk):
    # SequenceLen 512 gives 128-key sliding windows on the S layers; 150
    # tokens cross them.
    cfg = latent_cfg(seq=512, window="SL")
    w = G.init_weights(cfg, seed=3, perturb=0.1)
    m = oracle_model(orc, cfg, w)
    ids = np.random.default_rng(0).integers(0, cfg.vocab_size, (1, 150)).astype(np.int32)
    full = m.forward(ids)
    dec = m.forward_decode(ids, chunk)
    err = np.abs(full - dec).max() / np.abs(full).max()
    assert err < 2e-6, err


@pytest.mark.parametrize("kv", [4, 2, 1])
def test_latent_gradients_match_finite_differences(orc, kv):
    cfg = latent_cfg(kv=kv, balance=1e-2)
    w = G.init_weights(cfg, seed=7, perturb=0.1).astype(np.float64)
    sh = orc.ModelShape.from_config(cfg)
    rng = np.random.default_rng(1)
    ids = rng.integers(0, cfg.vocab_size, (2, 10)).astype(np.int32)
    tg = rng.integers(0, cfg.vocab_size, (2, 10)).astype(np.int32)
    tg[:, :2] = -1
    m = orc.OracleModel(sh, w, np.float64)
    _, g = m.ce_loss(ids, tg)

    def total(wv):
        mm = orc.OracleModel(sh, wv, np.float64)
        loss, _ = mm.ce_loss(ids, tg, want_grads=False)
        return loss + mm.aux_loss()

    tab = orc.param_table(sh)
    frozen = np.zeros(w.size, bool)
    for name, r, c, off in tab:
        if name.endswith("router_bias"):
            frozen[off:off + r * c] = True
            assert not np.any(g[off:off + r * c])  # no gradient reaches the bias
    eps = 1e-6
    d = rng.standard_normal(w.size)
    d[frozen] = 0
    fd = (total(w + eps * d) - total(w - eps * d)) / (2 * eps)
    an = float(g @ d)
    assert abs(fd - an) <= 1e-6 * abs(an), (fd, an)
    for name, r, c, off in tab:
        if name.endswith("router_bias"):
            continue
        for i in off + rng.integers(0, r * c, 2):
            e = np.zeros_like(w)
            e[i] = 1
            fdv = (total(w + eps * e) - total(w - eps * e)) / (2 * eps)
            assert abs(fdv - g[i]) <= 1e-7 + 1e-5 * abs(g[i]), (name, int(i - off), fdv, g[i])


def test_balance_loss_uniform_router_equals_weight(orc):
    cfg = latent_cfg(balance=3e-4)
    w = G.init_weights(cfg, seed=3)
    sl = cfg.param_slices()
    for l in range(cfg.n_layer):
        for k in ("moe.router.weight", "moe.router_bias"):
            off, r, c = sl[f"transformer.h.{l}.{k}"]
            w[off:off + r * c] = 0
    m = oracle_model(orc, cfg, w, np.float64)
    ids = np.random.default_rng(2).integers(0, cfg.vocab_size, (3, 8)).astype(np.int32)
    m.ce_loss(ids, ids, want_grads=False)
    # every layer contributes exactly the weight (uniform probabilities); the
    # weight is a float32 config field
    assert abs(m.aux_loss() - cfg.n_layer * float(np.float32(3e-4))) < 1e-15


def test_routed_combine_closed_form(orc):
    """Experts equal to the shared expert and a zero router: each token's two
    routed outputs are the shared output weighted 1/E each, so the block is a
    dense SwiGLU block whose output projection is scaled by 1 + K/E."""
    cfg = latent_cfg()
    cfg.expert_hidden = cfg.shared_hidden  # same width for the copy
    w = G.init_weights(cfg, seed=4, perturb=0.1).astype(np.float64)  # exact 1 + K/E scaling
    sl = cfg.param_slices()
    E, K, C, H = cfg.n_experts, cfg.experts_per_token, cfg.n_embd, cfg.expert_hidden
    w2 = w.copy()
    for l in range(cfg.n_layer):
        p = f"transformer.h.{l}."

        def get(name, arr=w):
            off, r, c = sl[p + name]
            return arr[off:off + r * c].reshape(r, c)

        for k in ("moe.router.weight", "moe.router_bias"):
            get(k)[:] = 0
            get(k, w2)[:] = 0
        gate, up, proj = get("mlp.c_gate.weight"), get("mlp.c_fc.weight"), get("mlp.c_proj.weight")
        get("moe.experts.gate.weight")[:] = np.tile(gate, (E, 1))
        get("moe.experts.up.weight")[:] = np.tile(up, (E, 1))
        get("moe.experts.down.weight")[:] = np.tile(proj, (E, 1))
        # the closed form: no routed output, shared output scaled by 1 + K/E
        get("moe.experts.down.weight", w2)[:] = 0
        get("mlp.c_proj.weight", w2)[:] = proj * (1 + K / E)
    ids = np.random.default_rng(5).integers(0, cfg.vocab_size, (2, 9)).astype(np.int32)
    a = oracle_model(orc, cfg, w, np.float64).forward(ids)
    b = oracle_model(orc, cfg, w2, np.float64).forward(ids)
    assert np.abs(a - b).max() < 1e-9 * max(1.0, np.abs(a).max())


def test_dominant_expert_takes_every_token(orc):
    """A large router correction bias on one expert makes top-1 selection pick
    it for every token (selection uses logits + bias, moe.go:124,
    kernels/scalar/moe.go:33-40): zeroing every other expert's weights must
    then leave the output unchanged."""
    cfg = latent_cfg()
    cfg.experts_per_token = 1
    w = G.init_weights(cfg, seed=6, perturb=0.1)
    sl = cfg.param_slices()
    for l in range(cfg.n_layer):
        off, r, c = sl[f"transformer.h.{l}.moe.router_bias"]
        w[off:off + r * c] = [0.0, 0.0, 100.0, 0.0]
    w_only = w.copy()
    for l in range(cfg.n_layer):
        for k in ("moe.experts.gate.weight", "moe.experts.up.weight", "moe.experts.down.weight"):
            o2, r2, c2 = sl[f"transformer.h.{l}.{k}"]
            blk = w_only[o2:o2 + r2 * c2].reshape(cfg.n_experts, -1)
            blk[[0, 1, 3]] = 0
    ids = np.random.default_rng(8).integers(0, cfg.vocab_size, (2, 7)).astype(np.int32)
    a = oracle_model(orc, cfg, w, np.float64).forward(ids)
    b = oracle_model(orc, cfg, w_only, np.float64).forward(ids)
    assert np.array_equal(a, b)
    # and the bias really routes: moving it to expert 0 changes the output
    w_other = w.copy()
    for l in range(cfg.n_layer):
        off, r, c = sl[f"transformer.h.{l}.moe.router_bias"]
        w_other[off:off + r * c] = [100.0, 0.0, 0.0, 0.0]
    c_ = oracle_model(orc, cfg, w_other, np.float64).forward(ids)
    assert np.abs(a - c_).max() > 1e-6

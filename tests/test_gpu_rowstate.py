"""The rollout row state machine on the GPU (inference/engine.go:241-325,
336-369): tool calls with forced output, the thinking budget, and the
tokenizer's special ids and tool registry passed through
gn_generate_options.

The model is built so that its greedy continuation is known in closed
form.  InitWeights leaves every c_proj weight zero (the attention output
and MLP down projections, model/transformer.go:162), so the residual stream
of a token is a positive multiple of its normalized embedding; with unit
embedding rows E[t] and lm_head row u = 0.5 * sum of E[t] over the tokens t
whose designed successor is u, the successor's logit is 15*tanh(8/15) and
every other logit is a cross term of random 256-wide unit vectors (|.| <~
1.5).  With top-k 1 (only the maximum survives the mask, sampler.go:26-60)
or temperature 0 (argmax) every row follows the designed chain, so the
expected rows, masks and forced tokens are written out by hand from the
reference's state machine."""
import numpy as np
import pytest

from gonano_amd import config as G

pytestmark = pytest.mark.gpu

BOS, END, TSTART, TEND, TOSTART, TOEND, THSTART, THEND = 256, 260, 261, 262, 263, 264, 265, 266


def chain_model(successor, V=512, C=256, seed=0):
    cfg = G.Config(sequence_len=512, vocab_size=V, n_layer=2, n_head=2, n_kv_head=1, n_embd=C,
                   window_pattern="SSSL", rotary_dims=64)
    w = G.init_weights(cfg, seed=seed)
    sl = cfg.param_slices()
    E = np.random.default_rng(seed + 1).standard_normal((V, C)).astype(np.float32)
    E /= np.linalg.norm(E, axis=1, keepdims=True)
    off, r, c = sl["transformer.wte.weight"]
    w[off:off + r * c] = E.ravel()
    lm = np.zeros((r, c), np.float32)
    for t, u in successor.items():
        lm[u] += 0.5 * E[t]
    off, r2, c2 = sl["lm_head.weight"]
    assert (r2, c2) == lm.shape
    w[off:off + r * c] = lm.ravel()
    for name in sl:  # the residual stream carries the embedding alone
        if name.endswith("attn.c_proj.weight") or name.endswith("mlp.c_proj.weight"):
            o, rr, cc = sl[name]
            assert not w[o:o + rr * cc].any()
    return cfg, w


def _gen(cfg, w, prompts, S, N, T, k, options=None):
    from gonano_amd.session import Session
    with Session(cfg) as s:
        s.set_params(w)
        return s.generate_batch(np.asarray(prompts, np.int32), S, N, T, k,
                                np.arange(len(prompts), dtype=np.uint64) + 5, options=options,
                                masks=True)


def test_tool_call_forces_the_calculator_output(orc):
    """<|tool_start|> 1 + 2 <|tool_end|> is answered by forced
    <|tool_output_start|> 3 <|tool_output_end|> (engine.go:279-297), which
    the masks mark as forced; then <|assistant_end|> ends the row and is
    left out (engine.go:349-366).  The oracle's engine gives the same rows."""
    chain = {7: TSTART, TSTART: ord("1"), ord("1"): ord("+"), ord("+"): ord("2"),
             ord("2"): TEND, TOEND: END}
    cfg, w = chain_model(chain)
    prompts = [[5, 6, 7], [9, 8, 7]]
    for T, k in ((1.0, 1), (0.0, 50)):
        rows, masks = _gen(cfg, w, prompts, 3, 12, T, k)
        comp = [TSTART, ord("1"), ord("+"), ord("2"), TEND, TOSTART, ord("3"), TOEND]
        for g, p in enumerate(prompts):
            for i in range(3):
                r, m = rows[g * 3 + i], masks[g * 3 + i]
                assert r.tolist() == p + comp, (T, k, r.tolist())
                assert m.tolist() == [0] * 3 + [1] * 5 + [0] * 3
        m = orc.OracleModel(orc.ModelShape.from_config(cfg), w)
        want = m.generate_batch(np.array(prompts[0], np.int32), 3, 12, T, k, 5)
        assert [r.tolist() for r in want] == [r.tolist() for r in rows[:3]]


def test_thinking_budget_forces_think_end():
    """GenerateOptions{ThinkingBudget: 3}: after <|think_start|> the third
    reasoning token forces <|think_end|> (engine.go:298-313); a prompt that
    ends with <|think_start|> starts inside the trace (engine.go:226-236);
    without the options the trace runs on to max_tokens."""
    from gonano_amd.session import GenerateOptions
    x = ord("x")
    cfg, w = chain_model({9: THSTART, THSTART: x, x: x, THEND: END})
    rows, masks = _gen(cfg, w, [[1, 2, 9]], 2, 10, 1.0, 1, GenerateOptions(thinking_budget=3))
    for r, m in zip(rows, masks):
        assert r.tolist() == [1, 2, 9, THSTART, x, x, x, THEND]
        assert m.tolist() == [0, 0, 0, 1, 1, 1, 1, 0]
    rows, masks = _gen(cfg, w, [[1, 2, THSTART]], 2, 10, 1.0, 1,
                       GenerateOptions(thinking=True, thinking_budget=2))
    for r, m in zip(rows, masks):
        assert r.tolist() == [1, 2, THSTART, x, x, THEND]
        assert m.tolist() == [0, 0, 0, 1, 1, 0]
    # Thinking without a budget tracks the trace but forces nothing
    rows, _ = _gen(cfg, w, [[1, 2, 9]], 2, 10, 1.0, 1, GenerateOptions(thinking=True))
    assert all(r.tolist() == [1, 2, 9, THSTART] + [x] * 9 for r in rows)
    rows, _ = _gen(cfg, w, [[1, 2, 9]], 2, 10, 1.0, 1)
    assert all(r.tolist() == [1, 2, 9, THSTART] + [x] * 9 for r in rows)


def test_custom_special_ids_and_tool_registry(orc):
    """A tokenizer whose specials sit at 400..410 and whose byte b is id
    b + 1, with the host's tool registry as the callback: its ids decide the
    tool call, the forced output and the end of a row (260 is an ordinary
    token here), and rl_step pads with its <|assistant_end|>."""
    from gonano_amd.session import GenerateOptions, Session, use_calculator
    ids = dict(bos=400, assistant_end=404, tool_start=405, tool_end=406, tool_output_start=407,
               tool_output_end=408, think_start=409, think_end=410)
    calls = []

    def tool(call_ids):  # Tokenizer.Decode -> Registry.Execute -> Tokenizer.Encode
        calls.append(list(call_ids))
        res = use_calculator("".join(chr(i - 1) for i in call_ids))
        return None if res is None else [ord(ch) + 1 for ch in res]

    b = lambda ch: ord(ch) + 1  # noqa: E731
    chain = {11: 405, 405: b("1"), b("1"): b("+"), b("+"): b("2"), b("2"): 406, 408: 260,
             260: 404}
    cfg, w = chain_model(chain)
    opts = GenerateOptions(tool=tool, **ids)
    rows, masks = _gen(cfg, w, [[3, 11], [4, 11]], 2, 14, 1.0, 1, opts)
    comp = [405, b("1"), b("+"), b("2"), 406, 407, b("3"), 408, 260]
    for g in range(2):
        for i in range(2):
            r, m = rows[g * 2 + i], masks[g * 2 + i]
            assert r.tolist()[2:] == comp
            assert m.tolist() == [0, 0, 1, 1, 1, 1, 1, 0, 0, 0, 1]
    assert calls and all(c == [b("1"), b("+"), b("2")] for c in calls)
    # a call no tool understands forces nothing
    chain2 = {11: 405, 405: b("a"), b("a"): 406, 406: 260, 260: 404}
    cfg2, w2 = chain_model(chain2)
    rows, masks = _gen(cfg2, w2, [[3, 11]], 1, 8, 1.0, 1, opts)
    assert rows[0].tolist() == [3, 11, 405, b("a"), 406, 260]
    # rl_step_with pads with the tokenizer's <|assistant_end|> (chat_rl/main.go:157-180)
    prompts = np.array([[3, 11], [4, 11]], np.int32)
    rewards = np.array([1, 0, 0, 1], np.float32)
    with Session(cfg) as s:
        s.set_params(w)
        s.zero_grad()
        out = s.rl_step(prompts, 2, 14, 1.0, 1, np.array([5, 6], np.uint64), rewards, options=opts)
    L = out["max_len"]
    assert L == 11 and all(r.tolist()[2:] == comp for r in out["rows"])
    rows_ = [np.concatenate([r, np.full(L - len(r), 404, np.int32)]) for r in out["rows"]]
    inputs = np.stack([r[:-1] for r in rows_])
    targets = np.stack([r[1:] for r in rows_])
    targets[:, :2] = -1
    m = orc.OracleModel(orc.ModelShape.from_config(cfg), w)
    wl, _, _ = m.pg_step(inputs, targets, out["adv"], float(L))
    assert abs(out["loss"] - wl) <= 1e-4 * max(abs(wl), 1e-3)

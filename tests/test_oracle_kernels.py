"""Pins the oracle's kernels.Backend restatement to the reference's own known
answers (kernels/scalar/scalar_test.go, tensors/loss_test.go,
tensors/backward_test.go, model/layers/backward_test.go, model/model_test.go)
and to brute-force numpy computations on small inputs."""
import math

import numpy as np
import pytest

from conftest import assert_close

f32 = np.float32


def arr(*v):
    return np.array(v, f32)


def test_elementwise_known_answers(orc):  # scalar_test.go:12-38
    L = orc.lib()
    left, right = arr(1, 2, 3), arr(4, 5, 6)
    d = np.zeros(3, f32)
    L.orc_add(d, left, right, 3); assert_close(d, [5, 7, 9], 1e-6, 1e-6)
    L.orc_subtract(d, right, left, 3); assert_close(d, [3, 3, 3], 1e-6, 1e-6)
    L.orc_multiply(d, left, right, 3); assert_close(d, [4, 10, 18], 1e-6, 1e-6)
    L.orc_divide(d, right, left, 3); assert_close(d, [4, 2.5, 2], 1e-6, 1e-6)
    L.orc_scale(d, left, 2.0, 3); assert_close(d, [2, 4, 6], 1e-6, 1e-6)
    L.orc_add_scaled(d, left, right, 0.5, 3); assert_close(d, [3, 4.5, 6], 1e-6, 1e-6)
    L.orc_negate(d, left, 3); assert_close(d, [-1, -2, -3], 1e-6, 1e-6)
    L.orc_abs(d, arr(-1, 2, -3), 3); assert_close(d, [1, 2, 3], 1e-6, 1e-6)
    L.orc_square(d, left, 3); assert_close(d, [1, 4, 9], 1e-6, 1e-6)
    L.orc_relu_squared(d, arr(-1, 2, -3), 3); assert_close(d, [0, 4, 0], 1e-6, 1e-6)


def test_swiglu_known_answers(orc):  # scalar_test.go:40-92
    L = orc.lib()
    silu = lambda x: x / (1 + math.exp(-x))
    d = np.zeros(4, f32)
    L.orc_swiglu(d, arr(0, 1, -1, 2), arr(1, 1, 2, -3), 0.0, 4)
    assert_close(d, [silu(0), silu(1), silu(-1) * 2, silu(2) * -3], 1e-5, 1e-6)
    L.orc_swiglu(d, arr(20, 1, 1, 2), arr(1, 20, -20, 1), 10.0, 4)
    assert_close(d, [silu(10), silu(1) * 10, silu(1) * -10, silu(2)], 1e-5, 1e-6)
    gate, up, dout = arr(0.5, 1.5), arr(2.0, -1.0), arr(1.0, 2.0)
    dg, du = np.zeros(2, f32), np.zeros(2, f32)
    L.orc_swiglu_backward(dg, du, gate, up, dout, 10.0, 2)
    for i in range(2):
        g, u, o = float(gate[i]), float(up[i]), float(dout[i])
        s = 1 / (1 + math.exp(-g))
        assert_close(dg[i], o * u * s * (1 + g * (1 - s)), 1e-5, 1e-6)
        assert_close(du[i], o * g * s, 1e-5, 1e-6)
    # clamped positions carry no gradient through the clamped operand
    L.orc_swiglu_backward(dg, du, arr(20, 1), arr(1, 20), arr(1, 1), 10.0, 2)
    assert dg[0] == 0 and du[1] == 0


def test_transcendentals_and_reductions(orc):  # scalar_test.go:94-135
    L = orc.lib()
    d = np.zeros(1, f32)
    L.orc_exp(d, arr(1), 1); assert_close(d, [math.e], 1e-6, 1e-6)
    L.orc_sigmoid(d, arr(0), 1); assert_close(d, [0.5], 1e-6, 1e-6)
    L.orc_tanh(d, arr(0), 1); assert_close(d, [0], 1e-6, 1e-6)
    L.orc_rsqrt(d, arr(4), 1); assert_close(d, [0.5], 1e-6, 1e-6)
    assert L.orc_sum(arr(1, 2, 3, 4), 4) == 10
    assert L.orc_max(arr(1, 9, 3), 3) == 9
    assert L.orc_max(np.zeros(1, f32), 0) == 0
    assert L.orc_argmax(arr(1, 9, 3), 3) == 1
    assert L.orc_argmax(arr(5, 9, 9), 3) == 1  # ties resolve to the smaller index
    left, right = arr(1, 2, 3, 4, 5, 6), arr(7, 8, 9, 10, 11, 12)
    d = np.zeros(4, f32)
    L.orc_matmul(d, left, right, 2, 2, 3); assert_close(d, [58, 64, 139, 154], 1e-5, 1e-5)
    L.orc_matmul_transposed(d, left, right, 2, 2, 3); assert_close(d, [50, 68, 122, 167], 1e-5, 1e-5)
    assert abs(L.orc_dot(arr(1, 2, 3), arr(4, 5, 6), 3) - 32) < 1e-6


def test_matmul_brute_force(orc):
    rng = np.random.default_rng(0)
    for (m, n, k) in [(1, 1, 1), (7, 31, 13), (33, 17, 64)]:
        a = rng.standard_normal((m, k)).astype(f32)
        b = rng.standard_normal((k, n)).astype(f32)
        d = np.zeros((m, n), f32)
        orc.lib().orc_matmul(d, a, b, m, n, k)
        assert_close(d, a.astype(np.float64) @ b.astype(np.float64), 1e-6, 1e-6)
        bt = np.ascontiguousarray(b.T)
        orc.lib().orc_matmul_transposed(d, a, bt, m, n, k)
        assert_close(d, a.astype(np.float64) @ b.astype(np.float64), 1e-6, 1e-6)


def test_rows(orc):  # scalar_test.go:137-151
    L = orc.lib()
    d = np.zeros(4, f32)
    L.orc_softmax_last_dim(d, arr(1, 2, 3, 4), 2, 2)
    assert abs(d.astype(np.float64).sum() - 2) <= 1e-6
    assert_close(d[:2], np.exp([1, 2]) / np.exp([1, 2]).sum(), 1e-6, 1e-7)
    L.orc_rmsnorm_last_dim(d, arr(1, 1, 1, 1), 2, 2, 1e-6)
    assert_close(d, [1, 1, 1, 1], 1e-5, 1e-5)
    x = np.random.default_rng(1).standard_normal((5, 33)).astype(f32)
    y = np.zeros_like(x)
    L.orc_rmsnorm_last_dim(y, x, 5, 33, 1e-6)
    want = x / np.sqrt((x.astype(np.float64) ** 2).mean(1, keepdims=True) + 1e-6)
    assert_close(y, want, 1e-6, 1e-7)


def _np_attention(q, k, v, offset, window):
    s = q.astype(np.float64) @ k.astype(np.float64).T
    qpos = offset + np.arange(q.shape[0])[:, None]
    kj = np.arange(k.shape[0])[None, :]
    masked = (kj > qpos) | ((window >= 0) & (qpos - kj > window))
    s = np.where(masked, -1e30, s)
    m = s.max(1, keepdims=True)
    p = np.exp(s - m)
    tot = p.sum(1, keepdims=True)
    return (p / tot) @ v.astype(np.float64), (m + np.log(tot))[:, 0]


@pytest.mark.parametrize("qlen,klen,offset,window", [(2, 2, 0, -1), (5, 9, 4, -1), (4, 40, 36, 7),
                                                     (1, 300, 299, 128), (7, 7, 0, 0)])
def test_attention_forward_brute_force(orc, qlen, klen, offset, window):
    rng = np.random.default_rng(qlen * 100 + klen)
    D = 8
    q = rng.standard_normal((qlen, D)).astype(f32)
    k = rng.standard_normal((klen, D)).astype(f32)
    v = rng.standard_normal((klen, D)).astype(f32)
    out = np.zeros((qlen, D), f32)
    lse = np.zeros(qlen, f32)
    orc.lib().orc_attention_forward(q, k, v, out, lse.ctypes.data, None, 0, qlen, klen, D, offset,
                                    window)
    wo, wl = _np_attention(q, k, v, offset, window)
    assert_close(out, wo, 1e-5, 1e-6)
    assert_close(lse, wl, 1e-5, 1e-6)
    # split-K shards + combine equal the full pass (model/model_test.go:230-250)
    for splits in (2, 5):
        per = (klen + splits - 1) // splits
        acc = np.zeros((splits, qlen, D), f32)
        mx = np.zeros((splits, qlen), f32)
        sm = np.zeros((splits, qlen), f32)
        for s in range(splits):
            a, m_, s_ = np.zeros((qlen, D), f32), np.zeros(qlen, f32), np.zeros(qlen, f32)
            orc.lib().orc_attention_forward_split(q, k, v, a, m_, s_, None, 0, qlen, klen, D, offset,
                                                  window, s * per, min(s * per + per, klen))
            acc[s], mx[s], sm[s] = a, m_, s_
        o2, l2 = np.zeros((qlen, D), f32), np.zeros(qlen, f32)
        orc.lib().orc_attention_combine(acc, mx, sm, splits, o2, l2.ctypes.data, qlen, D)
        assert_close(o2, wo, 1e-4, 1e-5)
        assert_close(l2, wl, 1e-4, 1e-5)


def test_attention_reference_case_and_backward_fd(orc):  # scalar_test.go:153-186
    L = orc.lib()
    q = arr(1, 0, 0, 1); k = arr(1, 0, 0, 1); v = arr(1, 0, 0, 1)
    out, lse = np.zeros(4, f32), np.zeros(2, f32)
    L.orc_attention_forward(q, k, v, out, lse.ctypes.data, None, 0, 2, 2, 2, 0, -1)
    assert_close(out[:2], [1, 0], 1e-5, 1e-6)
    # backward vs central differences of sum(dO * O) on a random case
    rng = np.random.default_rng(3)
    qlen, klen, D, off, win = 3, 6, 4, 3, 2
    q = rng.standard_normal((qlen, D)).astype(f32)
    k = rng.standard_normal((klen, D)).astype(f32)
    v = rng.standard_normal((klen, D)).astype(f32)
    do = rng.standard_normal((qlen, D)).astype(f32)
    o, l = _np_attention(q, k, v, off, win)
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    L.orc_attention_backward(q, k, v, o.astype(f32), do, l.astype(f32), None, None, 0, dq, dk, dv,
                             qlen, klen, D, off, win)
    f = lambda q_, k_, v_: float((_np_attention(q_, k_, v_, off, win)[0] * do).sum())
    eps = 1e-3
    for name, x, g in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        num = np.zeros_like(x, dtype=np.float64)
        for idx in np.ndindex(x.shape):
            xp, xm = x.astype(np.float64).copy(), x.astype(np.float64).copy()
            xp[idx] += eps; xm[idx] -= eps
            args_p = {"q": q, "k": k, "v": v}; args_m = dict(args_p)
            args_p[name] = xp; args_m[name] = xm
            num[idx] = (f(**{a + "_": b for a, b in args_p.items()}) -
                        f(**{a + "_": b for a, b in args_m.items()})) / (2 * eps)
        assert_close(g, num, 1e-3, 1e-4, name)


def test_moe_and_indexer_known_answers(orc):  # scalar_test.go:188-235
    L = orc.lib()
    probs, sel, w = np.zeros(3, f32), np.zeros(2, np.int32), np.zeros(2, f32)
    L.orc_moe_gate_topk(arr(0, 0, 0), arr(0, 1, 2), probs, sel, w, 1, 3, 2)
    assert_close(probs, [1 / 3] * 3, 1e-6, 1e-6)
    assert list(sel) == [2, 1]
    assert_close(w, [1 / 3] * 2, 1e-6, 1e-6)
    got = np.zeros(6, np.int32)
    L.orc_topk_indices(got, arr(0.1, 0.9, 0.3, 0.7, 0.5, 0.2, 0.5, 0.2), 2, 4, 3)
    assert list(got) == [1, 3, 2, 0, 2, 1]
    d = np.zeros(6, f32)
    L.orc_grouped_matmul_transposed(d, arr(1, 2, 3, 4, 5, 6), arr(1, 0, 0, 1, 2, 0, 0, 3),
                                    np.array([2, 1], np.int32), 2, 2, 2)
    assert_close(d, [1, 2, 3, 4, 10, 18], 1e-6, 1e-6)
    rng = np.random.default_rng(5)
    q = rng.standard_normal((3, 2, 4)).astype(f32)
    k = rng.standard_normal((5, 2, 4)).astype(f32)
    hw = arr(0.7, 1.3)
    s = np.zeros((3, 5), f32)
    L.orc_indexer_scores(s, q, k, hw, 3, 5, 2, 4)
    dots = np.einsum("rhd,bhd->rbh", q.astype(np.float64), k.astype(np.float64))
    assert_close(s, (np.maximum(dots, 0) * hw).sum(-1), 1e-5, 1e-6)
    bm = np.zeros((3, 2), f32)
    L.orc_indexer_block_max(bm, s, 3, 5, 3)
    assert_close(bm, np.stack([s[:, :3].max(1), s[:, 3:].max(1)], 1), 0, 0)


def test_cross_entropy_known_values(orc):
    """tensors/loss_test.go:8-43 and backward_test.go:70-89 through the PG
    step of a model-free restatement: nll = lse - z_t; grad = softmax - onehot."""
    z = np.array([[0, 0, 5, 0], [1, 1, 1, 1], [2, 0, 0, 0]], np.float64)
    lse = np.log(np.exp(z).sum(1))
    assert abs((lse[0] - z[0, 2]) - (math.log(math.exp(5) + 3) - 5)) < 1e-12
    assert abs((lse[2] - z[2, 0]) - (math.log(math.exp(2) + 3) - 2)) < 1e-12
    d = np.zeros(3, f32)
    orc.lib().orc_softmax_last_dim(d, arr(0, 0, 0), 1, 3)
    d[1] -= 1
    assert_close(d, [1 / 3, -2 / 3, 1 / 3], 1e-5, 1e-6)

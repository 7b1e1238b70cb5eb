"""Parity of the HIP kernels.Backend primitives with the oracle
(kernels/scalar restated) on identical inputs, at the shapes and tolerances
of the reference's own scalar-vs-SIMD parity suite
(kernels/simd/parity_test.go: vector tails {1,7,31,64,513,1031}; MatMul up to
400x128x512 at 2e-3/1e-4; rows 1e-4; attention forward 2e-3, backward 5e-3;
exact top-k and MoE selection with ties)."""
import numpy as np
import pytest

from conftest import assert_close

pytestmark = pytest.mark.gpu

LENGTHS = [1, 7, 31, 64, 513, 1031]
f32 = np.float32


@pytest.fixture(scope="module")
def be():
    from gonano_amd.backend import HipBackend
    return HipBackend(0)


def data(n, seed=0, positive=False):
    """kerneltest.Data / DataB (kernels/kerneltest/compare.go:12-26) plus noise."""
    i = np.arange(n)
    if positive:
        base = (i % 5) + 0.5
    else:
        base = (i % 7) - 3.5 + 0.1 * (i % 3)
    return (base + 0.01 * np.random.default_rng(seed).standard_normal(n)).astype(f32)


@pytest.mark.parametrize("n", LENGTHS)
def test_elementwise(be, orc, n):
    L = orc.lib()
    a, b, p = data(n, 1), data(n, 2), data(n, 3, True)
    cases = [
        ("Add", (a, b), "orc_add"), ("Subtract", (a, b), "orc_subtract"),
        ("Multiply", (a, b), "orc_multiply"), ("Divide", (a, p), "orc_divide"),
        ("Negate", (a,), "orc_negate"), ("Abs", (a,), "orc_abs"), ("Square", (a,), "orc_square"),
        ("ReluSquared", (a,), "orc_relu_squared"), ("Exp", (a,), "orc_exp"),
        ("Sigmoid", (a,), "orc_sigmoid"), ("Tanh", (a,), "orc_tanh"), ("Rsqrt", (p,), "orc_rsqrt"),
    ]
    for name, args, oname in cases:
        got, want = np.zeros(n, f32), np.zeros(n, f32)
        getattr(be, name)(got, *args)
        getattr(L, oname)(want, *args, n)
        assert_close(got, want, 1e-5, 1e-6, name)
    got, want = np.zeros(n, f32), np.zeros(n, f32)
    be.Scale(got, a, 0.37); L.orc_scale(want, a, 0.37, n)
    assert_close(got, want, 1e-6, 1e-7, "Scale")
    be.AddScaled(got, a, b, -1.5); L.orc_add_scaled(want, a, b, -1.5, n)
    assert_close(got, want, 1e-6, 1e-7, "AddScaled")
    for clamp in (0.0, 10.0, 2.0):
        g, u, do = data(n, 4) * 4, data(n, 5) * 4, data(n, 6)
        got, want = np.zeros(n, f32), np.zeros(n, f32)
        be.SwiGLU(got, g, u, clamp); L.orc_swiglu(want, g, u, clamp, n)
        assert_close(got, want, 1e-5, 1e-6, "SwiGLU")
        gg, gu, wg, wu = (np.zeros(n, f32) for _ in range(4))
        be.SwiGLUBackward(gg, gu, g, u, do, clamp)
        L.orc_swiglu_backward(wg, wu, g, u, do, clamp, n)
        assert_close(gg, wg, 1e-5, 1e-6, "SwiGLUBackward gate")
        assert_close(gu, wu, 1e-5, 1e-6, "SwiGLUBackward up")


def test_aliasing(be):
    a = data(513, 1)
    b = data(513, 2)
    want = a + b
    be.Add(a, a, b)  # destination aliases the left source
    assert_close(a, want, 1e-7, 0, "aliased Add")


@pytest.mark.parametrize("n", LENGTHS + [0, 100000])
def test_reductions(be, orc, n):
    L = orc.lib()
    v = data(max(n, 1), 7)[:n] if n else np.zeros(0, f32)
    vv = v if n else np.zeros(1, f32)
    assert abs(be.Sum(vv[:n] if n else vv[:0]) - float(np.sum(v.astype(np.float64)))) <= 1e-4 * max(1, abs(float(np.sum(v))))
    if n:
        assert be.Max(v) == L.orc_max(v, n)
        v2 = v.copy()
        v2[n // 3] = v2.max()  # a tie: the smaller index wins
        assert be.ArgMax(v2) == L.orc_argmax(v2, n)
        w = data(n, 8)
        assert abs(be.DotProduct(v, w) - L.orc_dot(v, w, n)) <= 1e-4 * max(1, abs(L.orc_dot(v, w, n)))
    else:
        assert be.Max(vv[:0]) == 0
        assert be.ArgMax(vv[:0]) == 0


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (2, 2, 3), (7, 31, 13), (64, 64, 64), (33, 513, 65),
                                   (400, 128, 512), (128, 400, 512), (3, 1031, 7)])
def test_matmul(be, orc, m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    a = rng.standard_normal((m, k)).astype(f32)
    b = rng.standard_normal((k, n)).astype(f32)
    bt = np.ascontiguousarray(b.T)
    got, want = np.zeros((m, n), f32), np.zeros((m, n), f32)
    be.MatMul(got, a, b, m, n, k)
    orc.lib().orc_matmul(want, a, b, m, n, k)
    assert_close(got, want, 2e-3, 1e-4, "MatMul")
    got2 = np.zeros((m, n), f32)
    be.MatMulTransposed(got2, a, bt, m, n, k)
    assert_close(got2, want, 2e-3, 1e-4, "MatMulTransposed")


def test_matmul_known_answer(be):  # kernels/scalar/scalar_test.go:123-130
    left = np.array([1, 2, 3, 4, 5, 6], f32)
    right = np.array([7, 8, 9, 10, 11, 12], f32)
    d = np.zeros(4, f32)
    be.MatMul(d, left, right, 2, 2, 3)
    assert_close(d, [58, 64, 139, 154], 1e-5, 1e-5)
    be.MatMulTransposed(d, left, right, 2, 2, 3)
    assert_close(d, [50, 68, 122, 167], 1e-5, 1e-5)


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 7), (5, 513), (17, 1031), (2, 65536)])
def test_rows(be, orc, rows, cols):
    x = (np.random.default_rng(cols).standard_normal((rows, cols)) * 3).astype(f32)
    got, want = np.zeros_like(x), np.zeros_like(x)
    be.SoftmaxLastDim(got, x, rows, cols)
    orc.lib().orc_softmax_last_dim(want, x, rows, cols)
    assert_close(got, want, 1e-4, 1e-7, "SoftmaxLastDim")
    be.RMSNormLastDim(got, x, rows, cols, 1e-6)
    orc.lib().orc_rmsnorm_last_dim(want, x, rows, cols, 1e-6)
    assert_close(got, want, 1e-4, 1e-6, "RMSNormLastDim")


def test_topk_and_moe(be, orc):
    L = orc.lib()
    scores = np.array([0.1, 0.9, 0.3, 0.7, 0.5, 0.2, 0.5, 0.2], f32)
    got = np.zeros(6, np.int32)
    be.TopKIndices(got, scores, 2, 4, 3)
    assert list(got) == [1, 3, 2, 0, 2, 1]
    rng = np.random.default_rng(3)
    for rows, count, k in [(7, 16, 2), (64, 24, 6), (5, 300, 16), (3, 5, 5)]:
        s = rng.integers(-4, 4, (rows, count)).astype(f32)  # many ties
        got, want = np.zeros(rows * k, np.int32), np.zeros(rows * k, np.int32)
        be.TopKIndices(got, s, rows, count, k)
        L.orc_topk_indices(want, s, rows, count, k)
        assert (got == want).all()
        logits = (rng.standard_normal((rows, count))).astype(f32)
        bias = rng.integers(-1, 2, count).astype(f32)
        outs = [[np.zeros(rows * count, f32), np.zeros(rows * k, np.int32), np.zeros(rows * k, f32)]
                for _ in range(2)]
        be.MoEGateTopK(logits, bias, *outs[0], rows, count, k)
        L.orc_moe_gate_topk(logits, bias, *outs[1], rows, count, k)
        assert_close(outs[0][0], outs[1][0], 1e-5, 1e-7, "probs")
        assert (outs[0][1] == outs[1][1]).all()
        assert_close(outs[0][2], outs[1][2], 1e-5, 1e-7, "weights")


def test_grouped_matmul_and_indexer(be, orc):
    L = orc.lib()
    d = np.zeros(6, f32)
    be.GroupedMatMulTransposed(d, np.array([1, 2, 3, 4, 5, 6], f32),
                               np.array([1, 0, 0, 1, 2, 0, 0, 3], f32), [2, 1], 2, 2, 2)
    assert_close(d, [1, 2, 3, 4, 10, 18], 1e-6, 1e-6)
    rng = np.random.default_rng(4)
    counts = np.array([3, 0, 17, 5], np.int32)
    x = rng.standard_normal((25, 48)).astype(f32)
    w = rng.standard_normal((4, 33, 48)).astype(f32)
    got, want = np.zeros((25, 33), f32), np.zeros((25, 33), f32)
    be.GroupedMatMulTransposed(got, x, w, counts, 4, 33, 48)
    L.orc_grouped_matmul_transposed(want, x, w, counts, 4, 33, 48)
    assert_close(got, want, 2e-3, 1e-4, "grouped")
    q = rng.standard_normal((9, 2, 64)).astype(f32)
    k = rng.standard_normal((37, 2, 64)).astype(f32)
    hw = np.array([0.6, 1.4], f32)
    got, want = np.zeros((9, 37), f32), np.zeros((9, 37), f32)
    be.IndexerScores(got, q, k, hw, 9, 37, 2, 64)
    L.orc_indexer_scores(want, q, k, hw, 9, 37, 2, 64)
    assert_close(got, want, 1e-4, 1e-5, "IndexerScores")
    g1, g2 = np.zeros((9, 5), f32), np.zeros((9, 5), f32)
    be.IndexerBlockMax(g1, want, 9, 37, 8)
    L.orc_indexer_block_max(g2, want, 9, 37, 8)
    assert (g1 == g2).all()


ATTN_CASES = [  # (qlen, klen, dim, offset, window, segments)
    (16, 16, 32, 0, -1, False),      # causal prefill
    (1, 300, 128, 299, -1, False),   # decode
    (4, 97, 64, 93, 17, False),      # sliding window
    (33, 33, 16, 0, 5, False),
    (20, 20, 8, 0, -1, True),        # sample-level segments
]


@pytest.mark.parametrize("qlen,klen,dim,offset,window,seg", ATTN_CASES)
def test_attention(be, orc, qlen, klen, dim, offset, window, seg):
    from gonano_amd.backend import (AttentionBackwardParameters, AttentionBackwardResult,
                                    AttentionCombineParameters, AttentionForwardParameters,
                                    AttentionForwardResult, AttentionSplitParameters,
                                    AttentionSplitResult)
    L = orc.lib()
    rng = np.random.default_rng(qlen * 7 + klen)
    q = rng.standard_normal((qlen, dim)).astype(f32)
    k = rng.standard_normal((klen, dim)).astype(f32)
    v = rng.standard_normal((klen, dim)).astype(f32)
    segs = np.repeat(np.arange(4), (klen + 3) // 4)[:klen].astype(np.int32) if seg else None
    sp = segs.ctypes.data if seg else None
    out, lse = np.zeros((qlen, dim), f32), np.zeros(qlen, f32)
    be.AttentionForward(AttentionForwardParameters(q, k, v, qlen, klen, dim, offset, window, segs),
                        AttentionForwardResult(out, lse))
    wo, wl = np.zeros((qlen, dim), f32), np.zeros(qlen, f32)
    L.orc_attention_forward(q, k, v, wo, wl.ctypes.data, sp, klen if seg else 0, qlen, klen, dim,
                            offset, window)
    assert_close(out, wo, 2e-3, 1e-5, "AttentionForward")
    assert_close(lse, wl, 2e-3, 1e-5, "LogSumExp")
    # split-K shards + combine
    parts = []
    per = (klen + 2) // 3
    for s in range(3):
        r = AttentionSplitResult(np.zeros((qlen, dim), f32), np.zeros(qlen, f32), np.zeros(qlen, f32))
        be.AttentionForwardSplit(AttentionSplitParameters(q, k, v, qlen, klen, dim, offset, window,
                                                          s * per, min(klen, s * per + per), segs), r)
        wa, wm, ws = np.zeros((qlen, dim), f32), np.zeros(qlen, f32), np.zeros(qlen, f32)
        L.orc_attention_forward_split(q, k, v, wa, wm, ws, sp, klen if seg else 0, qlen, klen, dim,
                                      offset, window, s * per, min(klen, s * per + per))
        assert_close(r.Maximum, wm, 1e-4, 1e-5, "split max")
        assert_close(r.Sum, ws, 2e-3, 1e-5, "split sum")
        assert_close(r.Accumulator, wa, 2e-3, 1e-4, "split accumulator")
        parts.append(r)
    co, cl = np.zeros((qlen, dim), f32), np.zeros(qlen, f32)
    be.AttentionCombine(AttentionCombineParameters(parts, qlen, dim), AttentionForwardResult(co, cl))
    assert_close(co, wo, 2e-3, 1e-4, "combined output")
    # backward accumulates
    do = rng.standard_normal((qlen, dim)).astype(f32)
    init = [rng.standard_normal(x.shape).astype(f32) for x in (q, k, v)]
    got = [x.copy() for x in init]
    want = [x.copy() for x in init]
    be.AttentionBackward(AttentionBackwardParameters(q, k, v, wo, do, wl, qlen, klen, dim, offset,
                                                     window, None, segs),
                         AttentionBackwardResult(*got))
    L.orc_attention_backward(q, k, v, wo, do, wl, None, sp, klen if seg else 0, *want, qlen, klen,
                             dim, offset, window)
    for g, w, nm in zip(got, want, "qkv"):
        assert_close(g, w, 5e-3, 1e-4, "d" + nm)


@pytest.mark.parametrize("m,n,k", [(2000, 6000, 512), (4096, 3072, 768), (256, 12288, 1024)])
def test_matmul_wide_engine(be, m, n, k):
    """Products large enough for the 256 x 256-tile engine (at least 192
    workgroups): MatMulTransposed (x.W^T, both operands K-contiguous) and
    MatMul (B contiguous in N), against numpy in float64.  2000 x 6000
    leaves a partial last tile in both dimensions (loaded shifted back to
    end at M and N, the overlap not stored twice)."""
    rng = np.random.default_rng(m + n + k)
    a = rng.standard_normal((m, k)).astype(f32)
    b = rng.standard_normal((k, n)).astype(f32)
    want = a.astype(np.float64) @ b.astype(np.float64)
    got = np.zeros((m, n), f32)
    be.MatMul(got, a, b, m, n, k)
    assert_close(got, want, 1e-4, 1e-4, "MatMul")
    got2 = np.zeros((m, n), f32)
    be.MatMulTransposed(got2, a, np.ascontiguousarray(b.T), m, n, k)
    assert_close(got2, want, 1e-4, 1e-4, "MatMulTransposed")


@pytest.mark.parametrize("m,n,k", [(256, 3072, 768), (256, 768, 3072), (256, 1280, 768),
                                   (256, 768, 768), (32, 96, 32), (64, 480, 544),
                                   (512, 1280, 1280), (96, 640, 2048)])
@pytest.mark.parametrize("mode", ["1", None])
def test_matmul_slim_engine(be, monkeypatch, m, n, k, mode):
    """Decode-sized x.W^T products (M a multiple of 32 up to 1024, N a
    multiple of 96, 128 or 160): the slim-tile engine (GN_GEMM_SLIM=1: every
    eligible product; unset: the default choice between it and
    gemm_kernel), including K ranges that are not a whole number of ring
    rounds (32 x 96 x 32: one real K tile of eight, the rest zeros) and split
    K summed by the reduction kernel, against numpy in float64."""
    if mode is None:
        monkeypatch.delenv("GN_GEMM_SLIM", raising=False)
    else:
        monkeypatch.setenv("GN_GEMM_SLIM", mode)
    rng = np.random.default_rng(m * 7 + n + k)
    a = rng.standard_normal((m, k)).astype(f32)
    w = rng.standard_normal((n, k)).astype(f32)
    want = a.astype(np.float64) @ w.astype(np.float64).T
    got = np.zeros((m, n), f32)
    be.MatMulTransposed(got, a, w, m, n, k)
    assert_close(got, want, 1e-4, 1e-4, "MatMulTransposed")

"""The host contracts of the boundary (kernels/backend.go:8-20, the
reference's panics in tensors/ops.go:8-17) on the device:

* re-entrancy: the reference calls its backend from many goroutines at
  once (model/attention.go:311-320, tensors/loss.go:30-37); the gn_*
  primitives called from several host threads concurrently give the
  single-threaded results bit for bit;
* misuse returns a non-zero status with a message instead of crashing: bad
  shapes and ids, configs the reference's Validate rejects, an allocation
  beyond the device's memory (after which the thread and the device keep
  working);
* non-finite logits: rows with -Inf entries sample exactly as the oracle's;
  rows holding NaN -- where the reference's result follows the internals of
  Go's sort.Slice, which no restatement reproduces -- return a valid id
  without disturbing the other rows."""
import ctypes as C
import threading

import numpy as np
import pytest

from gonano_amd import config as G

pytestmark = pytest.mark.gpu


def _work(seed):
    """A few primitives on fixed inputs: MatMulTransposed, SoftmaxLastDim,
    RMSNormLastDim, AttentionForward, TopKIndices."""
    from gonano_amd.backend import HipBackend
    b = HipBackend()
    rng = np.random.default_rng(seed)
    a = rng.standard_normal((37, 96)).astype(np.float32)
    w = rng.standard_normal((53, 96)).astype(np.float32)
    out = {}
    d = np.zeros((37, 53), np.float32)
    b.MatMulTransposed(d, a, w, 37, 53, 96)
    out["mm"] = d
    s = np.zeros_like(a)
    b.SoftmaxLastDim(s, a, 37, 96)
    out["sm"] = s
    r = np.zeros_like(a)
    b.RMSNormLastDim(r, a, 37, 96, 1e-6)
    out["rms"] = r
    q = rng.standard_normal((20, 128)).astype(np.float32)
    k = rng.standard_normal((20, 128)).astype(np.float32)
    v = rng.standard_normal((20, 128)).astype(np.float32)
    from gonano_amd.backend import AttentionForwardParameters, AttentionForwardResult
    res = AttentionForwardResult(np.zeros((20, 128), np.float32), np.zeros(20, np.float32))
    b.AttentionForward(AttentionForwardParameters(q, k, v, 20, 20, 128), res)
    out["att"], out["lse"] = res.Output, res.LogSumExp
    idx = np.zeros((37, 5), np.int32)
    b.TopKIndices(idx, a, 37, 96, 5)
    out["topk"] = idx
    return out


def test_primitives_from_concurrent_threads():
    seeds = list(range(6))
    want = {sd: _work(sd) for sd in seeds}
    errors = []
    stop = threading.Event()

    def worker(tid):
        try:
            for it in range(8):
                if stop.is_set():
                    return
                sd = seeds[(tid + it) % len(seeds)]
                got = _work(sd)
                for key, val in want[sd].items():
                    if not np.array_equal(got[key], val):
                        errors.append((tid, it, sd, key))
                        stop.set()
                        return
        except Exception as e:  # noqa: BLE001
            errors.append((tid, repr(e)))
            stop.set()

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    assert not errors, errors[:5]


def test_bad_shapes_and_ids_return_status():
    from gonano_amd import _lib
    from gonano_amd.session import Session
    L = _lib.lib()
    a = np.ones(6, np.float32)
    d = np.zeros(6, np.float32)
    assert L.gn_matmul(d, a, a, -1, 2, 3) != 0 and L.gn_last_error()
    assert L.gn_softmax_last_dim(d, a, 2, -3) != 0 and L.gn_last_error()
    assert L.gn_rmsnorm_last_dim(d, a, -2, 3, 1e-6) != 0 and L.gn_last_error()
    i = np.zeros(6, np.int32)
    assert L.gn_topk_indices(i, a, 2, 3, -1) != 0 and L.gn_last_error()
    cfg = G.Config(sequence_len=256, vocab_size=512, n_layer=2, n_head=2, n_kv_head=1, n_embd=256,
                   window_pattern="SSSL", rotary_dims=64)
    w = G.init_weights(cfg, seed=1)
    with Session(cfg) as s:
        s.set_params(w)
        ids = np.zeros((1, 8), np.int32)
        bad_t = ids.copy()
        bad_t[0, 3] = cfg.vocab_size  # target outside the vocabulary
        with pytest.raises(_lib.HipError, match="out of range") as e:
            s.policy_gradient_step(ids, bad_t, np.ones(1, np.float32), 9.0)
        assert e.value.code == 1
        bad_i = ids.copy()
        bad_i[0, 0] = 10_000  # token outside the embedding table
        with pytest.raises(_lib.HipError, match="out of range"):
            s.forward(bad_i)
        with pytest.raises(_lib.HipError):  # longer than the rotary cache
            s.forward(np.zeros((1, cfg.sequence_len + 1), np.int32))
        with pytest.raises(_lib.HipError):  # context beyond the rotary table
            s.generate_batch(np.zeros((1, 8), np.int32), 2, cfg.sequence_len * 10, 1.0, 50,
                             np.zeros(1, np.uint64))
        # the session still works after the rejections
        assert np.isfinite(s.forward(ids)).all()
    for kw in (dict(n_embd=250), dict(n_kv_head=3), dict(n_head=4, n_embd=256)):
        bad = dict(sequence_len=64, vocab_size=64, n_layer=1, n_head=2, n_kv_head=1, n_embd=256,
                   window_pattern="L", rotary_dims=0)
        bad.update(kw)
        c = _lib.GnConfig(bad["sequence_len"], bad["vocab_size"], bad["n_layer"], bad["n_head"],
                          bad["n_kv_head"], bad["n_embd"], 0, b"L")
        h = C.c_void_p()
        assert L.gn_session_create(C.byref(c), 0, C.byref(h)) != 0, kw
        assert L.gn_last_error()


def test_allocation_beyond_device_memory_fails_cleanly():
    """A model whose parameters alone exceed the device's 288 GB (vocab 2^26
    at width 1024: 512 GiB of embeddings) is refused with GN_ERR_OOM at
    creation, before any kernel runs; the thread and the device keep
    working afterwards (the failed allocation's error does not resurface)."""
    from gonano_amd import _lib
    from gonano_amd.backend import HipBackend
    from gonano_amd.session import Session
    huge = G.Config(sequence_len=64, vocab_size=1 << 26, n_layer=1, n_head=8, n_kv_head=2,
                    n_embd=1024, window_pattern="L", rotary_dims=0)
    with pytest.raises(_lib.HipError) as e:
        Session(huge)
    assert e.value.code == 3, e.value
    d = np.zeros((4, 4), np.float32)
    HipBackend().MatMulTransposed(d, np.eye(4, dtype=np.float32), np.eye(4, dtype=np.float32),
                                  4, 4, 4)
    assert np.array_equal(d, np.eye(4))
    cfg = G.Config(sequence_len=64, vocab_size=256, n_layer=1, n_head=2, n_kv_head=1, n_embd=256,
                   window_pattern="L", rotary_dims=0)
    with Session(cfg) as s:
        s.set_params(G.init_weights(cfg, seed=2))
        assert np.isfinite(s.forward(np.zeros((1, 4), np.int32))).all()


def test_non_finite_logits(orc):
    from gonano_amd.backend import sample_next_token
    rng = np.random.default_rng(5)
    V = 4096
    z = rng.standard_normal((6, V)).astype(np.float32)
    z[1, ::3] = -np.inf                 # a caller's masked entries
    z[2, :V - 10] = -np.inf             # fewer finite entries than k
    z[3, 17] = np.inf                   # one +Inf entry wins
    z[4, 5] = np.nan
    z[5, :] = np.nan
    clean = [0, 1, 2, 3]
    for T, k in ((1.0, 50), (0.0, 50), (0.8, 0)):
        g = orc.GoRNG(77)
        st = np.array(g.hi_lo, np.uint64)
        got = sample_next_token(z, st, T, k)
        assert np.all((got >= 0) & (got < V)), got
        # the clean rows draw from their own stream positions: compare each
        for r in clean:
            gr = orc.GoRNG(77)
            if T > 0:
                gr.advance(r * V)
            want = orc.sample_next_token(z[r:r + 1], gr, T, k)[0]
            assert got[r] == want, (T, k, r, got[r], want)
        assert got[3] == 17
        assert tuple(int(x) for x in st) == (g.hi_lo if T <= 0 else _advanced(orc, 77, 6 * V))


def _advanced(orc, seed, n):
    g = orc.GoRNG(seed)
    g.advance(n)
    return g.hi_lo

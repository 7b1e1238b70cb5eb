"""The allocation-free sampler entry point (gn_sample_next_token_static)
against gn_sample_next_token through the C-ABI: bit-exact sampled ids and
the same advanced RNG state on two calls in a row, the second smaller than
the first (the static staging array keeps the first call's contents),
calls from eight threads at once (the library serializes them on the
device's lock), plus the size limits it rejects without touching the
GPU."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _case(rng, rows, vocab):
    z = (rng.standard_normal((rows, vocab)) * 2).astype(np.float32)
    z[:, ::97] = z[:, :1]  # ties at and around the threshold
    return np.round(z * 64).astype(np.float32) / 64


def test_static_sampler_matches_allocating_entry_point():
    from gonano_amd.backend import sample_next_token, sample_next_token_static
    rng = np.random.default_rng(21)
    # the first call fills most of the static array; the second, smaller one
    # must not see the first call's logits, ids or state
    for rows, vocab, temp, k, seed in [(256, 65536, 1.0, 50, 7), (3, 4096, 0.8, 20, 12345),
                                       (5, 1000, 0.0, 50, 1)]:
        z = _case(rng, rows, vocab)
        a = np.array([seed, seed ^ 0x9E3779B97F4A7C15], np.uint64)
        b = a.copy()
        want = sample_next_token(z, a, temp, k)
        got = sample_next_token_static(z, b, temp, k)
        assert np.array_equal(got, want), (rows, vocab, np.nonzero(got != want))
        assert np.array_equal(a, b)


def test_static_sampler_concurrent_threads():
    """Eight threads sample different logits through the one staging array
    at the same time; each gets exactly the ids and state the allocating
    entry point gives for its own inputs."""
    import threading
    from gonano_amd.backend import sample_next_token, sample_next_token_static
    rng = np.random.default_rng(33)
    cases = [(_case(rng, 64 + 16 * i, 4096 * (1 + i % 4)), 1000 + i) for i in range(8)]
    want, got, states = {}, {}, {}
    for i, (z, seed) in enumerate(cases):
        a = np.array([seed, seed * 3 + 1], np.uint64)
        want[i] = (sample_next_token(z, a, 1.0, 50), a.copy())

    def work(i):
        z, seed = cases[i]
        for _ in range(5):
            b = np.array([seed, seed * 3 + 1], np.uint64)
            got.setdefault(i, []).append((sample_next_token_static(z, b, 1.0, 50), b.copy()))

    threads = [threading.Thread(target=work, args=(i,)) for i in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for i in range(8):
        assert len(got[i]) == 5
        for ids, st in got[i]:
            assert np.array_equal(ids, want[i][0]), i
            assert np.array_equal(st, want[i][1]), i


def test_static_sampler_rejects_sizes_beyond_its_buffer():
    from gonano_amd import _lib
    from gonano_amd.backend import sample_next_token_static
    st = np.array([1, 2], np.uint64)
    with pytest.raises(_lib.HipError) as e:
        sample_next_token_static(np.zeros((257, 65536), np.float32), st, 1.0, 50)
    assert e.value.code == 1 and "static buffer" in str(e.value)
    with pytest.raises(_lib.HipError) as e:
        sample_next_token_static(np.zeros((65537, 1), np.float32), st, 1.0, 50)
    assert e.value.code == 1
    assert st.tolist() == [1, 2]

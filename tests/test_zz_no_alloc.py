"""The allocation-free sampler entry point (gn_sample_next_token_static)
against gn_sample_next_token through the C-ABI: bit-exact sampled ids and
the same advanced RNG state on two calls in a row, the second smaller than
the first (the static staging array keeps the first call's contents), plus
the size limits it rejects without touching the GPU."""
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

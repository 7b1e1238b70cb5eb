"""The device prefix cache in the rollout prefill: Engine.Cache / Engine.Prefix
(inference/engine.go:44-51, 120-173) over CacheManager (inference/cache.go)
and PrefixCache (inference/prefix.go).

* A prompt whose longest stored strict prefix has m tokens prefills only its
  last P - m tokens against the stored keys/values, decode-cache rows and
  previous-token embedding; every column of every row it then samples is
  checked against the oracle's full prefill by teacher forcing, for
  continuations over a sliding-window boundary, of one token (the smear
  seeded alone) and of a longer stored extension (the longest prefix wins),
  on a dense model, a latent-attention MoE model and two compressed-attention
  models (stored prefixes ending inside a compressed block; one with
  hierarchical sparse selection, one with MoE), whose continuations compress
  the whole sequences from the stored compressor logits.
* The bookkeeping -- strict and longest prefix, LRU order, MaxEntries,
  MaxBytes, TTL from storage, maxPrefix, Invalidate, a batch seen as
  successive calls -- follows the reference's cache.go/prefix.go, checked by
  hand-written sequences (cache_test.go's cases) and against a restatement
  of CacheManager over a random sequence of calls.
"""
import time

import numpy as np
import pytest

from gonano_amd import config as G
from tf_check import teacher_forced_group

pytestmark = pytest.mark.gpu


def _dense():
    # window pattern SSSL at sequence_len 512: short windows of 128 tokens
    return G.Config(sequence_len=512, vocab_size=2048, n_layer=2, n_head=2, n_kv_head=1,
                    n_embd=256, window_pattern="SSSL", rotary_dims=64)


def _latent():
    cfg = G.config_for_depth_ratio(4, 2048, 64, 128, 512, "SSSL", 1)
    cfg.n_layer = 2
    return G.apply_latent_preset(cfg, mla_latent=128, n_experts=4, experts_per_token=2,
                                 expert_hidden=256)


def _compressed_sparse():
    # compressed attention (ratio 4, SWA 64) with hierarchical top-3 selection
    # and a Full / Reindex / Reuse layer group; no encoder-decoder split
    cfg = G.Config(sequence_len=512, vocab_size=2048, n_layer=3, n_head=2, n_kv_head=1,
                   n_embd=256, window_pattern="SSSL", rotary_dims=64, compression_ratio=4,
                   swa_window=64, sparse_topk=3, indexer_pool=2, indexer_candidates=8,
                   indexer_dim=16, reuse_pattern="FRU")
    cfg.validate()
    return cfg


def _compressed():
    # compressed attention over every earlier block (no selection), a Full and
    # a Reuse layer, with the DeepSeekMoE feed-forward
    cfg = G.Config(sequence_len=512, vocab_size=2048, n_layer=2, n_head=2, n_kv_head=1,
                   n_embd=256, window_pattern="SSSL", rotary_dims=64, compression_ratio=4,
                   swa_window=64, reuse_pattern="FU")
    cfg = G.enable_moe(cfg, n_experts=4, experts_per_token=2, expert_hidden=64,
                       shared_hidden=96, balance_weight=1e-2)
    cfg.validate()
    return cfg


@pytest.mark.parametrize("make,perturb", [(_dense, 0.1), (_latent, 0.05), (_compressed_sparse, 0.1),
                                          (_compressed, 0.1)],
                         ids=["dense", "latent", "compressed_sparse", "compressed"])
def test_cached_continuation_matches_full_prefill(orc, make, perturb):
    from gonano_amd.session import Session
    cfg = make()
    w = G.init_weights(cfg, seed=23, perturb=perturb)
    V = cfg.vocab_size
    rng = np.random.default_rng(41)
    base = rng.integers(0, V, (3, 150)).astype(np.int32)
    # call 2: base 0 and 2 extended by 90 tokens (the continuation's queries
    # see keys across the 128-token window), a fresh prompt, base 0 extended
    # differently
    ext = np.concatenate([base[[0, 1, 2, 0]], rng.integers(0, V, (4, 90))], axis=1).astype(np.int32)
    ext[1] = rng.integers(0, V, 240)
    # call 3: one-token continuations of two stored extensions (240 beats
    # 150), and base 1 extended by 91
    last = np.concatenate([ext[[0, 3]], rng.integers(0, V, (2, 1))], axis=1).astype(np.int32)
    third = np.concatenate([base[[1]], rng.integers(0, V, (1, 91))], axis=1).astype(np.int32)
    calls = [(base, [0, 0, 0]), (ext, [150, 0, 150, 150]),
             (np.concatenate([last, third]), [240, 240, 150])]
    S, N = 3, 6
    out = []
    with Session(cfg) as s:
        s.set_params(w)
        s.set_prefix_cache(max_entries=16)
        for i, (prompts, want_hits) in enumerate(calls):
            seeds = (100 * i + np.arange(len(prompts))).astype(np.uint64)
            rows = s.generate_batch(prompts, S, N, 1.0, 50, seeds)
            assert s.prefix_cache_hits(len(prompts)).tolist() == want_hits, i
            out.append((prompts, seeds, rows))
        assert s.prefix_cache_len()[0] == 3 + 4 + 3
    m = orc.OracleModel(orc.ModelShape.from_config(cfg), w)
    checked = 0
    for prompts, seeds, rows in out:
        for g in range(len(prompts)):
            checked += teacher_forced_group(orc, m, prompts[g], rows[g * S:(g + 1) * S], seeds[g],
                                            N, 1.0, 50)
    assert checked >= 10 * S * 4


class _CacheManager:
    """inference/cache.go CacheManager (in-memory tier) restated over token
    tuples, without limits other than MaxEntries: Lookup (79-119), Store
    (121-161), evictLocked (216-231)."""

    def __init__(self, max_entries=0):
        self.max_entries = max_entries
        self.order = []  # oldest first

    def lookup(self, toks):
        best = None
        for e in self.order:
            if 0 < len(e) < len(toks) and (best is None or len(e) > len(best)) and \
                    tuple(toks[:len(e)]) == e:
                best = e
        if best is None:
            return 0
        self.order.remove(best)
        self.order.append(best)
        return len(best)

    def store(self, toks):
        t = tuple(toks)
        if t in self.order:
            self.order.remove(t)
        self.order.append(t)
        while self.max_entries and len(self.order) > self.max_entries:
            self.order.pop(0)


def _small():
    return G.Config(sequence_len=128, vocab_size=64, n_layer=1, n_head=2, n_kv_head=1,
                    n_embd=256, window_pattern="L", rotary_dims=0)


def _call(s, prompts, n=1):
    prompts = np.asarray(prompts, np.int32).reshape(len(prompts), -1)
    s.generate_batch(prompts, 1, n, 1.0, 0, np.arange(len(prompts), dtype=np.uint64))
    return s.prefix_cache_hits(len(prompts)).tolist()


def test_lookup_store_and_eviction():
    """cache_test.go's cases on the device cache: a strict prefix only, the
    longest prefix, LRU eviction by count, replacement of an equal prompt,
    Invalidate, and dropping every entry when the parameters change."""
    from gonano_amd.session import Session
    cfg = _small()
    a = list(range(1, 9))
    with Session(cfg) as s:
        s.set_params(G.init_weights(cfg, seed=4, perturb=0.1))
        assert _call(s, [a]) == [0]                       # the cache is off: nothing stored
        assert s.prefix_cache_len() == (0, 0)
        s.set_prefix_cache(max_entries=2)
        assert _call(s, [a]) == [0]
        n, b1 = s.prefix_cache_len()
        assert n == 1 and b1 > 0
        assert _call(s, [a]) == [0]                       # equal, not a strict prefix: replaced
        assert s.prefix_cache_len()[0] == 1
        assert _call(s, [a + [9, 10]]) == [8]
        assert _call(s, [a + [9, 10, 11]]) == [10]        # the longest prefix wins
        # LRU: order is now a+[9,10], a+[9,10,11]; a was evicted by count
        assert _call(s, [a + [12]]) == [0]
        assert _call(s, [a + [9, 10, 11, 12]]) == [11]
        assert _call(s, [[5] + a], n=0) == [0]           # max_tokens 0 still stores
        assert s.prefix_cache_len()[0] == 2
        s.prefix_cache_invalidate()
        assert s.prefix_cache_len() == (0, 0)
        assert _call(s, [a]) == [0] and _call(s, [a + [9]]) == [8]
        s.set_params(G.init_weights(cfg, seed=5, perturb=0.1))  # new weights: entries dropped
        assert s.prefix_cache_len() == (0, 0)
        assert _call(s, [a + [9, 10]]) == [0]
        s.set_prefix_cache(enabled=False)
        assert s.prefix_cache_len() == (0, 0)


def test_bytes_ttl_and_max_prefix():
    """MaxBytes evicts least recently used entries (the new one too when it
    alone is too large); TTL expires an entry counted from its storage
    (a hit does not renew it); maxPrefix keeps longer entries from hitting
    (prefix.go:38-60)."""
    from gonano_amd.session import Session
    cfg = _small()
    a = list(range(1, 9))
    with Session(cfg) as s:
        s.set_params(G.init_weights(cfg, seed=4, perturb=0.1))
        s.set_prefix_cache()
        _call(s, [a])
        b8 = s.prefix_cache_len()[1]
        _call(s, [a + [9, 10, 11, 12, 13, 14, 15, 16]])
        b16 = s.prefix_cache_len()[1] - b8
        assert b16 > b8
        s.prefix_cache_invalidate()
        s.set_prefix_cache(max_bytes=b8 + b16)
        _call(s, [a])
        _call(s, [a + list(range(20, 28))])
        assert s.prefix_cache_len() == (2, b8 + b16)
        _call(s, [list(range(30, 38))])                 # 3 entries do not fit: the oldest goes
        assert s.prefix_cache_len() == (2, b8 + b16)
        assert _call(s, [a + [50]]) == [0]
        s.set_prefix_cache(max_bytes=b8 - 1)            # smaller than any entry: all evicted
        assert s.prefix_cache_len() == (0, 0)
        _call(s, [a])
        assert s.prefix_cache_len() == (0, 0)
        s.set_prefix_cache(ttl=2.0)
        _call(s, [a])
        time.sleep(1.2)
        assert _call(s, [a + [9]]) == [8]               # a hit does not renew the entry
        time.sleep(1.2)
        assert _call(s, [a + [10]]) == [0]
        assert s.prefix_cache_len()[0] == 2             # a+[9] and a+[10], a expired
        s.set_prefix_cache(enabled=False)
        s.set_prefix_cache(max_entries=1, max_prefix=6)  # NewPrefixCache(6)
        _call(s, [a])
        assert _call(s, [a + [9]]) == [0]
        _call(s, [a[:5]])
        assert _call(s, [a[:5] + [7, 7]]) == [5]


def test_batch_is_seen_as_successive_calls_and_random_sequence():
    """A batch of prompts uses the cache as successive GenerateWith calls
    would: an earlier group's store evicts the entry a later group would have
    hit.  Then a random sequence of calls against the restated CacheManager."""
    from gonano_amd.session import Session
    cfg = _small()
    a = list(range(1, 9))
    with Session(cfg) as s:
        s.set_params(G.init_weights(cfg, seed=4, perturb=0.1))
        s.set_prefix_cache(max_entries=1)
        _call(s, [a])
        assert _call(s, [list(range(20, 30)), a + [1, 2]]) == [0, 0]
        s.set_prefix_cache(max_entries=2)
        s.prefix_cache_invalidate()
        _call(s, [a])
        assert _call(s, [list(range(20, 30)), a + [1, 2]]) == [0, 8]
        s.set_prefix_cache(enabled=False)

        rng = np.random.default_rng(8)
        bases = [list(rng.integers(0, 64, 6)) for _ in range(3)]
        s.set_prefix_cache(max_entries=4)
        ref = _CacheManager(max_entries=4)
        for it in range(40):
            G_ = int(rng.integers(1, 4))
            P = int(rng.integers(6, 13))
            prompts = []
            for _ in range(G_):
                b = bases[int(rng.integers(0, 3))]
                tail = [int(x) for x in rng.integers(0, 3, P - 6)]  # few symbols: many matches
                prompts.append(b + tail)
            want = []
            for p in prompts:
                want.append(ref.lookup(p))
                ref.store(p)
            assert _call(s, prompts) == want, it
            assert s.prefix_cache_len()[0] == len(ref.order), it


def test_rl_step_uses_the_cache_and_unsupported_models():
    """gn_rl_step prefills through the cache too (its rollout is
    GenerateBatchWith); CED models refuse it (the reference's engine skips
    them), the same compressed model without CED takes it."""
    from gonano_amd import _lib
    from gonano_amd.session import Session
    cfg = _small()
    with Session(cfg) as s:
        s.set_params(G.init_weights(cfg, seed=4, perturb=0.1))
        s.set_prefix_cache()
        s.zero_grad()
        p = np.arange(1, 11, dtype=np.int32).reshape(1, 10)
        s.rl_step(p, 2, 3, 1.0, 0, np.array([3], np.uint64), np.array([1, 0], np.float32))
        s.rl_step(np.concatenate([p, [[7, 7]]], axis=1).astype(np.int32), 2, 3, 1.0, 0,
                  np.array([3], np.uint64), np.array([1, 0], np.float32))
        assert s.prefix_cache_hits(1).tolist() == [10]
    fl = G.config_for_depth_ratio(4, 2048, 64, 128, 512, "SSSL", 1)
    fl.n_layer = 2
    G.apply_flash_preset(fl, sparse_topk=4, swa_window=128, n_experts=4)
    assert fl.ced
    with Session(fl) as s:
        with pytest.raises(_lib.HipError) as e:
            s.set_prefix_cache()
        assert e.value.code == 4
    fl.ced = False  # the same compressed model without the encoder-decoder split
    with Session(fl) as s:
        s.set_prefix_cache()
        assert s.prefix_cache_len() == (0, 0)


def test_disk_tier(tmp_path):
    """CacheOptions.DiskDir (cache.go:25-28, 145-150, 254-284): entries are
    written to the directory and read back for the call that hits them, with
    the same results as the device-memory tier (bit for bit: the state makes
    the round trip unchanged); eviction, a replaced prompt and invalidation
    delete the files; a file that cannot be read (here: truncated) drops its
    entry and the lookup misses.  On a compressed-attention model, whose
    entries carry the compressor logits."""
    from gonano_amd.session import Session
    cfg = _compressed_sparse()
    w = G.init_weights(cfg, seed=23, perturb=0.1)
    V = cfg.vocab_size
    rng = np.random.default_rng(5)
    base = rng.integers(0, V, (2, 70)).astype(np.int32)
    ext = np.concatenate([base, rng.integers(0, V, (2, 30))], axis=1).astype(np.int32)
    calls = [base, ext, np.concatenate([ext, rng.integers(0, V, (2, 5))], axis=1).astype(np.int32)]
    results = {}
    for tier in ("memory", "disk"):
        d = tmp_path / "kv"
        with Session(cfg) as s:
            s.set_params(w)
            s.set_prefix_cache(max_entries=8, disk_dir=str(d) if tier == "disk" else "")
            out = []
            for i, prompts in enumerate(calls):
                rows = s.generate_batch(prompts, 2, 4, 1.0, 50,
                                        (10 * i + np.arange(2)).astype(np.uint64))
                out.append((rows, s.prefix_cache_hits(2).tolist(), s.prefix_cache_len()))
                if tier == "disk":
                    assert len(list(d.iterdir())) == s.prefix_cache_len()[0] == 2 * (i + 1)
            results[tier] = out
            if tier == "disk":
                # a truncated file: its entry is dropped and the prompt misses
                f = sorted(d.iterdir(), key=lambda p: p.stat().st_mtime)[-1]
                f.write_bytes(f.read_bytes()[:100])
                n0 = s.prefix_cache_len()[0]
                probe = np.concatenate([calls[2], rng.integers(0, V, (2, 1))], axis=1)
                s.generate_batch(probe.astype(np.int32), 1, 1, 1.0, 50, np.arange(2, dtype=np.uint64))
                assert sorted(s.prefix_cache_hits(2).tolist()) == [0, 105]
                assert s.prefix_cache_len()[0] == n0 - 1 + 2
                # eviction deletes files
                s.set_prefix_cache(max_entries=3, disk_dir=str(d))
                assert s.prefix_cache_len()[0] == 3 and len(list(d.iterdir())) == 3
                s.prefix_cache_invalidate()
                assert s.prefix_cache_len() == (0, 0) and not list(d.iterdir())
    for (ra, ha, la), (rb, hb, lb) in zip(results["memory"], results["disk"]):
        assert ha == hb and la == lb
        assert np.array_equal(ra, rb)
    assert [h for _, h, _ in results["disk"]] == [[0, 0], [70, 70], [100, 100]]

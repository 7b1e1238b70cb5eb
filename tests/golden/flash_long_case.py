"""The flash long-prompt parity case shared by tests/golden/make_flash_long.py
(which writes the oracle's results into flash_long.npz) and the GPU test
(tests/test_gpu_flash_long.py): the model, its weights and the inputs."""
import numpy as np

from gonano_amd import config as G

P, S, N, T_PG, GSAMPLE, TOPN = 8192, 16, 4, 8703, 256, 64
SEED_GROUP, ADV = 1000, 0.3


def config():
    """The flash d12 preset (6:1 heads, compression 4, top-16 sparse selection
    over 128 candidates, SWA 512, FRU reuse, CED, 16 experts of 768,
    SequenceLen 16384) at 3 layers (one Full, one Reindex, one Reuse layer)
    and V = 4096."""
    cfg = G.config_for_depth_ratio(12, 4096, 64, 128, 16384, "SSSL", 1)
    cfg.n_kv_head = 1
    cfg.n_layer = 3
    return G.apply_flash_preset(cfg, sparse_topk=16, swa_window=512, n_experts=16)


def weights(cfg):
    return G.init_weights(cfg, seed=41, perturb=0.02)


def inputs(cfg):
    """The 8192-token prompt, and the policy-gradient sequence: the prompt,
    511 more tokens, targets only after the prompt."""
    rng = np.random.default_rng(5)
    prompt = rng.integers(0, cfg.vocab_size, P).astype(np.int32)
    tail = rng.integers(0, cfg.vocab_size, T_PG - P).astype(np.int32)
    pg_in = np.concatenate([prompt, tail])[None, :]
    pg_tg = rng.integers(0, cfg.vocab_size, (1, T_PG)).astype(np.int32)
    pg_tg[:, :P] = -1
    return prompt, pg_in, pg_tg


def sample_indices(cfg):
    """Per parameter tensor, the GSAMPLE gradient entries the fixture keeps."""
    out = []
    for i, (name, r, c, off) in enumerate(cfg.param_table()):
        n = r * c
        out.append(np.sort(np.random.default_rng(i).choice(n, min(GSAMPLE, n), replace=False)))
    return out

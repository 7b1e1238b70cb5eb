"""ctypes wrapper over oracle/liboracle.so, the CPU restatement of gonano's
RL-step arithmetic.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker.  The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i32pn = C.c_void_p  # optional int32 array: pass _ptr(array) or None
_u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
_i64 = C.c_int64


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


class OrcConfig(C.Structure):
    _fields_ = [
        ("sequence_len", C.c_int32),
        ("vocab_size", C.c_int32),
        ("n_layer", C.c_int32),
        ("n_head", C.c_int32),
        ("n_kv_head", C.c_int32),
        ("n_embd", C.c_int32),
        ("rotary_dims", C.c_int32),
        ("window_pattern", C.c_char * 16),
        ("mla_latent", C.c_int32),
        ("mla_rope_dims", C.c_int32),
        ("n_experts", C.c_int32),
        ("experts_per_token", C.c_int32),
        ("expert_hidden", C.c_int32),
        ("shared_hidden", C.c_int32),
        ("moe_clamp", C.c_float),
        ("moe_scale", C.c_float),
        ("balance_weight", C.c_float),
        ("compression_ratio", C.c_int32),
        ("swa_window", C.c_int32),
        ("sparse_topk", C.c_int32),
        ("indexer_dim", C.c_int32),
        ("indexer_heads", C.c_int32),
        ("indexer_pool", C.c_int32),
        ("indexer_candidates", C.c_int32),
        ("indexer_weight", C.c_float),
        ("reuse_pattern", C.c_char * 16),
        ("ced", C.c_int32),
    ]


class OrcPCG(C.Structure):
    _fields_ = [("hi", C.c_uint64), ("lo", C.c_uint64)]


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        build()
    L = C.CDLL(LIB_PATH)
    v = None
    sig = {
        "orc_opt_state_floats": (C.c_int64, [C.c_void_p, C.c_int]),
        "orc_opt_step": (v, [_f32p, _f32p, C.c_void_p, C.c_int, _f32p, _i32p]),
        "orc_polar_express": (v, [_f32p, _i64, _i64, C.c_int]),
        "orc_add": (v, [_f32p, _f32p, _f32p, _i64]),
        "orc_subtract": (v, [_f32p, _f32p, _f32p, _i64]),
        "orc_multiply": (v, [_f32p, _f32p, _f32p, _i64]),
        "orc_divide": (v, [_f32p, _f32p, _f32p, _i64]),
        "orc_scale": (v, [_f32p, _f32p, C.c_float, _i64]),
        "orc_add_scaled": (v, [_f32p, _f32p, _f32p, C.c_float, _i64]),
        "orc_negate": (v, [_f32p, _f32p, _i64]),
        "orc_abs": (v, [_f32p, _f32p, _i64]),
        "orc_square": (v, [_f32p, _f32p, _i64]),
        "orc_relu_squared": (v, [_f32p, _f32p, _i64]),
        "orc_swiglu": (v, [_f32p, _f32p, _f32p, C.c_float, _i64]),
        "orc_swiglu_backward": (v, [_f32p, _f32p, _f32p, _f32p, _f32p, C.c_float, _i64]),
        "orc_exp": (v, [_f32p, _f32p, _i64]),
        "orc_sigmoid": (v, [_f32p, _f32p, _i64]),
        "orc_tanh": (v, [_f32p, _f32p, _i64]),
        "orc_rsqrt": (v, [_f32p, _f32p, _i64]),
        "orc_sum": (C.c_float, [_f32p, _i64]),
        "orc_max": (C.c_float, [_f32p, _i64]),
        "orc_argmax": (C.c_int64, [_f32p, _i64]),
        "orc_matmul": (v, [_f32p, _f32p, _f32p, _i64, _i64, _i64]),
        "orc_matmul_transposed": (v, [_f32p, _f32p, _f32p, _i64, _i64, _i64]),
        "orc_dot": (C.c_float, [_f32p, _f32p, _i64]),
        "orc_softmax_last_dim": (v, [_f32p, _f32p, _i64, _i64]),
        "orc_rmsnorm_last_dim": (v, [_f32p, _f32p, _i64, _i64, C.c_float]),
        "orc_indexer_scores": (v, [_f32p, _f32p, _f32p, _f32p, _i64, _i64, _i64, _i64]),
        "orc_indexer_block_max": (v, [_f32p, _f32p, _i64, _i64, _i64]),
        "orc_topk_indices": (v, [_i32p, _f32p, _i64, _i64, _i64]),
        "orc_moe_gate_topk": (v, [_f32p, _f32p, _f32p, _i32p, _f32p, _i64, _i64, _i64]),
        "orc_grouped_matmul_transposed": (v, [_f32p, _f32p, _f32p, _i32p, _i64, _i64, _i64]),
        "orc_attention_forward": (v, [_f32p, _f32p, _f32p, _f32p, C.c_void_p, C.c_void_p, _i64,
                                      _i64, _i64, _i64, _i64, _i64]),
        "orc_attention_backward": (v, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, C.c_void_p,
                                       C.c_void_p, _i64, _f32p, _f32p, _f32p, _i64, _i64, _i64,
                                       _i64, _i64]),
        "orc_attention_forward_split": (v, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, C.c_void_p,
                                            _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64]),
        "orc_attention_combine": (v, [_f32p, _f32p, _f32p, _i64, _f32p, C.c_void_p, _i64, _i64]),
        "orc_rng_new": (v, [C.POINTER(OrcPCG), C.c_uint64]),
        "orc_rng_uint64": (C.c_uint64, [C.POINTER(OrcPCG)]),
        "orc_rng_float32": (C.c_float, [C.POINTER(OrcPCG)]),
        "orc_rng_advance": (v, [C.POINTER(OrcPCG), C.c_uint64, C.c_uint64]),
        "orc_kth_largest": (C.c_float, [_f32p, _i64, _i64]),
        "orc_sample_multinomial": (C.c_int64, [C.POINTER(OrcPCG), _f32p, _i64, C.c_float]),
        "orc_sample_next_token": (v, [_f32p, _i64, _i64, C.POINTER(OrcPCG), C.c_float, _i64, _i32p]),
        "orc_gumbel_from_uniform": (C.c_float, [C.c_float]),
        "orc_calculator": (C.c_int, [C.c_char_p, C.c_char_p, C.c_size_t]),
        "orc_param_count": (C.c_int, [C.POINTER(OrcConfig)]),
        "orc_param_info": (C.c_int64, [C.POINTER(OrcConfig), C.c_int, C.c_char_p,
                                       C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "orc_param_total": (C.c_int64, [C.POINTER(OrcConfig)]),
        "orc_window_sizes": (v, [C.POINTER(OrcConfig), _i32p]),
        "orc_num_threads": (C.c_int, []),
        "orc_aux_loss_f32": (C.c_double, [C.c_void_p]),
        "orc_indexer_topk": (C.c_int, [_f32p, C.c_int, C.c_int, _i32p]),
        "orc_indexer_scores_rows": (v, [_f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                                        _f32p]),
        "orc_select_rows": (v, [_f32p] + [C.c_int] * 9 + [_i32p, _i32p, _i32pn, _i32pn]),
        "orc_fine_select": (v, [_f32p, _f32p, _f32p, C.c_int, C.c_int, _i32p, C.c_int, C.c_int,
                                C.c_int, _i32p, _i32p]),
        "orc_restrict_to_pool": (v, [_f32p, _f32p, C.c_int, C.c_int, _i32p, _i32p, C.c_int]),
        "orc_set_freeze_targets_f32": (v, [C.c_void_p, C.c_int]),
        "orc_set_freeze_targets_f64": (v, [C.c_void_p, C.c_int]),
        "orc_distill_loss_f32": (C.c_double, [C.c_void_p]),
        "orc_model_set_params_f32": (v, [C.c_void_p, _f32p]),
        "orc_prefill_ced_f32": (v, [C.c_void_p, _i32p, C.c_int, _f32p]),
        "orc_prefill_ced_f64": (v, [C.c_void_p, _i32p, C.c_int, _f64p]),
        "orc_model_set_params_f64": (v, [C.c_void_p, _f64p]),
        "orc_distill_loss_f64": (C.c_double, [C.c_void_p]),
        "orc_channel_compress": (v, [C.c_int, C.c_int, C.c_int, _f32p, _f32p, _f32p, _f32p]),
        "orc_merge_attention_rows": (v, [_f32p, _f32p, _f32p, _f32p, _f32p, _f32p, C.c_int,
                                         C.c_int]),
        "orc_aux_loss_f64": (C.c_double, [C.c_void_p]),
    }
    for sfx, fp in (("_f32", _f32p), ("_f64", _f64p)):
        sig.update({
            "orc_model_new" + sfx: (C.c_void_p, [C.POINTER(OrcConfig), fp]),
            "orc_model_free" + sfx: (v, [C.c_void_p]),
            "orc_forward" + sfx: (v, [C.c_void_p, _i32p, C.c_int, C.c_int, fp]),
            "orc_forward_decode" + sfx: (v, [C.c_void_p, _i32p, C.c_int, C.c_int, C.c_int, fp]),
            "orc_pg_step" + sfx: (C.c_double, [C.c_void_p, _i32p, _i32p, C.c_int, C.c_int, _f32p,
                                               C.c_float, fp, fp]),
            "orc_ce_loss" + sfx: (C.c_double, [C.c_void_p, _i32p, _i32p, C.c_int, C.c_int,
                                               C.c_void_p]),
            "orc_distill_step" + sfx: (C.c_double, [C.c_void_p, _f32p, _i32p, C.c_void_p, C.c_int,
                                                    C.c_int, C.c_float, C.c_int, fp]),
            "orc_generate_batch" + sfx: (v, [C.c_void_p, _i32p, C.c_int, C.c_int, C.c_int,
                                             C.c_float, C.c_int, C.c_uint64, _i32p, _i32p]),
            "orc_decode_forced" + sfx: (v, [C.c_void_p, _i32p, C.c_int, C.c_int, _i32p, C.c_int,
                                            fp]),
            "orc_rotary_table" + sfx: (v, [C.c_int, C.c_int, fp, fp]),
            "orc_apply_rotary" + sfx: (v, [fp, fp, C.c_int, C.c_int, C.c_int, fp, fp]),
            "orc_rl_step" + sfx: (C.c_double, [C.c_void_p, _i32p, C.c_int, C.c_int, C.c_int,
                                               C.c_int, C.c_float, C.c_int, _u64p, _f32p, _i32p,
                                               _i32p, _f32p, C.POINTER(C.c_int32), _i32p, _i32p,
                                               fp, fp]),
        })
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _ptr(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------------------
# Config helpers (model/config.go restated for the test side)
# ---------------------------------------------------------------------------
@dataclass
class ModelShape:
    sequence_len: int
    vocab_size: int
    n_layer: int
    n_head: int
    n_kv_head: int
    n_embd: int
    rotary_dims: int
    window_pattern: str
    # latent preset, resolved (0 = dense): see gonano_amd.config.Config
    mla_latent: int = 0
    mla_rope_dims: int = 0
    n_experts: int = 0
    experts_per_token: int = 0
    expert_hidden: int = 0
    shared_hidden: int = 0
    moe_clamp: float = 0.0
    moe_scale: float = 0.0
    balance_weight: float = 0.0
    compression_ratio: int = 0
    swa_window: int = 0
    # flash preset: CSA indexer, cross-layer reuse, CED
    sparse_topk: int = 0
    indexer_dim: int = 0
    indexer_heads: int = 0
    indexer_pool: int = 0
    indexer_candidates: int = 0
    indexer_weight: float = 0.0
    reuse_pattern: str = ""
    ced: int = 0

    @classmethod
    def from_config(cls, cfg) -> "ModelShape":
        """The oracle's shape of a gonano_amd.config.Config."""
        return cls(cfg.sequence_len, cfg.vocab_size, cfg.n_layer, cfg.n_head, cfg.n_kv_head,
                   cfg.n_embd, cfg.rotary_dims, cfg.window_pattern, cfg.mla_latent,
                   cfg.mla_rope_dimension if cfg.mla_latent > 0 else 0, cfg.n_experts,
                   cfg.experts_per_token, cfg.expert_hidden, cfg.shared_hidden, cfg.moe_clamp,
                   cfg.moe_scale, cfg.balance_weight, cfg.compression_ratio, cfg.swa_window,
                   cfg.sparse_topk, cfg.indexer_dim, cfg.indexer_heads, cfg.indexer_pool,
                   cfg.indexer_candidates, cfg.indexer_weight, cfg.reuse_pattern, int(cfg.ced))

    def orc(self) -> OrcConfig:
        return OrcConfig(self.sequence_len, self.vocab_size, self.n_layer, self.n_head,
                         self.n_kv_head, self.n_embd, self.rotary_dims,
                         self.window_pattern.encode(), self.mla_latent, self.mla_rope_dims,
                         self.n_experts, self.experts_per_token, self.expert_hidden,
                         self.shared_hidden, self.moe_clamp, self.moe_scale,
                         self.balance_weight, self.compression_ratio, self.swa_window,
                         self.sparse_topk, self.indexer_dim, self.indexer_heads,
                         self.indexer_pool, self.indexer_candidates, self.indexer_weight,
                         self.reuse_pattern.encode(), self.ced)


def param_table(shape: ModelShape):
    """[(name, rows, cols, offset)] in the sorted-name order."""
    L = lib()
    cfg = shape.orc()
    out, off = [], 0
    buf = C.create_string_buffer(96)
    for i in range(L.orc_param_count(C.byref(cfg))):
        r, c = C.c_int64(), C.c_int64()
        n = L.orc_param_info(C.byref(cfg), i, buf, C.byref(r), C.byref(c))
        out.append((buf.value.decode(), r.value, c.value, off))
        off += n
    return out


def window_sizes(shape: ModelShape) -> np.ndarray:
    out = np.zeros(shape.n_layer, np.int32)
    lib().orc_window_sizes(C.byref(shape.orc()), out)
    return out


class OracleModel:
    """Dense transformer oracle (float32 by default, float64 when dtype=np.float64)."""

    def __init__(self, shape: ModelShape, params: np.ndarray, dtype=np.float32):
        self.shape = shape
        self.dtype = np.dtype(dtype)
        self.sfx = "_f64" if self.dtype == np.float64 else "_f32"
        self._cfg = shape.orc()
        self.params = np.ascontiguousarray(params, dtype=self.dtype)
        self.total = lib().orc_param_total(C.byref(self._cfg))
        assert self.params.size == self.total, (self.params.size, self.total)
        self._m = getattr(lib(), "orc_model_new" + self.sfx)(C.byref(self._cfg), self.params)

    def __del__(self):
        if getattr(self, "_m", None):
            getattr(lib(), "orc_model_free" + self.sfx)(self._m)
            self._m = None

    def _fn(self, name):
        return getattr(lib(), name + self.sfx)

    def forward(self, ids: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        B, T = ids.shape
        out = np.zeros((B, T, self.shape.vocab_size), self.dtype)
        self._fn("orc_forward")(self._m, ids, B, T, out)
        return out

    def forward_decode(self, ids: np.ndarray, chunk: int = 1) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        B, T = ids.shape
        out = np.zeros((B, T, self.shape.vocab_size), self.dtype)
        self._fn("orc_forward_decode")(self._m, ids, B, T, chunk, out)
        return out

    def pg_step(self, inputs, targets, adv, norm):
        inputs = np.ascontiguousarray(inputs, np.int32)
        targets = np.ascontiguousarray(targets, np.int32)
        adv = np.ascontiguousarray(adv, np.float32)
        B, T = inputs.shape
        nll = np.zeros(B * T, self.dtype)
        grads = np.zeros(self.total, self.dtype)
        loss = self._fn("orc_pg_step")(self._m, inputs, targets, B, T, adv, float(norm), nll, grads)
        return loss, nll.reshape(B, T), grads

    def distill_step(self, teacher_logits, inputs, mask=None, temperature=1.0, accum=1):
        """trainer.DistillStep given the teacher's logits [B, T, V]."""
        inputs = np.ascontiguousarray(inputs, np.int32)
        B, T = inputs.shape
        tl = np.ascontiguousarray(teacher_logits, np.float32)
        mk = None if mask is None else np.ascontiguousarray(mask, np.int32)
        grads = np.zeros(self.total, self.dtype)
        loss = self._fn("orc_distill_step")(self._m, tl, inputs,
                                            None if mk is None else mk.ctypes.data, B, T,
                                            float(temperature), int(accum), grads)
        return loss, grads

    def aux_loss(self) -> float:
        """MoE balance loss of the last training forward (pg_step / ce_loss)."""
        return self._fn("orc_aux_loss")(self._m)

    def prefill_ced(self, prompt: np.ndarray) -> np.ndarray:
        """Model.PrefillCED of one prompt: the last replayed row's logits."""
        prompt = np.ascontiguousarray(prompt, np.int32).reshape(-1)
        out = np.zeros(self.shape.vocab_size, self.dtype)
        self._fn("orc_prefill_ced")(self._m, prompt, prompt.size, out)
        return out

    def set_params(self, params: np.ndarray):
        self.params = np.ascontiguousarray(params, self.dtype)
        assert self.params.size == self.total
        self._fn("orc_model_set_params")(self._m, self.params)

    def freeze_targets(self, mode: int):
        """Indexer distillation targets: 0 computed, 1 computed and recorded,
        2 the recorded ones (finite-difference checks)."""
        self._fn("orc_set_freeze_targets")(self._m, mode)

    def distill_loss(self) -> float:
        """weight * sum over rows of -target . log softmax(I) of the last
        forward (the objective whose gradient the backward takes, targets
        held constant)."""
        return self._fn("orc_distill_loss")(self._m)

    def ce_loss(self, inputs, targets, want_grads=True):
        inputs = np.ascontiguousarray(inputs, np.int32)
        targets = np.ascontiguousarray(targets, np.int32)
        B, T = inputs.shape
        grads = np.zeros(self.total, self.dtype) if want_grads else None
        loss = self._fn("orc_ce_loss")(self._m, inputs, targets, B, T, _ptr(grads))
        return loss, grads

    def generate_batch(self, prompt, samples, max_tokens, temperature, top_k, seed):
        prompt = np.ascontiguousarray(prompt, np.int32)
        P = prompt.size
        rows = np.zeros((samples, P + max_tokens), np.int32)
        lens = np.zeros(samples, np.int32)
        self._fn("orc_generate_batch")(self._m, prompt, P, samples, max_tokens,
                                       float(temperature), top_k, seed, rows, lens)
        return [rows[s, :lens[s]].copy() for s in range(samples)]

    def decode_forced(self, prompt, cols):
        """The logits Engine.GenerateWith samples from for one group when the
        fed columns cols [ncols, S] are given: [ncols + 1, S, V] (the
        prefill's last logits, then those after each fed column)."""
        prompt = np.ascontiguousarray(prompt, np.int32).reshape(-1)
        cols = np.ascontiguousarray(cols, np.int32)
        ncols, S = cols.shape
        out = np.zeros((ncols + 1, S, self.shape.vocab_size), self.dtype)
        self._fn("orc_decode_forced")(self._m, prompt, prompt.size, S, cols, ncols, out)
        return out

    def rl_step(self, prompts, samples, max_tokens, temperature, top_k, seeds, rewards):
        prompts = np.ascontiguousarray(prompts, np.int32)
        G, P = prompts.shape
        Bt = G * samples
        W = P + max_tokens
        rows = np.zeros((Bt, W), np.int32)
        lens = np.zeros(Bt, np.int32)
        adv = np.zeros(Bt, np.float32)
        max_len = C.c_int32()
        inputs = np.zeros(Bt * W, np.int32)
        targets = np.zeros(Bt * W, np.int32)
        nll = np.zeros(Bt * W, self.dtype)
        grads = np.zeros(self.total, self.dtype)
        loss = self._fn("orc_rl_step")(
            self._m, prompts, G, P, samples, max_tokens, float(temperature), top_k,
            np.ascontiguousarray(seeds, np.uint64), np.ascontiguousarray(rewards, np.float32),
            rows, lens, adv, C.byref(max_len), inputs, targets, nll, grads)
        T = max_len.value - 1
        return dict(loss=loss, rows=[rows[b, :lens[b]].copy() for b in range(Bt)], lens=lens,
                    adv=adv, max_len=max_len.value, inputs=inputs[:Bt * T].reshape(Bt, T),
                    targets=targets[:Bt * T].reshape(Bt, T), nll=nll[:Bt * T].reshape(Bt, T),
                    grads=grads)


class GoRNG:
    """tensors.RNG: Go's math/rand/v2 PCG seeded as NewPCG(s, s^0x9e37...)."""

    def __init__(self, seed: int):
        self.state = OrcPCG()
        lib().orc_rng_new(C.byref(self.state), C.c_uint64(seed))

    def uint64(self) -> int:
        return lib().orc_rng_uint64(C.byref(self.state))

    def float32(self) -> float:
        return lib().orc_rng_float32(C.byref(self.state))

    def advance(self, n: int) -> None:
        lib().orc_rng_advance(C.byref(self.state), C.c_uint64(n >> 64),
                              C.c_uint64(n & ((1 << 64) - 1)))

    @property
    def hi_lo(self):
        return self.state.hi, self.state.lo


def sample_next_token(logits: np.ndarray, rng: GoRNG, temperature: float, top_k: int):
    logits = np.ascontiguousarray(logits, np.float32)
    rows, vocab = logits.shape
    out = np.zeros(rows, np.int32)
    lib().orc_sample_next_token(logits, rows, vocab, C.byref(rng.state), float(temperature),
                                top_k, out)
    return out


def rotary_table(positions: int, rotary_dim: int):
    """precomputeRotary (model/rotary.go:16-30): cos, sin [positions, R/2]."""
    c = np.zeros((positions, rotary_dim // 2), np.float32)
    s = np.zeros_like(c)
    lib().orc_rotary_table_f32(positions, rotary_dim, c, s)
    return c, s


def apply_rotary(x: np.ndarray, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    """ApplyRotary (model/rotary.go:43-75) of one token's heads x [heads, D]
    with one table row (R/2 entries each): the model's own rotation."""
    x = np.ascontiguousarray(x, np.float32)
    heads, D = x.shape
    out = np.zeros_like(x)
    c = np.ascontiguousarray(cos_row, np.float32)
    s = np.ascontiguousarray(sin_row, np.float32)
    lib().orc_apply_rotary_f32(out, x, heads, D, 2 * c.size, c, s)
    return out


def calculator(expr: str):
    out = C.create_string_buffer(512)
    ok = lib().orc_calculator(expr.encode(), out, 512)
    return out.value.decode() if ok else None


class OracleOptimizer:
    """MuonAdamW.Step restated in C (oracle/optimizer.c) over a gn_opt_param
    table (gonano_amd.optimizer.OPT_PARAM_DTYPE layout); test infrastructure."""

    def __init__(self, table: np.ndarray):
        self.table = np.ascontiguousarray(table)
        n = len(self.table)
        self.state = np.zeros(lib().orc_opt_state_floats(self.table.ctypes.data, n), np.float32)
        self.steps = np.zeros(n, np.int32)

    def step(self, params: np.ndarray, grads: np.ndarray) -> None:
        """One step in place on the flat parameter vector."""
        assert params.dtype == np.float32 and grads.dtype == np.float32
        lib().orc_opt_step(params, np.ascontiguousarray(grads), self.table.ctypes.data,
                           len(self.table), self.state, self.steps)


def polar_express(u: np.ndarray, steps: int = 5) -> np.ndarray:
    """The Muon orthogonalization of a float32 matrix (optimizer/muon.go:50-74)."""
    x = np.ascontiguousarray(u, np.float32).copy()
    lib().orc_polar_express(x, x.shape[0], x.shape[1], steps)
    return x

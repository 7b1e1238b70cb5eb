"""Loads libgnhip.so (the HIP backend's C ABI, include/gonano_hip.h) with
ctypes.  There is no fallback: if the library is missing the import fails."""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgnhip.so")

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
i64 = C.c_int64
vp = C.c_void_p


class GnConfig(C.Structure):
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


class GnTiming(C.Structure):
    _fields_ = [
        ("rollout_ms", C.c_double),
        ("decode_attn_ms", C.c_double),
        ("decode_attn_launches", C.c_int64),
        ("decode_attn_bytes", C.c_double),
        ("train_ms", C.c_double),
        ("gemm_ms", C.c_double),
        ("gemm_flops", C.c_double),
        ("gemm_launches", C.c_int64),
        ("gemm_wide_ms", C.c_double),
        ("gemm_wide_flops", C.c_double),
        ("gemm_wide_launches", C.c_int64),
        ("loss_ms", C.c_double),
        ("loss_bytes", C.c_double),
        ("loss_launches", C.c_int64),
    ]


# int32_t (*)(void *user, const int32_t *call, int32_t n, int32_t *out, int32_t cap)
GnToolFn = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.POINTER(C.c_int32), C.c_int32,
                       C.POINTER(C.c_int32), C.c_int32)


class GnGenerateOptions(C.Structure):
    _fields_ = [
        ("thinking", C.c_int32),
        ("thinking_budget", C.c_int32),
        ("bos", C.c_int32),
        ("assistant_end", C.c_int32),
        ("tool_start", C.c_int32),
        ("tool_end", C.c_int32),
        ("tool_output_start", C.c_int32),
        ("tool_output_end", C.c_int32),
        ("think_start", C.c_int32),
        ("think_end", C.c_int32),
        ("tool", GnToolFn),
        ("tool_user", C.c_void_p),
    ]


class GnPrefixCacheOptions(C.Structure):
    _fields_ = [
        ("max_entries", C.c_int32),
        ("max_prefix", C.c_int32),
        ("max_bytes", C.c_int64),
        ("ttl_seconds", C.c_double),
        ("disk_dir", C.c_char_p),
    ]


class HipError(RuntimeError):
    """A gn_* call returned a non-zero gn_status (the reference panics)."""

    def __init__(self, fn: str, code: int, msg: str):
        super().__init__(f"{fn}: status {code}: {msg}")
        self.code = code


_SIGS = {
    "gn_last_error": (C.c_char_p, []),
    "gn_device_count": (C.c_int, []),
    "gn_set_device": (C.c_int, [C.c_int]),
    "gn_synchronize": (C.c_int, []),
    "gn_add": (C.c_int, [f32p, f32p, f32p, i64]),
    "gn_subtract": (C.c_int, [f32p, f32p, f32p, i64]),
    "gn_multiply": (C.c_int, [f32p, f32p, f32p, i64]),
    "gn_divide": (C.c_int, [f32p, f32p, f32p, i64]),
    "gn_scale": (C.c_int, [f32p, f32p, C.c_float, i64]),
    "gn_add_scaled": (C.c_int, [f32p, f32p, f32p, C.c_float, i64]),
    "gn_negate": (C.c_int, [f32p, f32p, i64]),
    "gn_abs": (C.c_int, [f32p, f32p, i64]),
    "gn_square": (C.c_int, [f32p, f32p, i64]),
    "gn_relu_squared": (C.c_int, [f32p, f32p, i64]),
    "gn_swiglu": (C.c_int, [f32p, f32p, f32p, C.c_float, i64]),
    "gn_swiglu_backward": (C.c_int, [f32p, f32p, f32p, f32p, f32p, C.c_float, i64]),
    "gn_exp": (C.c_int, [f32p, f32p, i64]),
    "gn_sigmoid": (C.c_int, [f32p, f32p, i64]),
    "gn_tanh": (C.c_int, [f32p, f32p, i64]),
    "gn_rsqrt": (C.c_int, [f32p, f32p, i64]),
    "gn_sum": (C.c_int, [f32p, i64, C.POINTER(C.c_float)]),
    "gn_max": (C.c_int, [f32p, i64, C.POINTER(C.c_float)]),
    "gn_argmax": (C.c_int, [f32p, i64, C.POINTER(C.c_int64)]),
    "gn_matmul": (C.c_int, [f32p, f32p, f32p, i64, i64, i64]),
    "gn_matmul_transposed": (C.c_int, [f32p, f32p, f32p, i64, i64, i64]),
    "gn_dot_product": (C.c_int, [f32p, i64, f32p, i64, C.POINTER(C.c_float)]),
    "gn_indexer_scores": (C.c_int, [f32p, f32p, f32p, f32p, i64, i64, i64, i64]),
    "gn_indexer_block_max": (C.c_int, [f32p, f32p, i64, i64, i64]),
    "gn_topk_indices": (C.c_int, [i32p, f32p, i64, i64, i64]),
    "gn_moe_gate_topk": (C.c_int, [f32p, f32p, f32p, i32p, f32p, i64, i64, i64]),
    "gn_grouped_matmul_transposed": (C.c_int, [f32p, f32p, f32p, i32p, i64, i64, i64]),
    "gn_softmax_last_dim": (C.c_int, [f32p, f32p, i64, i64]),
    "gn_rmsnorm_last_dim": (C.c_int, [f32p, f32p, i64, i64, C.c_float]),
    "gn_attention_forward": (C.c_int, [f32p, f32p, f32p, vp, i64, i64, i64, i64, i64, i64, f32p, vp]),
    "gn_attention_backward": (C.c_int, [f32p, f32p, f32p, f32p, f32p, f32p, vp, vp, i64, i64, i64,
                                        i64, i64, i64, f32p, f32p, f32p]),
    "gn_attention_forward_split": (C.c_int, [f32p, f32p, f32p, vp, i64, i64, i64, i64, i64, i64,
                                             i64, i64, f32p, f32p, f32p]),
    "gn_attention_combine": (C.c_int, [C.POINTER(vp), C.POINTER(vp), C.POINTER(vp), i64, i64, i64,
                                       f32p, vp]),
    "gn_session_create": (C.c_int, [C.POINTER(GnConfig), C.c_int, C.POINTER(vp)]),
    "gn_session_destroy": (C.c_int, [vp]),
    "gn_session_param_total": (C.c_int, [vp, C.POINTER(C.c_int64)]),
    "gn_session_param_count": (C.c_int, [vp, C.POINTER(C.c_int32)]),
    "gn_session_param_info": (C.c_int, [vp, C.c_int32, C.c_char_p, C.c_size_t, C.POINTER(C.c_int64),
                                        C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
    "gn_session_set_params": (C.c_int, [vp, f32p, i64]),
    "gn_session_get_params": (C.c_int, [vp, f32p, i64]),
    "gn_session_get_grads": (C.c_int, [vp, f32p, i64]),
    "gn_session_zero_grads": (C.c_int, [vp]),
    "gn_forward": (C.c_int, [vp, i32p, C.c_int32, C.c_int32, f32p]),
    "gn_generate_batch": (C.c_int, [vp, i32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                    C.c_int32, u64p, i32p, i32p]),
    "gn_policy_gradient_step": (C.c_int, [vp, i32p, i32p, C.c_int32, C.c_int32, f32p, C.c_float,
                                          C.POINTER(C.c_float), vp]),
    "gn_rl_step": (C.c_int, [vp, i32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                             C.c_int32, u64p, f32p, i32p, i32p, f32p, C.POINTER(C.c_int32),
                             C.POINTER(C.c_float)]),
    "gn_generate_options_default": (C.c_int, [C.POINTER(GnGenerateOptions)]),
    "gn_generate_batch_with": (C.c_int, [vp, i32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                         C.c_float, C.c_int32, u64p, C.POINTER(GnGenerateOptions),
                                         i32p, i32p, vp]),
    "gn_rl_step_with": (C.c_int, [vp, i32p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_float,
                                  C.c_int32, u64p, C.POINTER(GnGenerateOptions), f32p, i32p, i32p,
                                  f32p, C.POINTER(C.c_int32), C.POINTER(C.c_float)]),
    "gn_use_calculator": (C.c_int, [C.c_char_p, C.c_char_p, C.c_size_t, C.POINTER(C.c_int32)]),
    "gn_sample_next_token": (C.c_int, [f32p, i64, i64, u64p, C.c_float, i64, i32p]),
    "gn_sample_next_token_static": (C.c_int, [f32p, i64, i64, u64p, C.c_float, i64, i32p]),
    "gn_softcap_order_check": (C.c_int, [u64p]),
    "gn_session_set_timing": (C.c_int, [vp, C.c_int]),
    "gn_session_get_timing": (C.c_int, [vp, C.POINTER(GnTiming)]),
    "gn_session_synchronize": (C.c_int, [vp]),
    "gn_session_aux_loss": (C.c_int, [vp, C.POINTER(C.c_double)]),
    "gn_session_set_decode_graph": (C.c_int, [vp, C.c_int]),
    "gn_session_set_prefix_cache": (C.c_int, [vp, C.POINTER(GnPrefixCacheOptions)]),
    "gn_session_prefix_cache_invalidate": (C.c_int, [vp]),
    "gn_session_prefix_cache_len": (C.c_int, [vp, C.POINTER(C.c_int32), C.POINTER(C.c_int64)]),
    "gn_session_prefix_cache_hits": (C.c_int, [vp, i32p, C.c_int32]),
    "gn_distill_step": (C.c_int, [vp, vp, i32p, vp, C.c_int32, C.c_int32, C.c_float, C.c_int32,
                                  C.POINTER(C.c_float)]),
    "gn_optimizer_create": (C.c_int, [vp, vp, C.c_int32, C.POINTER(C.c_void_p)]),
    "gn_optimizer_step": (C.c_int, [vp]),
    "gn_optimizer_state_size": (C.c_int, [vp, C.POINTER(C.c_int64)]),
    "gn_optimizer_get_state": (C.c_int, [vp, f32p, i64]),
    "gn_optimizer_set_hyper": (C.c_int, [vp, vp, vp, vp, C.c_int32]),
    "gn_session_update_router_bias": (C.c_int, [vp, C.c_float]),
    "gn_session_moe_loads": (C.c_int, [vp, C.POINTER(C.c_double), i64]),
    "gn_optimizer_destroy": (C.c_int, [vp]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: run `python -m gonano_amd.build` "
                              "(or __graft_entry__.build()) first")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(fn: str, status: int) -> None:
    if status != 0:
        raise HipError(fn, status, lib().gn_last_error().decode(errors="replace"))


def call(fn: str, *args) -> None:
    check(fn, getattr(lib(), fn)(*args))


def exported_symbols() -> list[str]:
    return list(_SIGS)

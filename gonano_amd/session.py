"""Device-resident RL-step session over the HIP C ABI.

Mirrors the reference entry points this path replaces:
Transformer.Forward (model/transformer.go:211-214),
Engine.GenerateBatchWith (inference/engine.go:336-369),
trainer.PolicyGradientStep (trainer/rl.go:14-60), and the body of
cmd/chat_rl's step loop (cmd/chat_rl/main.go:101-183).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from ._lib import GnConfig, GnGenerateOptions, GnPrefixCacheOptions, GnTiming, GnToolFn, call, lib
from .config import Config


class GenerateOptions:
    """inference.GenerateOptions (inference/engine.go:25-34) plus the ids the
    host's tokenizer gives the engine (Tokenizer.EncodeSpecial / BOSTokenID)
    and its tool registry: tool(call_ids) -> result ids, or None when no
    tool understands the call (Registry.Execute over Tokenizer.Decode /
    Encode).  Defaults: the byte-level tokenizer, thinking off, the built-in
    calculator."""

    def __init__(self, thinking: bool = False, thinking_budget: int = 0, tool=None, **ids):
        o = GnGenerateOptions()
        call("gn_generate_options_default", C.byref(o))
        o.thinking = 1 if thinking else 0
        o.thinking_budget = int(thinking_budget)
        for k, v in ids.items():
            if k not in ("bos", "assistant_end", "tool_start", "tool_end", "tool_output_start",
                         "tool_output_end", "think_start", "think_end"):
                raise TypeError(f"unknown special id {k}")
            setattr(o, k, int(v))
        self._tool = tool
        self._cb = None
        if tool is not None:
            def cb(user, ids_p, n, out_p, cap):
                res = tool([ids_p[i] for i in range(n)])
                if res is None:
                    return -1
                res = list(res)
                if len(res) > cap:
                    return cap + 1
                for i, v in enumerate(res):
                    out_p[i] = int(v)
                return len(res)
            self._cb = GnToolFn(cb)
            o.tool = self._cb
        self.c = o

    def __getattr__(self, name):
        return getattr(self.__dict__["c"], name)


def use_calculator(expression: str):
    """inference.UseCalculator (inference/tooluse.go:83-90) through the C ABI:
    the result string, or None when the calculator rejects the expression."""
    out = C.create_string_buffer(512)
    ok = C.c_int32()
    call("gn_use_calculator", expression.encode(), out, 512, C.byref(ok))
    return out.value.decode() if ok.value else None


def gn_config_of(cfg: Config) -> GnConfig:
    """The C-ABI gn_config of a host Config (resolved preset values)."""
    return GnConfig(cfg.sequence_len, cfg.vocab_size, cfg.n_layer, cfg.n_head,
                    cfg.n_kv_head, cfg.n_embd, cfg.rotary_dims, cfg.window_pattern.encode(),
                    cfg.mla_latent, cfg.mla_rope_dimension if cfg.mla else 0,
                    cfg.n_experts, cfg.experts_per_token, cfg.expert_hidden,
                    cfg.shared_hidden, cfg.moe_clamp, cfg.moe_scale, cfg.balance_weight,
                    cfg.compression_ratio if cfg.compression > 1 else 0,
                    cfg.swa_window if cfg.compression > 1 else 0,
                    cfg.sparse_topk, cfg.indexer_dim, cfg.indexer_heads, cfg.indexer_pool,
                    cfg.indexer_candidates, cfg.indexer_weight, cfg.reuse_pattern.encode(),
                    int(cfg.ced))


class Session:
    def __init__(self, cfg: Config, device: int = 0):
        cfg.validate()
        self.cfg = cfg
        self._c = gn_config_of(cfg)
        h = C.c_void_p()
        call("gn_session_create", C.byref(self._c), device, C.byref(h))
        self._h = h
        t = C.c_int64()
        call("gn_session_param_total", self._h, C.byref(t))
        self.param_total = t.value

    def close(self):
        if getattr(self, "_h", None):
            lib().gn_session_destroy(self._h)
            self._h = None

    __del__ = close

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- parameters -----------------------------------------------------------
    def param_table(self):
        n = C.c_int32()
        call("gn_session_param_count", self._h, C.byref(n))
        out = []
        buf = C.create_string_buffer(128)
        r, c, o = C.c_int64(), C.c_int64(), C.c_int64()
        for i in range(n.value):
            call("gn_session_param_info", self._h, i, buf, 128, C.byref(r), C.byref(c), C.byref(o))
            out.append((buf.value.decode(), r.value, c.value, o.value))
        return out

    def set_params(self, params: np.ndarray):
        params = np.ascontiguousarray(params, np.float32)
        call("gn_session_set_params", self._h, params, params.size)

    def get_params(self) -> np.ndarray:
        out = np.zeros(self.param_total, np.float32)
        call("gn_session_get_params", self._h, out, out.size)
        return out

    def grads(self) -> np.ndarray:
        out = np.zeros(self.param_total, np.float32)
        call("gn_session_get_grads", self._h, out, out.size)
        return out

    def zero_grad(self):
        call("gn_session_zero_grads", self._h)

    def update_router_bias(self, speed: float | None = None):
        """Transformer.UpdateRouterBias (model/transformer.go:121-131) with
        speed = Config.MoERouterBiasUpdate() unless given."""
        if speed is None:
            speed = self.cfg.router_bias_update if self.cfg.router_bias_update > 0 else 0.001
        call("gn_session_update_router_bias", self._h, float(speed))

    def moe_loads(self) -> np.ndarray:
        """MoE.loadCounts of every layer, [n_layer, n_experts] (float64)."""
        E = self.cfg.n_experts
        out = np.zeros((self.cfg.n_layer if E > 0 else 0, E), np.float64)
        call("gn_session_moe_loads", self._h, out.ctypes.data_as(C.POINTER(C.c_double)), out.size)
        return out

    # -- compute --------------------------------------------------------------
    def forward(self, ids: np.ndarray) -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int32)
        B, T = ids.shape
        out = np.zeros((B, T, self.cfg.vocab_size), np.float32)
        call("gn_forward", self._h, ids, B, T, out)
        return out

    def generate_batch(self, prompts: np.ndarray, samples: int, max_tokens: int,
                       temperature: float, top_k: int, seeds, options: GenerateOptions = None,
                       masks: bool = False):
        """Engine.GenerateBatchWith for every group (one prompt row each):
        the rows (prompt + completion, terminal token excluded) and, with
        masks=True, GenerateBatchWith's masks (1 sampled, 0 prompt/forced)."""
        prompts = np.ascontiguousarray(np.atleast_2d(prompts), np.int32)
        G, P = prompts.shape
        rows = np.zeros((G * samples, P + max_tokens), np.int32)
        lens = np.zeros(G * samples, np.int32)
        mk = np.zeros((G * samples, P + max_tokens), np.int32) if masks else None
        if options is None and not masks:
            call("gn_generate_batch", self._h, prompts, G, P, samples, max_tokens,
                 float(temperature), top_k, np.ascontiguousarray(seeds, np.uint64), rows, lens)
        else:
            call("gn_generate_batch_with", self._h, prompts, G, P, samples, max_tokens,
                 float(temperature), top_k, np.ascontiguousarray(seeds, np.uint64),
                 None if options is None else C.byref(options.c), rows, lens,
                 None if mk is None else mk.ctypes.data_as(C.c_void_p))
        out = [rows[i, :lens[i]].copy() for i in range(G * samples)]
        if masks:
            return out, [mk[i, :lens[i]].copy() for i in range(G * samples)]
        return out

    def policy_gradient_step(self, inputs, targets, advantages, norm: float):
        inputs = np.ascontiguousarray(inputs, np.int32)
        targets = np.ascontiguousarray(targets, np.int32)
        adv = np.ascontiguousarray(advantages, np.float32)
        B, T = inputs.shape
        nll = np.zeros(B * T, np.float32)
        loss = C.c_float()
        call("gn_policy_gradient_step", self._h, inputs, targets, B, T, adv, float(norm),
             C.byref(loss), nll.ctypes.data_as(C.c_void_p))
        return loss.value, nll.reshape(B, T)

    def distill_step(self, teacher: "Session", inputs, mask=None, temperature: float = 1.0,
                     grad_accum_steps: int = 1) -> float:
        """trainer.DistillStep (trainer/distill.go:13-46): the teacher session
        scores inputs, this session's gradients accumulate the forward-KL
        distillation loss; returns the mean per-position loss."""
        inputs = np.ascontiguousarray(inputs, np.int32)
        B, T = inputs.shape
        mk = None if mask is None else np.ascontiguousarray(mask, np.int32)
        loss = C.c_float()
        call("gn_distill_step", self._h, teacher._h, inputs,
             None if mk is None else mk.ctypes.data_as(C.c_void_p), B, T, float(temperature),
             int(grad_accum_steps), C.byref(loss))
        return loss.value

    def rl_step(self, prompts, samples, max_tokens, temperature, top_k, seeds, rewards,
                options: GenerateOptions = None):
        prompts = np.ascontiguousarray(prompts, np.int32)
        G, P = prompts.shape
        Bt = G * samples
        rows = np.zeros((Bt, P + max_tokens), np.int32)
        lens = np.zeros(Bt, np.int32)
        adv = np.zeros(Bt, np.float32)
        max_len = C.c_int32()
        loss = C.c_float()
        seeds = np.ascontiguousarray(seeds, np.uint64)
        rewards = np.ascontiguousarray(rewards, np.float32)
        if options is None:
            call("gn_rl_step", self._h, prompts, G, P, samples, max_tokens, float(temperature),
                 top_k, seeds, rewards, rows, lens, adv, C.byref(max_len), C.byref(loss))
        else:
            call("gn_rl_step_with", self._h, prompts, G, P, samples, max_tokens,
                 float(temperature), top_k, seeds, C.byref(options.c), rewards, rows, lens, adv,
                 C.byref(max_len), C.byref(loss))
        return dict(loss=loss.value, rows=[rows[b, :lens[b]].copy() for b in range(Bt)],
                    lens=lens, adv=adv, max_len=max_len.value)

    # -- timing ---------------------------------------------------------------
    def set_timing(self, enabled: bool):
        call("gn_session_set_timing", self._h, 1 if enabled else 0)

    def aux_loss(self) -> float:
        """Transformer.AuxiliaryLoss: the MoE balance loss of the last
        policy-gradient step (model/transformer.go:108-116)."""
        v = C.c_double()
        call("gn_session_aux_loss", self._h, C.byref(v))
        return v.value

    def synchronize(self):
        """Waits until the session stream is idle."""
        call("gn_session_synchronize", self._h)

    def set_decode_graph(self, enabled: bool):
        """Replay rollout decode steps from one captured HIP graph (default)
        or launch every kernel of every step."""
        call("gn_session_set_decode_graph", self._h, 1 if enabled else 0)

    def set_prefix_cache(self, max_entries: int = 0, max_bytes: int = 0, ttl: float = 0.0,
                         max_prefix: int = 0, enabled: bool = True, disk_dir: str = ""):
        """Engine.Cache = NewCacheManager(CacheOptions{MaxEntries, MaxBytes,
        TTL, DiskDir}) on the device (inference/cache.go:17-77); max_entries=1
        with max_prefix is Engine.Prefix = NewPrefixCache(maxPrefix)
        (inference/prefix.go:29-35).  disk_dir: the on-disk tier (entries
        written there, read back for the call that hits them).  enabled=False
        turns it off and drops every entry.  Generate and RL-step calls then
        prefill only what follows each prompt's longest cached strict
        prefix."""
        if not enabled:
            call("gn_session_set_prefix_cache", self._h, None)
            return
        o = GnPrefixCacheOptions(max_entries, max_prefix, max_bytes, ttl,
                                 os.fsencode(disk_dir) if disk_dir else None)
        call("gn_session_set_prefix_cache", self._h, C.byref(o))

    def prefix_cache_invalidate(self):
        """CacheManager.Invalidate (inference/cache.go:162-174)."""
        call("gn_session_prefix_cache_invalidate", self._h)

    def prefix_cache_len(self) -> tuple[int, int]:
        """CacheManager.Len (inference/cache.go:176-180) and the entries'
        device bytes."""
        n, b = C.c_int32(), C.c_int64()
        call("gn_session_prefix_cache_len", self._h, C.byref(n), C.byref(b))
        return n.value, b.value

    def prefix_cache_hits(self, groups: int) -> np.ndarray:
        """Per group of the last generate call, the prompt tokens its cache
        lookup matched (0: a miss)."""
        out = np.zeros(groups, np.int32)
        call("gn_session_prefix_cache_hits", self._h, out, groups)
        return out

    def timing(self) -> dict:
        t = GnTiming()
        call("gn_session_get_timing", self._h, C.byref(t))
        return {f: getattr(t, f) for f, _ in GnTiming._fields_}

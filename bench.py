"""RL-step benchmark on one MI355X (the benchmark's metric: rollout tokens/sec
and RL-step ms at the d12 dense config, plus the achieved fraction of the
fp32-MFMA and HBM peaks).

A step is one cmd/chat_rl step without the optimizer: 16 prompts x 16
rollouts x 256 new tokens, the teacher-forced log-prob recompute over the
padded [256, 511] batch, group-mean advantages of Bernoulli(0.3) rewards and
the PG loss forward/backward over the full 65536 vocabulary.  Inputs are
synthetic (uniform prompt ids, InitWeights-distributed random weights) and
resident in HBM before the timed region.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config d12|d2|d20|latent_d12|flash_d12]
                    [--phase rl|train|rollout|optimizer|prefix] [--no-graph]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP32_MFMA_PEAK_TFLOPS = 157.3
METRIC = "rollout tokens/sec + RL-step ms at d12 on 1 MI355X; % of HBM/fp32-MFMA peak"

WORKLOADS = {
    # name: (config factory, groups, prompt len, samples, new tokens, temperature, reward p)
    "d12": ("dense_d12", 16, 256, 16, 256, 1.0, 0.3),
    "d2": ("dense_d2", 4, 32, 8, 24, 1.0, 0.3),
    # the benchmark's d20 workload: 32 prompts of 512 tokens x 16 samples, 1024 new tokens, T=0.8,
    # rewards uniform on {0, 1} (Bernoulli(0.5))
    "d20": ("dense_d20", 32, 512, 16, 1024, 0.8, 0.5),
    # the benchmark's latent d12 workload (the group split is unspecified there: 16 x 16 as d12)
    "latent_d12": ("latent_d12", 16, 256, 16, 256, 1.0, 0.3),
    # the benchmark's flash d12 workload: 64 rollouts (4 groups x 16) of 8192-token prompts + 512 new tokens
    "flash_d12": ("flash_d12", 4, 8192, 16, 512, 1.0, 0.3),
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_baseline(cfg, w, prompts, S: int, N: int, temp: float) -> dict:
    """The oracle (a scalar C port of the reference's arithmetic, float64
    accumulation, OpenMP over rows) generating rollouts on the same weights.

    Bounded sample: ONE prompt group of the workload (all S samples), timed
    once with 1 new token (prefill) and once with 1 + STEPS new tokens; the
    difference gives the cost of one batched decode step.  The reported rate
    is the workload's per-group token count over the time one group would
    take, prefill + N decode steps, so it is in the same unit and the same
    prefill/decode mix as the GPU's value.

    Prompts longer than PREFIX (the flash workload's 8192 tokens, ~100 s of
    oracle prefill) are sampled on their first PREFIX tokens and the
    prefill time is scaled by layer-tokens: every layer reads every prompt
    token, except a CED decoder layer, which replays only the last
    min(window, P) tokens (PrefillCED, model/transformer.go:363-449).  The
    per-token cost is taken as constant (the indexer's quadratic score term
    is ~8 % of a layer-token at P = 8192), so the scaled prefill is a slight
    underestimate and the CPU rate a slight overestimate."""
    from oracle import oracle as O
    P = prompts.shape[1]
    PREFIX = 1024
    Ps = min(P, PREFIX)
    # about 15 s of CPU work on 16 host threads: 128 decode steps of a d12
    # group, fewer for larger models and for long sampled prompts
    STEPS = 8 if Ps < P else max(8, min(128, int(128 * 1.3e8 / cfg.param_total())))
    m = O.OracleModel(O.ModelShape.from_config(cfg), w)

    def layer_tokens(p):
        split = cfg.ced_split
        if split <= 0:
            return cfg.n_layer * p
        return split * p + (cfg.n_layer - split) * min(cfg.swa_window or p, p)

    prompt = prompts[0, :Ps]
    t0 = time.perf_counter()
    m.generate_batch(prompt, S, 1, temp, 50, 0)
    t_prefill = time.perf_counter() - t0
    t0 = time.perf_counter()
    rows = m.generate_batch(prompt, S, 1 + STEPS, temp, 50, 0)
    t_long = time.perf_counter() - t0
    steps = max(1, max(len(r) for r in rows) - Ps - 1)
    t_step = max(t_long - t_prefill, 1e-9) / steps
    scale = layer_tokens(P) / layer_tokens(Ps)
    group_s = t_prefill * scale + N * t_step
    sample = (f"oracle rollout of 1 prompt group ({Ps} prompt tokens x {S} samples) on the "
              f"same weights: prefill {t_prefill:.2f} s, {steps} batched decode steps "
              f"{t_long - t_prefill:.2f} s")
    if Ps < P:
        sample += (f"; prefill scaled to the {P}-token prompt by layer-tokens "
                   f"(x{scale:.3f} = {t_prefill * scale:.1f} s)")
    return {"value": round(S * N / group_s, 2), "unit": "tokens/s",
            "cores": int(O.lib().orc_num_threads()), "kind": "port",
            "sample": sample + f"; value = {S}x{N} tokens / (prefill + {N} steps) = one "
                               f"group of the workload"}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--config", default="d12", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--phase", default="rl",
                    choices=["rl", "train", "rollout", "optimizer", "prefix"],
                    help="rl: the full RL step (the benchmark); train: only the recompute + "
                         "PG fwd/bwd on a synthetic batch of the workload's shape (for "
                         "counter profiles of the train-phase kernels); rollout: only the "
                         "rollouts (for kernel-trace and counter profiles of the decode "
                         "kernels in place); optimizer: only MuonAdamW steps with "
                         "cmd/chat_rl's parameter groups; prefix: the prompts' prefill "
                         "with and without the device prefix cache")
    ap.add_argument("--no-graph", action="store_true",
                    help="launch every decode kernel instead of replaying the captured decode "
                         "graph (for kernel-trace profiles: rocprofv3 --kernel-trace has "
                         "crashed on the graph replays)")
    ap.add_argument("--no-optimizer", action="store_true",
                    help="skip the (untimed by the metric) optimizer-step timing, e.g. in "
                         "kernel-trace profiles of the RL step")
    ap.add_argument("--rw-rate", action="store_true",
                    help="run only the rates of a 1 GiB device copy and of an in-place "
                         "rewrite of a [4096, 65536] tensor (the logits' read + write pattern)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a device copy of 1 GiB (5 times), the known-size "
                         "reference for HBM byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build runs the RL step on a single MI355X "
              "(sharding the rollout rows and the train micro-batches over one process per "
              "GPU is a design, not a build target here); use --gpus 1.",
              file=sys.stderr)
        return 2

    if args.copy_calibration:
        return copy_calibration()
    if args.rw_rate:
        return rw_rate()

    from gonano_amd import config as G
    from gonano_amd.session import Session

    factory, groups, P, S, N, temp, reward_p = WORKLOADS[args.config]
    cfg = getattr(G, factory)()
    log(f"bench: config {args.config} {cfg}")
    w = G.init_weights(cfg, seed=0)
    prompts = np.random.default_rng(1).integers(0, cfg.vocab_size, (groups, P)).astype(np.int32)
    reward_rng = np.random.default_rng(2)

    sess = Session(cfg)
    sess.set_params(w)
    sess.set_timing(True)
    if args.no_graph:
        sess.set_decode_graph(False)

    if args.phase == "train":
        return train_phase(args, sess, prompts, S, N, reward_rng, reward_p)
    if args.phase == "rollout":
        return rollout_phase(args, sess, prompts, S, N, temp)
    if args.phase == "optimizer":
        return optimizer_phase(args, cfg, sess, prompts)
    if args.phase == "prefix":
        return prefix_phase(args, cfg, sess, prompts, temp)

    def step(i: int):
        seeds = np.array([i * 1000 + g for g in range(groups)], np.uint64)
        rewards = (reward_rng.random(groups * S) < reward_p).astype(np.float32)
        sess.zero_grad()
        t0 = time.perf_counter()
        out = sess.rl_step(prompts, S, N, temp, 50, seeds, rewards)
        wall = time.perf_counter() - t0
        return out, wall, sess.timing()

    for i in range(args.warmup):
        out, wall, t = step(i)
        log(f"bench: warmup {i}: {wall * 1e3:.1f} ms (rollout {t['rollout_ms']:.1f} ms, "
            f"train {t['train_ms']:.1f} ms), loss {out['loss']:.6f}")
    walls, roll_ms, train_ms, toks = [], [], [], 0
    gemm = {"ms": 0.0, "flops": 0.0, "n": 0, "wide_ms": 0.0, "wide_flops": 0.0, "wide_n": 0,
            "loss_ms": 0.0, "loss_bytes": 0.0, "loss_n": 0}
    sess.synchronize()
    t_start = time.perf_counter()
    for i in range(args.steps):
        out, wall, t = step(args.warmup + i)
        walls.append(wall)
        roll_ms.append(t["rollout_ms"])
        train_ms.append(t["train_ms"])
        toks += int(np.sum(out["lens"] - P))
        add_gemm(gemm, t)
        log(f"bench: step {i}: {wall * 1e3:.1f} ms (rollout {t['rollout_ms']:.1f} ms, "
            f"train {t['train_ms']:.1f} ms), loss {out['loss']:.6f}, max_len {out['max_len']}")
    sess.synchronize()
    ms_step = 1e3 * (time.perf_counter() - t_start) / args.steps
    # Decode attention is timed per call with events the dispatch records
    # (kernel start, last kernel's end), which the timed rollouts (decode
    # steps replayed from a captured graph) cannot carry: one more rollout of
    # the same workload, untimed, launches every kernel.
    sess.set_decode_graph(False)
    sess.generate_batch(prompts, S, N, temp, 50,
                        np.array([(args.warmup + args.steps) * 1000 + g for g in range(groups)],
                                 np.uint64))
    t = sess.timing()
    attn_ms, attn_b, attn_n = t["decode_attn_ms"], t["decode_attn_bytes"], t["decode_attn_launches"]
    # RLStep's optimizer.Step (trainer/rl.go:65), outside the metric: timed
    # on the last step's gradients
    opt = None if args.no_optimizer else optimizer_timing(cfg, sess, steps=2)
    sess.close()

    rollout_s = sum(roll_ms) / 1e3
    value = toks / rollout_s
    attn_gbs = attn_b / (attn_ms / 1e3) / 1e9 if attn_ms else 0.0
    res = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (uniform prompt ids, InitWeights-distributed random weights, "
                "Bernoulli rewards)",
        "config": {
            "workload": f"{args.config} RL step: {groups} prompts x {S} samples, "
                        f"{P} prompt + {N} new tokens, T={temp}, top-k 50, "
                        f"Bernoulli({reward_p}) rewards, recompute + PG fwd/bwd, no optimizer",
            "model": (f"{'flash' if cfg.compression_ratio else 'latent' if cfg.mla else 'dense'}"
                      f" depth {cfg.n_layer} d_model "
                      f"{cfg.n_embd} heads {cfg.n_head}/{cfg.n_kv_head} vocab {cfg.vocab_size}"
                      + (f" MLA latent {cfg.mla_latent} rope {cfg.mla_rope_dimension}"
                         if cfg.mla else "")
                      + (f" HCA ratio {cfg.compression_ratio} SWA {cfg.swa_window}"
                         f" CSA top-{cfg.sparse_topk} pool {cfg.indexer_pool}"
                         f" FRU {cfg.reuse_pattern}{' CED' if cfg.ced else ''}"
                         if cfg.compression_ratio else "")
                      + (f" MoE 1 shared + {cfg.n_experts} routed x {cfg.expert_hidden}, "
                         f"top-{cfg.experts_per_token}" if cfg.moe else "")),
            "rollouts": groups * S, "global_batch": groups * S, "seq_len": P + N,
            "parallelism": "single GPU",
            "rollout_ms": round(sum(roll_ms) / len(roll_ms), 2),
            "rl_step_ms": round(ms_step, 2),
            "train_ms": round(sum(train_ms) / len(train_ms), 2),
        },
        "roofline": gemm_roofline(gemm, args.config),
        "pg_loss": pg_loss_roofline(gemm),
        "decode_attention": {
            "bound": "hbm", "achieved": round(attn_gbs, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(attn_gbs / HBM_PEAK_GBS, 4), "launches": attn_n,
            "avg_launch_ms": round(attn_ms / max(attn_n, 1), 5),
            "measured_on": "an extra untimed rollout of the workload with every kernel "
                           "launched: each step's attention call (attention kernel + split "
                           "combine) timed once, in place, by events the dispatch records "
                           "(hipExtLaunchKernelGGL: first kernel's start, last kernel's end)",
        },
    }
    if opt is not None:
        res["optimizer"] = opt
    if not args.no_cpu_baseline:
        log("bench: timing the CPU oracle on a bounded sample")
        res["cpu_baseline"] = cpu_baseline(cfg, w, prompts, S, N, temp)
    print(json.dumps(res), flush=True)
    return 0


def add_gemm(acc: dict, t: dict) -> None:
    """Adds one step's train-phase GEMM timing (all products; those on the
    wide-tile engine) and policy-gradient loss timing to acc."""
    acc["ms"] += t["gemm_ms"]; acc["flops"] += t["gemm_flops"]; acc["n"] += t["gemm_launches"]
    acc["wide_ms"] += t["gemm_wide_ms"]; acc["wide_flops"] += t["gemm_wide_flops"]
    acc["wide_n"] += t["gemm_wide_launches"]
    acc["loss_ms"] += t["loss_ms"]; acc["loss_bytes"] += t["loss_bytes"]
    acc["loss_n"] += t["loss_launches"]


def _part(ms: float, flops: float, n: int) -> dict:
    tf = flops / (ms / 1e3) / 1e12 if ms else 0.0
    return {"achieved": round(tf, 2), "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4), "launches": n,
            "avg_launch_ms": round(ms / max(n, 1), 4), "share_of_gemm_time": None}


def gemm_roofline(g: dict, config: str) -> dict:
    """The dominant kernels of the step: the train phase's fp32 products
    (recompute forward, PG backward, lm_head), timed live per launch with
    HIP events on the session stream.  Every product runs on the library's
    own kernels: the large ones on the wide-tile engine (256 x 256 tiles,
    gemm_wide_kernel), the rest on gemm_kernel; `parts` splits the two."""
    tf = g["flops"] / (g["ms"] / 1e3) / 1e12 if g["ms"] else 0.0
    wide = _part(g["wide_ms"], g["wide_flops"], g["wide_n"])
    own = _part(g["ms"] - g["wide_ms"], g["flops"] - g["wide_flops"], g["n"] - g["wide_n"])
    if g["ms"]:
        wide["share_of_gemm_time"] = round(g["wide_ms"] / g["ms"], 4)
        own["share_of_gemm_time"] = round(1 - g["wide_ms"] / g["ms"], 4)
    return {
        "kernel": "train-phase fp32 GEMMs (gemm_wide_kernel + gemm_kernel, all hand-written; "
                  "recompute + PG backward + lm_head)",
        "bound": "mfma", "achieved": round(tf, 2), "peak": FP32_MFMA_PEAK_TFLOPS,
        "unit": "TFLOP/s", "frac": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
        "traffic": gemm_traffic(config), "launches": g["n"],
        "avg_launch_ms": round(g["ms"] / max(g["n"], 1), 4),
        "parts": {"gemm_wide_kernel": wide, "gemm_kernel": own},
    }


def pg_loss_roofline(g: dict) -> dict:
    """The policy-gradient loss rows (pg_loss_rows_reg_kernel: softcap, log-
    softmax, NLL and the logits gradient written over the logits), timed
    per launch with HIP events; algorithmic bytes = the logits chunk read
    once and its gradient written once.  (`bench.py --rw-rate` times a
    plain in-place rewrite of a [4096, 65536] tensor, the same read + write
    pattern with no arithmetic.)"""
    gbs = g["loss_bytes"] / (g["loss_ms"] / 1e3) / 1e9 if g["loss_ms"] else 0.0
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "launches": g["loss_n"],
            "avg_launch_ms": round(g["loss_ms"] / max(g["loss_n"], 1), 4)}


def gemm_traffic(config: str):
    """HBM bytes per train-phase GEMM launch, from the committed rocprofv3
    --pmc summary of `bench.py --phase train` (FETCH_SIZE + WRITE_SIZE,
    each scaled by the copy-kernel calibration), or None if absent."""
    path = os.path.join(ROOT, "profiles", f"train_gemms_{config}_traffic.json")
    if not os.path.exists(path):
        return None
    with open(path) as f:
        return json.load(f).get("bytes_per_launch")


def rollout_phase(args, sess, prompts, S, N, temp) -> int:
    """Rollouts alone (Engine.GenerateBatchWith for every group), for kernel
    traces and counters of the decode kernels in their place in the step:
    warmup + timed rollouts, then the decode-attention figure of the last."""
    G_, P = prompts.shape
    for i in range(args.warmup):
        sess.generate_batch(prompts, S, N, temp, 50, np.arange(G_, dtype=np.uint64) + 1000 * i)
    sess.synchronize()
    t0 = time.perf_counter()
    toks, roll = 0, []
    for i in range(args.steps):
        rows = sess.generate_batch(prompts, S, N, temp, 50,
                                   np.arange(G_, dtype=np.uint64) + 1000 * (args.warmup + i))
        toks += sum(len(r) - P for r in rows)
        roll.append(sess.timing()["rollout_ms"])
    sess.synchronize()
    wall = time.perf_counter() - t0
    t = sess.timing()
    sess.close()
    attn = t["decode_attn_bytes"] / (t["decode_attn_ms"] / 1e3) / 1e9 if t["decode_attn_ms"] else 0
    print(json.dumps({
        "metric": "rollout tokens/s", "value": round(toks / wall, 1), "unit": "tokens/s",
        "steps": args.steps, "warmup": args.warmup, "graph": not args.no_graph,
        "rollout_ms": round(sum(roll) / len(roll), 2),
        "decode_attention_last_rollout": {
            "achieved_gbs": round(attn, 1), "frac": round(attn / HBM_PEAK_GBS, 4),
            "calls": t["decode_attn_launches"],
            "avg_call_ms": round(t["decode_attn_ms"] / max(t["decode_attn_launches"], 1), 5)}}),
        flush=True)
    return 0


def train_phase(args, sess, prompts, S, N, reward_rng, reward_p) -> int:
    """Recompute + PG forward/backward alone, on a synthetic batch shaped as
    the RL step's: each prompt repeated S times followed by N uniform tokens,
    inputs/targets shifted by one, targets before the prompt end masked
    (gn_rl_step's layout), group-mean advantages of Bernoulli rewards."""
    G_, P = prompts.shape
    V = sess.cfg.vocab_size
    rng = np.random.default_rng(3)
    rows = np.concatenate([np.repeat(prompts, S, 0),
                           rng.integers(0, V, (G_ * S, N)).astype(np.int32)], 1)
    inputs, targets = rows[:, :-1].copy(), rows[:, 1:].copy()
    targets[:, :P] = -1
    rewards = (reward_rng.random(G_ * S) < reward_p).astype(np.float32)
    adv = rewards - rewards.reshape(G_, S).mean(1).repeat(S)
    norm = float(P + N)
    for _ in range(args.warmup):
        sess.zero_grad()
        sess.policy_gradient_step(inputs, targets, adv, norm)
    sess.synchronize()
    t0 = time.perf_counter()
    gemm = {"ms": 0.0, "flops": 0.0, "n": 0, "wide_ms": 0.0, "wide_flops": 0.0, "wide_n": 0,
            "loss_ms": 0.0, "loss_bytes": 0.0, "loss_n": 0}
    train = []
    for _ in range(args.steps):
        sess.zero_grad()
        loss, _ = sess.policy_gradient_step(inputs, targets, adv, norm)
        t = sess.timing()
        train.append(t["train_ms"])
        add_gemm(gemm, t)
    sess.synchronize()
    ms = 1e3 * (time.perf_counter() - t0) / args.steps
    sess.close()
    print(json.dumps({
        "metric": "train phase (recompute + PG fwd/bwd) ms", "value": round(ms, 2),
        "unit": "ms", "higher_is_better": False, "steps": args.steps, "warmup": args.warmup,
        "train_ms": round(sum(train) / len(train), 2), "loss": loss,
        "gemm": gemm_roofline(gemm, args.config)}), flush=True)
    return 0


def optimizer_timing(cfg, sess, steps: int) -> dict:
    """MuonAdamW.Step with cmd/chat_rl's groups (cmd/chat_rl/main.go:68-71)
    on the session's current gradients: wall time per step (one untimed
    step first) and the Polar Express matrix-product work it contains
    (per Muon tensor and quintic step: Gram matrix, its square and the
    polynomial product, 4*r*c*min(r,c) + 2*min(r,c)^3 flops)."""
    from gonano_amd import optimizer as OPT
    table = OPT.chat_rl_table(cfg)
    mu = table[table["kind"] == OPT.KIND_MUON]
    r, c = mu["rows"].astype(np.float64), mu["cols"].astype(np.float64)
    g = np.minimum(r, c)
    flop = float((mu["ns_steps"] * (4 * r * c * g + 2 * g ** 3)).sum())
    with OPT.Optimizer(sess, table) as opt:
        opt.step()
        sess.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            opt.step()
        sess.synchronize()
        ms = 1e3 * (time.perf_counter() - t0) / steps
    kinds = {n: int((table["kind"] == k).sum()) for n, k in
             (("adamw", OPT.KIND_ADAMW), ("muon", OPT.KIND_MUON), ("sinkhorn", OPT.KIND_SINKHORN))}
    return {"ms_per_step": round(ms, 2), "tensors": kinds,
            "polar_express_tflop": round(flop / 1e12, 4),
            "note": "optimizer.Step of RLStep (trainer/rl.go:65), excluded from ms_per_step "
                    "as the metric defines the RL step without it; its kernels' times are in "
                    "profiles/optimizer_step_d12_kernel_stats.md"}


def optimizer_phase(args, cfg, sess, prompts) -> int:
    """Optimizer steps alone (for kernel-trace profiles): gradients from one
    policy-gradient step on the first prompts, then warmup + timed steps."""
    rng = np.random.default_rng(3)
    B, T = 4, prompts.shape[1]
    inputs = prompts[:B]
    targets = rng.integers(0, cfg.vocab_size, (B, T)).astype(np.int32)
    sess.zero_grad()
    sess.policy_gradient_step(inputs, targets, np.array([1, -1, 0.5, -0.5], np.float32),
                              float(T + 1))
    res = optimizer_timing(cfg, sess, steps=args.steps)
    sess.close()
    print(json.dumps({"config": args.config, "optimizer": res}), flush=True)
    return 0


def prefix_phase(args, cfg, sess, prompts, temp) -> int:
    """The prompts' prefill (Engine.GenerateWith's step 1, one sampled token
    per prompt) without and with the device prefix cache
    (inference/cache.go): the workload's prompts share their first 3/4 with
    a stored prompt (a system prompt prefilled once, then each prompt's own
    last quarter), so with the cache every prompt continues from the stored
    keys/values over its last quarter.  Both legs run the same prompts and
    return the same kind of rows; each call's host wall time is taken."""
    G_, P = prompts.shape
    m = 3 * P // 4
    prompts = prompts.copy()
    prompts[:, :m] = prompts[0, :m]
    seeds = np.arange(G_, dtype=np.uint64)

    def timed(n):
        out = []
        for _ in range(n):
            sess.synchronize()
            t0 = time.perf_counter()
            sess.generate_batch(prompts, 1, 1, temp, 50, seeds)
            out.append(1e3 * (time.perf_counter() - t0))
        return out

    timed(args.warmup)
    full = timed(args.steps)
    sess.set_prefix_cache(max_entries=4 * G_)
    sess.generate_batch(prompts[:1, :m], 1, 1, temp, 50, seeds[:1])  # the shared prefix, stored
    timed(args.warmup)
    cached = timed(args.steps)
    hits = sess.prefix_cache_hits(G_)
    entries, nbytes = sess.prefix_cache_len()
    sess.close()
    assert (hits == m).all(), hits
    med = lambda v: float(np.median(v))  # noqa: E731
    print(json.dumps({
        "metric": "prompt prefill ms (one sampled token per prompt)", "config": args.config,
        "prompts": G_, "prompt_len": P, "cached_prefix": m, "steps": args.steps,
        "full_prefill_ms": round(med(full), 3), "cached_prefill_ms": round(med(cached), 3),
        "speedup": round(med(full) / med(cached), 2),
        "prefill_tokens_full": G_ * P, "prefill_tokens_cached": G_ * (P - m),
        "cache_entries": entries, "cache_bytes": nbytes}), flush=True)
    return 0


def copy_calibration() -> int:
    """A plain device copy of known size for scaling HBM byte counters:
    torch's copy kernel run 5 times over 1 GiB (reads 1 GiB, writes 1 GiB)."""
    import torch
    n = 1 << 28  # floats = 1 GiB
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": 4 * n, "copies": 5}), flush=True)
    return 0


def rw_rate() -> int:
    """Rates of a 1 GiB device copy and of an in-place rewrite of a
    [4096, 65536] float32 tensor (torch's elementwise multiply: each float
    read once and written once, the pattern of a kernel that rewrites the
    logits it reads), timed with events after two untimed passes."""
    import torch
    n = 1 << 28
    src = torch.ones(n, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)

    def rate(fn) -> float:
        for _ in range(2):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(5):
            fn()
        b.record()
        torch.cuda.synchronize()
        return round(2 * 4 * n / (a.elapsed_time(b) / 5 / 1e3) / 1e9, 1)

    copy_gbs = rate(lambda: dst.copy_(src))
    x = src.view(4096, 65536)
    inplace_gbs = rate(lambda: x.mul_(1.0))
    print(json.dumps({"copy_gbs": copy_gbs, "copy_frac": round(copy_gbs / HBM_PEAK_GBS, 4),
                      "inplace_rw_gbs": inplace_gbs,
                      "inplace_rw_frac": round(inplace_gbs / HBM_PEAK_GBS, 4)}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Writes tests/golden/flash_long.npz: the oracle's results for the flash
workload's prompt length (8192-token prompts, SequenceLen 16384), which the
oracle needs many minutes to compute and the GPU test
(tests/test_gpu_flash_long.py) therefore reads from this file.  The case --
model, weights, inputs, sampled gradient entries -- is
tests/golden/flash_long_case.py.  Stored:

  fwd_last   Transformer.Forward logits of the prompt's last position
  rows       Engine.GenerateBatchWith of one group (16 samples, 4 new
             tokens, T 1.0, top-k 50, group seed 1000): the oracle's tokens
             (-1 past a row's terminal token)
  step_top   per decode step and row, the 64 largest logits' indices and
  step_val   values on the oracle's own trajectory
  loss32/64, nll32/64
             PolicyGradientStep over one 8703-token sequence (the prompt,
             511 generated tokens; the prompt positions without targets),
             advantage 0.3, norm 8704, from the oracle's float32 and
             float64 builds
  g_norm32/64, g_idx, g_val32/64
             per parameter tensor: the gradient's norm and its values at
             GSAMPLE indices drawn with default_rng(tensor number)

    python tests/golden/make_flash_long.py
"""
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import flash_long_case as case  # noqa: E402
from oracle import oracle as orc  # noqa: E402

T0 = time.time()


def log(msg):
    print(f"[{time.time() - T0:7.0f} s] {msg}", flush=True)


def main():
    cfg = case.config()
    w = case.weights(cfg)
    prompt, pg_in, pg_tg = case.inputs(cfg)
    P, S, N, T_PG, TOPN = case.P, case.S, case.N, case.T_PG, case.TOPN
    m32 = orc.OracleModel(orc.ModelShape.from_config(cfg), w)
    out = {}
    log("forward")
    out["fwd_last"] = m32.forward(prompt[None, :])[0, -1].astype(np.float32)
    log("rollout")
    got = m32.generate_batch(prompt, S, N, 1.0, 50, case.SEED_GROUP)
    rows = np.full((S, N), -1, np.int32)  # -1: past the row's terminal token
    for i, r in enumerate(got):
        rows[i, :len(r) - P] = r[P:]
    out["rows"] = rows
    log("decode (teacher forced)")
    cols = np.ascontiguousarray(np.maximum(rows[:, :N - 1], 0).T)
    z = m32.decode_forced(prompt, cols)  # [N, S, V]
    top = np.argsort(-z, axis=-1, kind="stable")[..., :TOPN]
    out["step_top"] = top.astype(np.int32)
    out["step_val"] = np.take_along_axis(z, top, -1).astype(np.float32)
    adv = np.array([case.ADV], np.float32)
    idx = case.sample_indices(cfg)
    for name, dt in (("32", np.float32), ("64", np.float64)):
        log("pg step float" + name)
        m = m32 if dt == np.float32 else orc.OracleModel(orc.ModelShape.from_config(cfg),
                                                         w.astype(np.float64), dtype=np.float64)
        loss, nll, g = m.pg_step(pg_in, pg_tg, adv, float(T_PG + 1))
        out["loss" + name] = np.float64(loss)
        out["nll" + name] = np.asarray(nll, np.float64).reshape(1, T_PG)[:, P:]
        norms, vals = [], []
        for (pname, r, c, off), ix in zip(cfg.param_table(), idx):
            t = np.asarray(g[off:off + r * c], np.float64)
            norms.append(np.linalg.norm(t))
            vals.append(t[ix])
        out["g_norm" + name] = np.array(norms)
        out["g_val" + name] = np.concatenate(vals)
    out["g_idx"] = np.concatenate(idx).astype(np.int64)
    np.savez_compressed(os.path.join(HERE, "flash_long.npz"), **out)
    log("written")


if __name__ == "__main__":
    main()

"""Teacher-forced check of one rollout group against the oracle.

Engine.GenerateWith (inference/engine.go:131-325) samples step t of a group
from the logits of the columns fed before it, with the group's own RNG
stream consuming S*V draws per step (tensors/random.go:60-80).  Given the
rows another engine produced, the oracle recomputes those logits with the
same columns fed (orc_decode_forced) and samples every step from the group
stream; each sampled token of a row must equal the row's token.  This checks
every column of every row without depending on the oracle's own rollout
staying on the same tokens (a near-tie flip early on would otherwise change
every later column).

A row that ends before max_tokens ended on a terminal token, which the
oracle must sample there.  A row's tokens after its terminal token are not returned
(GenerateBatchWith, engine.go:349-366): its later columns are fed as 0 --
rows are independent, so this changes no other row's logits -- and it is
not checked past its end.  After a row's <|tool_end|> the next columns may
be forced tool output, so checking of that row stops there.
"""
import numpy as np


def teacher_forced_group(orc, model, prompt, rows, seed, max_tokens, temperature, top_k,
                         tool_end=262, terminals=(256, 260)):
    """Checks one group's rows (prompt + completion) and returns the number
    of sampled tokens compared."""
    prompt = np.asarray(prompt, np.int32).reshape(-1)
    P, S = prompt.size, len(rows)
    ncols = max_tokens - 1
    cols = np.zeros((max(ncols, 0), S), np.int32)
    for i, r in enumerate(rows):
        assert np.array_equal(r[:P], prompt), "row does not start with its prompt"
        comp = np.asarray(r[P:P + ncols], np.int32)
        cols[:comp.size, i] = comp
    z = model.decode_forced(prompt, cols)
    rng = orc.GoRNG(int(seed))
    live = [True] * S
    checked = 0
    for t in range(max_tokens):
        want = orc.sample_next_token(np.ascontiguousarray(z[t], np.float32), rng, temperature,
                                     top_k)
        for i, r in enumerate(rows):
            if not live[i]:
                continue
            if P + t >= len(r):
                # the row ended here: its (unrecorded) token was a terminal one
                assert want[i] in terminals, f"row {i} ended at step {t}; oracle samples {want[i]}"
                live[i] = False
                continue
            assert r[P + t] == want[i], f"row {i} step {t}: got {r[P + t]}, oracle samples {want[i]}"
            checked += 1
            if r[P + t] == tool_end:
                live[i] = False
        if not any(live):
            break
    return checked

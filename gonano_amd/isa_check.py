"""Checks the gfx950 assembly of the library's kernels for the wide-store
data hazard: a store of more than 8 bytes (global/flat/buffer
*_dwordx3/x4) whose data registers are written by the VALU instruction
right after it.  The hardware may read the store data after that write
(measured on MI355X: the last lanes of 16-lane groups stored the new
value).  The compiler inserts the required wait state for global and flat
stores but not for buffer stores that take their offset from an SGPR, so
kernels store through global pointers; this check keeps it that way.

    python -m gonano_amd.isa_check      # compiles every .hip, prints findings
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import sys
import tempfile

from . import build

_KERNEL = re.compile(r"^(_Z[^\s:]+):", re.M)
_RANGE = re.compile(r"v\[(\d+):(\d+)\]")
_DEST = re.compile(r"v_\S+\s+(?:v(\d+)|v\[(\d+):(\d+)\])")


def _store_data(line: str):
    """(first, last) data VGPR of a store wider than 8 bytes, else None."""
    if line.startswith(("global_store_dwordx", "flat_store_dwordx")):
        regs = _RANGE.findall(line)
        data = regs[1] if len(regs) >= 2 else None  # address first, then data
    elif line.startswith("buffer_store_dwordx"):
        regs = _RANGE.findall(line)
        data = regs[0] if regs else None
    else:
        return None
    if not data:
        return None
    lo, hi = int(data[0]), int(data[1])
    return (lo, hi) if hi - lo + 1 > 2 else None


def scan(asm: str) -> list[str]:
    """Findings 'kernel: store | next instruction' in one assembly file."""
    out = []
    labels = [(m.start(), m.group(1)) for m in _KERNEL.finditer(asm)]
    for i, (pos, name) in enumerate(labels):
        end = labels[i + 1][0] if i + 1 < len(labels) else len(asm)
        lines = [l.strip() for l in asm[pos:end].split("\n")]
        for j, line in enumerate(lines):
            rng = _store_data(line)
            if not rng:
                continue
            k = j + 1
            while k < len(lines) and (not lines[k] or lines[k].startswith((";", "."))):
                k += 1
            nxt = lines[k] if k < len(lines) else ""
            m = _DEST.match(nxt)
            if not m:
                continue
            first = int(m.group(1) or m.group(2))
            last = int(m.group(1) or m.group(3))
            if first <= rng[1] and last >= rng[0]:
                out.append(f"{name}: {line} | {nxt}")
    return out


def _asm(src: str, outdir: str) -> str:
    out = os.path.join(outdir, os.path.splitext(src)[0] + ".s")
    flags = [f for f in build.FLAGS if f not in ("-fPIC",)]
    cmd = [build.hipcc(), *flags, "--cuda-device-only", "-S", os.path.join(build.CSRC, src),
           "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"assembly of {src} failed\n{r.stderr}")
    with open(out) as f:
        return f.read()


def check() -> list[str]:
    """Compiles every device source to assembly and returns all findings."""
    srcs = [s for s in build.SOURCES if s.endswith(".hip")]
    with tempfile.TemporaryDirectory() as d:
        jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", "8")))
        with cf.ThreadPoolExecutor(jobs) as ex:
            asms = list(ex.map(lambda s: _asm(s, d), srcs))
    return [f"{src}: {f}" for src, a in zip(srcs, asms) for f in scan(a)]


if __name__ == "__main__":
    found = check()
    for f in found:
        print(f)
    print(f"{len(found)} wide-store hazards")
    sys.exit(1 if found else 0)

"""Checks the gfx950 assembly of the library's kernels for two hazards the
compiler does not cover.

Wide-store data hazard: a store of more than 8 bytes (global/flat/buffer
*_dwordx3/x4) whose data registers are written by the VALU instruction
right after it.  The hardware may read the store data after that write
(measured on MI355X: the last lanes of 16-lane groups stored the new
value).  The compiler inserts the required wait state for global and flat
stores but not for buffer stores that take their offset from an SGPR, so
kernels store through global pointers; this check keeps it that way.

Inline-asm MFMA results: the wide GEMM issues its MFMAs as inline asm
(accumulators tied to AGPRs), which the compiler's hazard recognizer does
not see as MFMAs, so it inserts no wait states before an instruction that
reads or rewrites their AGPRs.  Every such access must come at least
MFMA_GAP wait states (one per instruction, n + 1 per s_nop n) after the
asm MFMA that wrote the register, along every path including a loop's
back edge.  The requirement for a 16x16x4 f32 MFMA's result is 11-12;
the check asks for 16.

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


MFMA_GAP = 16
_AREG = re.compile(r"\ba(\d+)\b|\ba\[(\d+):(\d+)\]")
_LABEL = re.compile(r"^(\.?[A-Za-z_$][\w.$]*):")
_BRANCH = re.compile(r"^s_(?:c?branch\w*)\s+(\S+)")


def _aregs(operands: str) -> set[int]:
    s = set()
    for m in _AREG.finditer(operands):
        if m.group(1) is not None:
            s.add(int(m.group(1)))
        else:
            s.update(range(int(m.group(2)), int(m.group(3)) + 1))
    return s


def scan_mfma_gaps(asm: str) -> list[str]:
    """Findings 'kernel: access | distance' for AGPR accesses closer than
    MFMA_GAP wait states to the inline-asm MFMA that wrote the register."""
    out = []
    labels = [(m.start(), m.group(1)) for m in _KERNEL.finditer(asm)]
    for i, (pos, name) in enumerate(labels):
        end = labels[i + 1][0] if i + 1 < len(labels) else len(asm)
        # instructions: (text, is_asm_mfma, label or None)
        ins = []
        in_asm = False
        for raw in asm[pos:end].split("\n"):
            line = raw.strip()
            if line.startswith(";;#ASMSTART"):
                in_asm = True
                continue
            if line.startswith(";;#ASMEND"):
                in_asm = False
                continue
            if not line or line.startswith((";", ".p2align", ".section", ".globl", ".type")):
                continue
            lm = _LABEL.match(line)
            if lm:
                ins.append(("", False, lm.group(1)))
                continue
            if line.startswith("."):
                continue
            ins.append((line.split(";")[0].strip(), in_asm and line.startswith("v_mfma"), None))
        if not any(a for _, a, _ in ins):
            continue
        jumps: dict[str, list[int]] = {}
        for k, (t, _, _) in enumerate(ins):
            b = _BRANCH.match(t)
            if b:
                jumps.setdefault(b.group(1), []).append(k)

        def waits(t: str) -> int:
            if t.startswith("s_nop"):
                return int(t.split()[1], 0) + 1
            return 1

        def close_writer(k: int, regs: set[int]) -> int | None:
            """Smallest wait-state distance from an asm MFMA writing regs to
            instruction k, over the paths that reach k (None if >= MFMA_GAP)."""
            best = None
            stack = [(k - 1, 0, frozenset())]
            while stack:
                j, dist, seen = stack.pop()
                while j >= 0 and dist < MFMA_GAP:
                    t, is_mfma, lab = ins[j]
                    if lab is not None:
                        for src in jumps.get(lab, []):
                            if (lab, src) not in seen:
                                stack.append((src, dist, seen | {(lab, src)}))
                        j -= 1
                        continue
                    if is_mfma:
                        dst = _aregs(t.split(",")[0])
                        if dst & regs:
                            best = dist if best is None else min(best, dist)
                            break
                    dist += waits(t)
                    if t.startswith("s_branch"):
                        break  # no fall-through into k from here
                    j -= 1
            return best

        for k, (t, is_mfma, lab) in enumerate(ins):
            if lab is not None or is_mfma or not t:
                continue
            regs = _aregs(t.split(" ", 1)[1] if " " in t else "")
            if not regs:
                continue
            d = close_writer(k, regs)
            if d is not None:
                out.append(f"{name}: {t} | {d} wait states after an asm MFMA")
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
    return [f"{src}: {f}" for src, a in zip(srcs, asms) for f in scan(a) + scan_mfma_gaps(a)]


if __name__ == "__main__":
    found = check()
    for f in found:
        print(f)
    print(f"{len(found)} hazards")
    sys.exit(1 if found else 0)

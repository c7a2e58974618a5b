"""Check the library's gfx950 assembly for MFMA results read too early.

The kernels keep MFMA accumulators in ordinary VGPRs
(`-mllvm -amdgpu-mfma-vgpr-form`, build.py). With that flag the compiler's
hazard pass once emitted no wait states between an MFMA and a VALU read of
its result when a branch sat between them, and flash prefill read partly
accumulated scores. This scan guards against that coming back: for every
`v_mfma*` with a VGPR destination it follows the instruction stream, along
the fall-through and into branch targets, and reports any instruction that
reads one of the destination registers before the result's wait states
have passed (a 32x32 product needs 18, a 16x16 one 8; `s_nop n` counts
n + 1, any other instruction 1). A following MFMA that only accumulates
into the same registers (srcC) is not a read. Along a path on which no lane
is active (the fall-through of `s_cbranch_execnz`, the target of
`s_cbranch_execz`) vector instructions read nothing until a scalar
instruction writes `exec` again.

`python -m torchnative_amd.hazard_scan` compiles every source to assembly
with the build's flags and prints the findings; tests/test_hazard_scan.py
requires there to be none.
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

from . import build

WAIT = {"32x32": 18, "16x16": 8}
_LABEL = re.compile(r"^(\.LBB\d+_\d+):")
_FUNC = re.compile(r"^(_Z\S+):")


def _vregs(operand: str) -> set:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", operand)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", operand)
    return {int(m.group(1))} if m else set()


def _parse(lines):
    """(instructions [(op, operands, text)], labels {name: index})."""
    ins, labels = [], {}
    for raw in lines:
        t = raw.split(";")[0].strip()
        if not t:
            continue
        m = _LABEL.match(t)
        if m:
            labels[m.group(1)] = len(ins)
            continue
        if t.startswith("."):
            continue
        parts = t.replace(",", " ").split()
        ins.append((parts[0], parts[1:], t))
    return ins, labels


def _reads(op: str, args: list) -> set:
    """VGPRs an instruction reads."""
    if op.startswith("s_"):
        return set()
    if op.startswith(("ds_write", "buffer_store", "global_store", "flat_store", "scratch_store")):
        return set().union(*(_vregs(a) for a in args)) if args else set()
    if op.startswith("v_mfma"):
        return set().union(*(_vregs(a) for a in args[1:3]))  # A and B; C chains an accumulation
    return set().union(*(_vregs(a) for a in args[1:])) if len(args) > 1 else set()


def scan_function(lines, name="?", max_depth=4):
    """Findings [(function, mfma text, reader text, wait states before the read)]."""
    ins, labels = _parse(lines)
    found = []
    for i, (op, args, text) in enumerate(ins):
        if not op.startswith("v_mfma") or not args:
            continue
        dst = _vregs(args[0])
        if not dst:
            continue
        need = WAIT["32x32"] if "32x32" in op else WAIT["16x16"]
        todo, seen = [(i + 1, 0, 0, False)], set()
        while todo:
            j, waited, depth, idle = todo.pop()  # idle: exec is zero on this path
            while j < len(ins) and waited < need:
                if (j, waited, idle) in seen:
                    break
                seen.add((j, waited, idle))
                op2, args2, text2 = ins[j]
                if not idle and _reads(op2, args2) & dst:
                    found.append((name, text, text2, waited))
                    break
                if op2.startswith("s_") and args2 and args2[0] == "exec":
                    idle = False
                if op2.startswith("s_cbranch") or op2 == "s_branch":
                    target = args2[0] if args2 else ""
                    if target in labels and depth < max_depth:
                        todo.append((labels[target], waited + 1, depth + 1, idle or op2 == "s_cbranch_execz"))
                    if op2 == "s_branch":
                        break
                    if op2 == "s_cbranch_execnz":
                        idle = True  # the fall-through runs with no lane active
                if op2 == "s_endpgm":
                    break
                waited += int(args2[0], 0) + 1 if op2 == "s_nop" else 1
                j += 1
    return found


def scan_text(asm: str):
    lines = asm.split("\n")
    starts = [k for k, l in enumerate(lines) if _FUNC.match(l)]
    found = []
    for a, b in zip(starts, starts[1:] + [len(lines)]):
        found += scan_function(lines[a + 1:b], _FUNC.match(lines[a]).group(1))
    return found


def assembly(src: str, outdir: str) -> str:
    """The gfx950 device assembly of one source, built with the library's flags."""
    out = os.path.join(outdir, os.path.basename(src) + ".s")
    cmd = [build.HIPCC, *build.FLAGS, "--cuda-device-only", "-S", os.path.join(build.CSRC, src), "-o", out]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src}:\n{r.stderr[-2000:]}")
    with open(out) as fh:
        return fh.read()


def scan_sources(sources=None):
    """{source: findings} for the library's sources, compiled side by side."""
    sources = list(sources or build.SOURCES)
    with tempfile.TemporaryDirectory() as tmp, ThreadPoolExecutor(max_workers=len(sources)) as pool:
        texts = list(pool.map(lambda s: assembly(s, tmp), sources))
    return {s: scan_text(t) for s, t in zip(sources, texts)}


if __name__ == "__main__":
    bad = 0
    for src, found in scan_sources().items():
        for fn, mfma, reader, waited in found:
            bad += 1
            print(f"{src}: {fn[:70]}: `{reader}` reads `{mfma}` after {waited} wait states")
    print(f"{bad} early reads")
    sys.exit(1 if bad else 0)

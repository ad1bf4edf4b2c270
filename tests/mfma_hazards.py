"""Static check of the gfx950 assembly of the HIP kernels for MFMA data hazards.

The kernels issue every MFMA from inline asm with the accumulator tied in place and read an
accumulator only after ``drain()`` (24 wait states).  That discipline holds only if the
compiler never places an instruction that touches an MFMA's registers right after it -- which
it did once, copying an accumulator element at a control-flow merge 2 wait states after the
last MFMA of a chain.  This script compiles each ``csrc/*.hip`` to assembly and reports, per
kernel, every instruction within ``window`` wait states after a ``v_mfma*`` that

  * reads or writes a register the MFMA writes (RAW / WAW), other than the next MFMA of the
    same in-place chain, or
  * writes a register the MFMA reads as its accumulator input (WAR).

Wait states: one per instruction, ``s_nop N`` counts N + 1.  Code is followed in program
order (branches are not followed), which is how the straight-line MFMA chains are written.

Usage: ``python tests/mfma_hazards.py`` (exit status 1 if any hazard is found).
"""
from __future__ import annotations

import re
import subprocess
import sys
import tempfile
from pathlib import Path

PKG = Path(__file__).resolve().parents[1] / "atomic-ops_amd"
sys.path.insert(0, str(PKG))
from build_lib import HIPFLAGS, _hipcc  # noqa: E402

_RANGE = re.compile(r"v\[(\d+):(\d+)\]")
_ONE = re.compile(r"v(\d+)$")


def _regs(tok: str) -> set:
    tok = tok.strip()
    m = _RANGE.match(tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = _ONE.match(tok)
    return {int(m.group(1))} if m else set()


def scan(asm: str, window: int = 24) -> dict:
    """Return {kernel: [(mfma_line, other_line, kind), ...]} for the assembly text."""
    issues: dict = {}
    kern = None
    inflight = []                      # (age, dst regs, srcC regs not in dst, line)
    for i, line in enumerate(asm.splitlines()):
        m = re.match(r"^(_Z\w+):", line)
        if m:
            kern, inflight = m.group(1), []
            continue
        s = line.strip()
        if not s or s.startswith((";", ".")) or s.endswith(":"):
            continue
        op = s.split()[0]
        ops = [t.strip() for t in s[len(op):].split(",")]
        ws = int(re.match(r"s_nop (\d+)", s).group(1)) + 1 if op == "s_nop" else 1
        if op.startswith("v_mfma"):
            dst = _regs(ops[0])
            srcc = _regs(ops[3]) if len(ops) > 3 else set()
            ab = _regs(ops[1]) | _regs(ops[2])
            for age, d, c, li in inflight:
                if ab & d:
                    issues.setdefault(kern, []).append((li, i, "RAW-AB"))
                if dst & d and srcc != d:
                    issues.setdefault(kern, []).append((li, i, "WAW-MFMA"))
            inflight = [(age + ws, d, c, li) for age, d, c, li in inflight if age + ws < window]
            inflight.append((0, dst, srcc - dst, i))
            continue
        dest = set()
        if not op.startswith(("global_store", "ds_write", "buffer_store", "scratch_store", "s_")):
            if ops and ops[0]:
                dest = _regs(ops[0])
        reads = set()
        for t in (ops[1:] if dest else ops):
            if t:
                reads |= _regs(t.split()[0])
        for age, d, c, li in inflight:
            if dest & c:
                issues.setdefault(kern, []).append((li, i, "WAR"))
            if (reads | dest) & d:
                issues.setdefault(kern, []).append((li, i, "RAW"))
        inflight = [(age + ws, d, c, li) for age, d, c, li in inflight if age + ws < window]
    return issues


def check_all(window: int = 24, verbose: bool = True) -> dict:
    found = {}
    with tempfile.TemporaryDirectory() as td:
        for src in sorted((PKG / "csrc").glob("*.hip")):
            out = Path(td) / (src.stem + ".s")
            cmd = [_hipcc(), *HIPFLAGS, "--cuda-device-only", "-S", str(src), "-o", str(out)]
            r = subprocess.run(cmd, capture_output=True, text=True)
            if r.returncode != 0:
                raise RuntimeError(f"hipcc -S failed on {src.name}:\n{r.stderr}")
            iss = scan(out.read_text(), window)
            for k, v in iss.items():
                found[f"{src.name}:{k}"] = v
            if verbose:
                print(f"{src.name}: {sum(len(v) for v in iss.values())} hazard(s)")
    return found


if __name__ == "__main__":
    res = check_all()
    for k, v in res.items():
        print(k[:100], v[:4])
    sys.exit(1 if res else 0)

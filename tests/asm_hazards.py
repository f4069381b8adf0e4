"""Checker for in-flight LDS reads issued by inline asm in the gfx950 assembly of this build.

Several kernels read LDS fragments with inline ``ds_read_*`` statements and wait for them with an
explicit ``s_waitcnt lgkmcnt(N)`` (the compiler cannot see that such a read is a load, so it does
not insert that wait itself).  Until the wait, the destination registers hold stale data, and any
instruction the compiler places in between that reads or writes them (a copy to an AGPR under
register pressure, a reuse of the register) is a silent wrong-result hazard.  This module compiles
a HIP source to gfx950 assembly and scans every kernel linearly:

* an inline ``ds_read*`` (between ``;;#ASMSTART`` and ``;;#ASMEND``) becomes pending;
* every later DS instruction counts as issued after it (LDS operations complete in order);
* ``s_waitcnt lgkmcnt(N)`` retires a pending read once at least N DS operations were issued after
  it;
* any other instruction that names a register of a pending read is reported.

The scan follows the text order, so a pending read also reaches code placed after a branch; such a
report is checked by hand before the code is changed.
"""

from __future__ import annotations

import re
import subprocess
import tempfile
from pathlib import Path

REPO = Path(__file__).resolve().parents[1]
CSRC = REPO / "pymsst_amd" / "csrc"

_REG = re.compile(r"\b([va])(?:(\d+)|\[(\d+):(\d+)\])")
_LGKM = re.compile(r"lgkmcnt\((\d+)\)")


def device_asm(src: Path, out_dir: Path) -> Path:
    """gfx950 device assembly of ``src`` with the build's flags."""
    from pymsst_amd import build

    out = out_dir / (src.stem + ".s")
    flags = [f for f in build.HIPCC_FLAGS if f not in ("-fPIC", "-Wall", "-Wno-unused-function")]
    flags += build.extra_flags(src.name)
    cmd = [build.hipcc(), *flags, "--offload-device-only", "-S", str(src), "-o", str(out)]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return out


def _regs(text: str) -> set[tuple[str, int]]:
    out = set()
    for kind, single, lo, hi in _REG.findall(text):
        if single:
            out.add((kind, int(single)))
        else:
            out.update((kind, r) for r in range(int(lo), int(hi) + 1))
    return out


def kernels(asm: str) -> dict[str, list[str]]:
    """Kernel name -> its instruction lines (comments stripped, asm markers kept)."""
    out = {}
    for m in re.finditer(r"^(_Z\w+):\s*(?:;.*)?$", asm, re.M):
        name = m.group(1)
        end = asm.find(".Lfunc_end", m.end())
        body = asm[m.end(): end if end >= 0 else len(asm)]
        out[name] = body.splitlines()
    return out


def scan(lines: list[str]) -> list[str]:
    """Hazards of one kernel: uses of a pending inline-asm LDS read's registers before its wait."""
    pending: list[list] = []  # [registers, ds ops issued after, line]
    in_asm = False
    found = []
    for no, raw in enumerate(lines):
        line = raw.strip()
        if line.startswith(";;#ASMSTART"):
            in_asm = True
            continue
        if line.startswith(";;#ASMEND"):
            in_asm = False
            continue
        code = line.split(";", 1)[0].strip()
        if not code or code.endswith(":") or code.startswith("."):
            continue
        op = code.split()[0]
        if op == "s_waitcnt":
            m = _LGKM.search(code)
            if m:
                n = int(m.group(1))
                pending = [p for p in pending if p[1] < n]
            continue
        operands = code[len(op):]
        regs = _regs(operands)
        for p in pending:
            if regs & p[0]:
                found.append(f"line {no}: '{code}' touches {sorted(regs & p[0])[:4]} of the read at {p[2]}")
        if op.startswith("ds_"):
            for p in pending:
                p[1] += 1
            if in_asm and op.startswith("ds_read"):
                dest = operands.split(",")[0]
                pending.append([_regs(dest), 0, f"line {no} '{code}'"])
    return found


def check_source(src: Path) -> dict[str, list[str]]:
    """Hazards per kernel of one HIP source (kernels without any are left out)."""
    with tempfile.TemporaryDirectory() as tmp:
        asm = device_asm(src, Path(tmp)).read_text()
    result = {}
    for name, lines in kernels(asm).items():
        bad = scan(lines)
        if bad:
            result[name] = bad
    return result


_SCRATCH = re.compile(r"^\s*\.(?:amdhsa_)?private_segment_fixed_size:?\s+(\d+)", re.M)


def scratch_bytes(asm: str) -> dict[str, int]:
    """Per-lane scratch (register spill) bytes of every kernel of an assembly listing."""
    out = {}
    for m in re.finditer(r"^\s*\.amdhsa_kernel\s+(\S+)(.*?)\.end_amdhsa_kernel", asm, re.M | re.S):
        s = _SCRATCH.search(m.group(2))
        out[m.group(1)] = int(s.group(1)) if s else 0
    return out


def spills_of_source(src: Path) -> dict[str, int]:
    """Kernels of one HIP source that use scratch memory (spilled registers), with the bytes per lane."""
    with tempfile.TemporaryDirectory() as tmp:
        asm = device_asm(src, Path(tmp)).read_text()
    return {k: v for k, v in scratch_bytes(asm).items() if v}

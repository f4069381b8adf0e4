"""No inline-asm LDS read of any kernel has its registers touched before its explicit wait, and no
kernel spills registers to scratch memory.

Compiles every ``pymsst_amd/csrc/*.hip`` to gfx950 assembly with the build's flags and scans each
kernel (``tests/asm_hazards.py``).  Also checks that the scan finds a planted hazard.  A spill turns
a register-resident kernel into one that streams its accumulators through memory (a conditional
GEMM tile once made the mask-MLP forward spill 420 bytes per lane and run six times slower).
"""

from __future__ import annotations

import concurrent.futures as cf
import shutil

import pytest

from tests import asm_hazards as ah

pytestmark = pytest.mark.skipif(shutil.which("hipcc") is None and not ah.Path("/opt/rocm/bin/hipcc").exists(),
                                reason="hipcc not available")


def test_no_inline_lds_read_hazards():
    sources = sorted(ah.CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=8) as pool:
        results = dict(zip(sources, pool.map(ah.check_source, sources)))
    bad = {src.name: {k: v[:3] for k, v in r.items()} for src, r in results.items() if r}
    assert not bad, bad


def test_no_kernel_spills_registers():
    sources = sorted(ah.CSRC.glob("*.hip"))
    with cf.ThreadPoolExecutor(max_workers=8) as pool:
        results = dict(zip(sources, pool.map(ah.spills_of_source, sources)))
    bad = {src.name: r for src, r in results.items() if r}
    assert not bad, bad


def test_scratch_parser_reads_the_kernel_descriptor():
    asm = "\n".join([
        "\t.amdhsa_kernel _Z1av", "\t\t.amdhsa_private_segment_fixed_size 0", "\t.end_amdhsa_kernel",
        "\t.amdhsa_kernel _Z1bv", "\t\t.amdhsa_private_segment_fixed_size 420", "\t.end_amdhsa_kernel",
    ])
    assert ah.scratch_bytes(asm) == {"_Z1av": 0, "_Z1bv": 420}


def test_scan_finds_a_planted_copy():
    lines = [
        ";;#ASMSTART", "ds_read_b128 v[4:7], v1", ";;#ASMEND",
        "v_mov_b32_e32 v20, v5",  # reads a register of the read in flight
        ";;#ASMSTART", "s_waitcnt lgkmcnt(0)", ";;#ASMEND",
        "v_mfma_f32_16x16x32_bf16 a[0:3], v[4:7], v[8:11], 0",
    ]
    found = ah.scan(lines)
    assert len(found) == 1 and "v_mov_b32_e32 v20, v5" in found[0]
    # after the wait the same use is fine
    assert not ah.scan(lines[:3] + lines[4:7] + lines[3:4])


def test_wait_with_later_reads_still_covers_earlier_ones():
    lines = [
        ";;#ASMSTART", "ds_read_b128 v[4:7], v1", ";;#ASMEND",
        ";;#ASMSTART", "ds_read_b128 v[8:11], v2", ";;#ASMEND",
        ";;#ASMSTART", "s_waitcnt lgkmcnt(1)", ";;#ASMEND",
        "v_mov_b32_e32 v20, v5",   # first read retired
        "v_mov_b32_e32 v21, v9",   # second still in flight
    ]
    found = ah.scan(lines)
    assert len(found) == 1 and "v21" in found[0]

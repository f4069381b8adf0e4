"""The final-layer dz kernel's ring waits (``pymsst_amd/csrc/mask_dz.hip``, ``ring_step``) against a
model of one wave's vmcnt queue.

Loads and global->LDS DMAs of a wave retire in issue order, so ``s_waitcnt vmcnt(n)`` guarantees
that everything but the last ``n`` issued operations has landed.  The kernel issues the first
``S - 1`` chunks' DMAs, then one chunk per ring step, and before chunk ``c`` is read it waits with
an allowance computed in closed form.  The model issues the same sequence and counts the
operations issued after chunk ``c``'s last DMA: the allowance must equal that count (smaller waits
longer than needed, larger reads a stage that may not have landed).  The model also covers loads
issued right after the first chunks (``early``), as a variant that loads the epilogue's input
early would issue them, with their allowance for the chunks issued before them.  Planted mistakes,
one chunk too many allowed and early loads allowed for every chunk, are caught.
"""

from __future__ import annotations

import pytest

STAGES = 4  # kDzStages
NT = 2      # 16-row tiles per wave


def shapes():
    """(DT, weight DMAs per wave per chunk, epilogue units per thread) of the kernel's
    instantiations: HT = 16 DT hidden columns, kInstr = DT slab DMAs over 4 waves, 4 x 32 rows x
    HT / 8 units over 256 threads."""
    for dt in (8, 12):
        yield dt, dt // 4, 4 * 16 * NT * (16 * dt // 8) // 256


def allowance(c, nc, per_chunk, early=0, mistake=None):
    """The kernel's ring_step allowance for chunk c of nc (with `early` loads after the first chunks)."""
    after = min(nc - 1 - c, STAGES - 2)
    if mistake == "one_chunk_more":
        after += 1
    extra = early if (mistake == "early_always" or c < STAGES - 1) else 0
    return after * per_chunk + extra


def queue_mismatches(nc, npw, nvt, early=0, mistake=None):
    per_chunk = npw + nvt
    issued = []
    for c in range(min(STAGES - 1, nc)):
        issued += [("chunk", c)] * per_chunk
    issued += [("early", None)] * early
    bad = []
    for c in range(nc):
        last = max(i for i, op in enumerate(issued) if op == ("chunk", c))
        after_last = len(issued) - 1 - last
        allow = allowance(c, nc, per_chunk, early, mistake)
        if allow != after_last:
            bad.append((c, allow, after_last))
        if c + STAGES - 1 < nc:
            issued += [("chunk", c + STAGES - 1)] * per_chunk
    return bad


@pytest.mark.parametrize("with_early", [False, True])
def test_ring_wait_allowances_match_the_issue_order(with_early):
    for dt, npw, units in shapes():
        early = units if with_early else 0
        # the template bound of ring_vm_wait: (S - 2) (kMaxPW + NT) (+ the early loads)
        bound = (STAGES - 2) * ((dt + 3) // 4 + NT) + early
        for nc in range(1, 40):
            for nvt in range(NT + 1):
                assert not queue_mismatches(nc, npw, nvt, early), (dt, nc, nvt)
                assert max(allowance(c, nc, npw + nvt, early) for c in range(nc)) <= bound


def test_planted_allowance_mistakes_are_caught():
    dt, npw, units = next(iter(shapes()))
    assert not queue_mismatches(6, npw, NT)
    assert queue_mismatches(6, npw, NT, mistake="one_chunk_more")
    assert not queue_mismatches(6, npw, NT, early=units)
    assert queue_mismatches(6, npw, NT, early=units, mistake="early_always")

"""The final-layer dz kernel's ring waits (``pymsst_amd/csrc/mask_dz.hip``, ``ring_step``) against a
model of one wave's vmcnt queue.

Loads and global->LDS DMAs of a wave retire in issue order, so ``s_waitcnt vmcnt(n)`` guarantees
that everything but the last ``n`` issued operations has landed.  The kernel issues the first
``S - 1`` chunks' DMAs, then (with a tanh input) its epilogue's x loads, then one chunk per ring
step, and before chunk ``c`` is read it waits with an allowance computed in closed form.  The model
issues the same sequence and counts the operations issued after chunk ``c``'s last DMA: the
allowance must equal that count (smaller waits longer than needed, larger reads a stage that may
not have landed).  A planted mistake, the x loads allowed for every chunk rather than only the chunks
issued before them, is caught.
"""

from __future__ import annotations

import pytest

STAGES = 4  # kDzStages
NT = 2      # 16-row tiles per wave


def shapes():
    """(DT, weight DMAs per wave per chunk, x loads per thread) of the kernel's instantiations:
    HT = 16 DT hidden columns, kInstr = DT slab DMAs over 4 waves, 4 x 32 rows x HT / 8 units
    over 256 threads."""
    for dt in (8, 12):
        yield dt, dt // 4, 4 * 16 * NT * (16 * dt // 8) // 256


def allowance(c, nc, per_chunk, x_loads, planted=False):
    """The kernel's ring_step allowance for chunk c of nc."""
    after = min(nc - 1 - c, STAGES - 2)
    extra = x_loads if (planted or c < STAGES - 1) else 0
    return after * per_chunk + extra


def queue_mismatches(nc, npw, nvt, x_loads, planted=False):
    per_chunk = npw + nvt
    issued = []
    for c in range(min(STAGES - 1, nc)):
        issued += [("chunk", c)] * per_chunk
    issued += [("x", None)] * x_loads
    bad = []
    for c in range(nc):
        last = max(i for i, op in enumerate(issued) if op == ("chunk", c))
        after_last = len(issued) - 1 - last
        allow = allowance(c, nc, per_chunk, x_loads, planted)
        if allow != after_last:
            bad.append((c, allow, after_last))
        if c + STAGES - 1 < nc:
            issued += [("chunk", c + STAGES - 1)] * per_chunk
    return bad


@pytest.mark.parametrize("tanh", [False, True])
def test_ring_wait_allowances_match_the_issue_order(tanh):
    for dt, npw, xl in shapes():
        x_loads = xl if tanh else 0
        # the template bound of ring_vm_wait: (S - 2) (kMaxPW + NT) + kXLoads
        bound = (STAGES - 2) * ((dt + 3) // 4 + NT) + x_loads
        for nc in range(1, 40):
            for nvt in range(NT + 1):
                assert not queue_mismatches(nc, npw, nvt, x_loads), (dt, nc, nvt)
                assert max(allowance(c, nc, npw + nvt, x_loads) for c in range(nc)) <= bound


def test_planted_allowance_mistake_is_caught():
    dt, npw, xl = next(iter(shapes()))
    assert queue_mismatches(6, npw, NT, xl, planted=True)
    assert not queue_mismatches(6, npw, NT, xl)

"""The tanh table of the one-pass mask-MLP forward (``mask_mlp.hip``).

The hidden layer rounds z to the storage dtype before the tanh (fr.py:338-340), so the kernel reads
tanh from a table of every non-negative 16-bit pattern (sign restored after the lookup).  These
tests check that table, as the library builds it on the host, against an independent computation:
float64 tanh rounded once to bf16 (by comparing the two neighbouring patterns) or to fp16 (numpy's
float64 -> float16 conversion).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch


def _bf16_rne(t):
    """Nearest bf16 pattern to float64 ``t`` >= 0 (ties to even), by comparing the two neighbours."""
    f = np.float32(t)
    bits = int(np.array(f, dtype=np.float32).view(np.uint32))
    if np.float64(f) > t:  # the float32 rounding went up: step back to a float32 <= t
        bits -= 1
    lo = bits >> 16
    lo_v = float(np.array(lo << 16, dtype=np.uint32).view(np.float32))
    hi_v = float(np.array((lo + 1) << 16, dtype=np.uint32).view(np.float32))
    d_lo, d_hi = t - lo_v, hi_v - t
    if d_lo < d_hi or (d_lo == d_hi and lo % 2 == 0):
        return lo
    return lo + 1


def _reference_table(dtype):
    """float64 tanh of every non-negative pattern, rounded once; NaN patterns map to -1 (any NaN)."""
    pats = np.arange(32768, dtype=np.uint16)
    vals = torch.from_numpy(pats.view(np.int16)).view(dtype).double().numpy()
    ref = np.empty(32768, dtype=np.int64)
    for b, v in enumerate(vals):
        t = np.tanh(v)
        if np.isnan(t):
            ref[b] = -1
        elif dtype == torch.float16:
            ref[b] = int(np.array(np.float16(t)).view(np.uint16))  # numpy rounds float64 -> float16 once
        else:
            ref[b] = _bf16_rne(float(t))
    return ref


def _matches(table, ref, dtype):
    nan = torch.from_numpy(table.view(np.int16)).view(dtype).isnan().numpy()
    return bool(np.all(np.where(ref < 0, nan, table.astype(np.int64) == ref)))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_library_tanh_table_is_correctly_rounded(dtype):
    """The table ``mask_mlp.hip`` loads into LDS: for every non-negative 16-bit pattern, the tanh
    rounded once to the dtype (NaN patterns give a NaN)."""
    import ctypes

    from pymsst_amd._lib import PMSST_BF16, PMSST_F16, load_library

    lib = load_library()
    out = (ctypes.c_uint16 * 32768)()
    assert lib.pmsst_mask_mlp_tanh_table(PMSST_BF16 if dtype == torch.bfloat16 else PMSST_F16, out, 32768) == 0
    table = np.frombuffer(out, dtype=np.uint16).copy()
    assert _matches(table, _reference_table(dtype), dtype)
    one = torch.tensor([1.0], dtype=dtype).view(torch.int16).item() & 0xFFFF
    inf = torch.tensor([float("inf")], dtype=dtype).view(torch.int16).item() & 0xFFFF
    assert table[inf] == one and table[0] == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_planted_truncation_is_caught(dtype):
    """A table rounded toward zero (float32 tanh, then truncated) fails the same comparison."""
    pats = np.arange(32768, dtype=np.uint16)
    vals = torch.from_numpy(pats.view(np.int16)).view(dtype).float()
    t = torch.tanh(vals).numpy()
    if dtype == torch.bfloat16:
        trunc = (t.view(np.uint32) >> 16).astype(np.uint16)
    else:
        trunc = np.array([np.float16(x) if np.isnan(x) else np.float16(np.float32(x)) for x in t])
        trunc = np.where(np.abs(trunc.astype(np.float64)) > np.abs(t), np.nextafter(trunc, np.float16(0)), trunc)
        trunc = trunc.astype(np.float16).view(np.uint16)
    assert not _matches(trunc, _reference_table(dtype), dtype)

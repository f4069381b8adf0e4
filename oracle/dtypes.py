"""Storage-dtype rounding for the oracle (test infrastructure only).

The reference kernels accumulate in fp32 and round every stored tensor to its
storage dtype (``static_cast<scalar_t>``, e.g. fused_band_split.cu:58,69).
The oracle computes in float64 and applies the same final rounding with
these helpers.  bf16 rounding is round-to-nearest-even on the fp32 bit
pattern, which is what ``static_cast<at::BFloat16>(float)`` does.
"""

from __future__ import annotations

import numpy as np

DTYPES = ("f32", "f16", "bf16")


def _bf16_round_f32(a32: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(a32, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(a32)
    bias = np.uint64(0x7FFF) + ((u >> np.uint64(16)) & np.uint64(1))
    r = ((u + bias) & np.uint64(0xFFFF0000)).astype(np.uint32)
    out = r.view(np.float32).copy()
    out[nan] = np.nan
    return out


def round_to(a, dtype: str) -> np.ndarray:
    """Round ``a`` to storage dtype ``dtype`` and return it as float64."""
    a = np.asarray(a, dtype=np.float64)
    if dtype == "f64":
        return a.copy()
    a32 = a.astype(np.float32)
    if dtype == "f32":
        return a32.astype(np.float64)
    if dtype == "f16":
        return a32.astype(np.float16).astype(np.float64)
    if dtype == "bf16":
        return _bf16_round_f32(a32).astype(np.float64)
    raise ValueError(f"unknown dtype {dtype!r}")


def to_f64(a) -> np.ndarray:
    """Exact float64 copy of an array (torch tensors are moved to CPU first)."""
    if hasattr(a, "detach"):
        a = a.detach().to("cpu")
        import torch

        if a.dtype in (torch.bfloat16, torch.float16):
            a = a.float()
        a = a.double().numpy()
    return np.asarray(a, dtype=np.float64)

"""Shared pytest configuration.

``gpu``-marked tests need a HIP GPU and the built ``libpymsst_amd.so``; the
driver runs them on an MI355X with ``-m gpu`` and everything else on the CPU
with ``-m "not gpu"``.

Parity bars used throughout (stated here once, applied by ``assert_parity``):

* fp32 outputs: ``max|a - ref| <= 1e-5 * max(1, max|ref|)`` -- the 1e-5
  max-abs bar for O(1) outputs, scaled for row reductions whose values grow
  with the row count (dgamma, dW, dbias).
* bf16 / fp16 outputs: ``max|a - ref| <= 2e-2 * max|ref|`` (2e-2 relative).

``ref`` is the float64 oracle in ``oracle/`` rounded to the output's storage
dtype.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

FP32_TOL = 1e-5
LOWP_TOL = 2e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built libpymsst_amd.so")


def to_np(t) -> np.ndarray:
    import torch

    if isinstance(t, torch.Tensor):
        t = t.detach().to("cpu")
        if t.dtype in (torch.bfloat16, torch.float16):
            t = t.float()
        return t.double().numpy()
    return np.asarray(t, dtype=np.float64)


def dt_name(dtype) -> str:
    import torch

    return {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}[dtype]


def parity_error(actual, ref, dtype_name: str) -> tuple[float, float]:
    """Return ``(err, bound)`` for the parity bar of ``dtype_name``."""
    a = to_np(actual)
    r = to_np(ref)
    assert a.shape == r.shape, f"shape {a.shape} != {r.shape}"
    err = float(np.max(np.abs(a - r))) if a.size else 0.0
    scale = float(np.max(np.abs(r))) if r.size else 0.0
    if dtype_name == "f32":
        bound = FP32_TOL * max(1.0, scale)
    else:
        bound = LOWP_TOL * max(scale, 1e-30)
    return err, bound


def assert_parity(actual, ref, dtype_name: str, what: str = "") -> None:
    a = to_np(actual)
    assert np.all(np.isfinite(a)), f"{what}: non-finite values"
    err, bound = parity_error(actual, ref, dtype_name)
    assert err <= bound, f"{what}: max abs err {err:.3e} > bound {bound:.3e} ({dtype_name})"


@pytest.fixture(scope="session")
def hip_ext():
    """The HIP extension object; GPU tests fail (not skip) if the library is missing on a GPU box."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP GPU in this environment")
    from pymsst_amd.fused_extension import load_fused_band_split_extension

    return load_fused_band_split_extension()


@pytest.fixture(autouse=True)
def _announce(request):
    # Name the running case on stderr before any GPU work so a fault names its test.
    if request.node.get_closest_marker("gpu") is not None:
        sys.stderr.write(f"\n[gpu-case] {request.node.nodeid}\n")
        sys.stderr.flush()
    yield


os.environ.setdefault("PYTHONHASHSEED", "0")

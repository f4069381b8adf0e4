"""Shared pytest configuration.

``gpu``-marked tests need a HIP GPU and the built ``libpymsst_amd.so``; the
driver runs them on an MI355X with ``-m gpu`` and everything else on the CPU
with ``-m "not gpu"``.

Parity bars used throughout (stated here once, applied by ``assert_parity``):

* fp32 outputs: ``max|a - ref| <= 1e-5 * max(1, max|ref|)`` -- the 1e-5
  max-abs bar for O(1) outputs, scaled for row reductions whose values grow
  with the row count (dgamma, dW, dbias).
* bf16 / fp16 outputs, per element: ``|a - ref| <= 2e-2 * (|ref| + rms_g(ref))`` --
  2e-2 relative, with a floor for elements near zero of 2e-2 times the RMS of the
  element's group (its band, for ragged per-band outputs; the whole tensor
  otherwise).  Near zero the error is set by the 16-bit rounding of the terms
  summed into the element (e.g. the bf16 MFMA operands), which scales with the
  group's magnitude, not with the element's.

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
LOWP_FLOOR = 2e-2  # absolute floor of the 16-bit bar, as a fraction of the group's rms(ref)


# fp32 checks whose bar was scaled above the flat 1e-5 (reference values larger than 1), and the
# model-level figures the tests report (loss-curve statistics, relative errors), printed at the end
# of the session
F32_SCALED: list = []
REPORTS: list = []


def _session_lists(name: str) -> list:
    """The list ``name`` of this module and of its other instance: pytest imports this file as
    ``conftest`` while the test modules import ``tests.conftest``."""
    out, seen = [], set()
    for mod in (sys.modules.get(__name__), sys.modules.get("conftest"), sys.modules.get("tests.conftest")):
        lst = getattr(mod, name, None)
        if lst is not None and id(lst) not in seen:
            seen.add(id(lst))
            out += lst
    return out


def pytest_terminal_summary(terminalreporter):
    scaled = _session_lists("F32_SCALED")
    if scaled:
        worst = sorted(scaled, key=lambda v: -v[1])[:5]
        terminalreporter.write_line(
            f"fp32 parity bars scaled by max(1, max|ref|): {len(scaled)} checks, largest scales: "
            + ", ".join(f"{w or '?'} x{sc:.3g}" for w, sc in worst))
    for tag, text in _session_lists("REPORTS"):
        terminalreporter.write_line(f"[model-parity] {tag}: {text}")


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


def by_band(axis: int, sizes) -> tuple:
    """Groups of a ragged per-band output: consecutive segments of ``sizes`` along ``axis``."""
    return ("sizes", axis, tuple(int(v) for v in sizes))


def by_index(axis: int) -> tuple:
    """Groups of a per-band output whose band is an axis of its own (e.g. ``[M, NB, O]``)."""
    return ("axis", axis)


def _group_rms(r: np.ndarray, groups) -> np.ndarray:
    """RMS of each element's group, broadcastable to ``r``."""
    if groups is None:
        return np.asarray(np.sqrt(np.mean(r * r)))
    if groups[0] == "axis":
        ax = groups[1] % r.ndim
        other = tuple(i for i in range(r.ndim) if i != ax)
        return np.sqrt(np.mean(r * r, axis=other, keepdims=True))
    ax, sizes = groups[1] % r.ndim, groups[2]
    assert sum(sizes) == r.shape[ax], f"group sizes {sum(sizes)} != axis length {r.shape[ax]}"
    segs = np.split(r, np.cumsum(sizes)[:-1], axis=ax)
    other = tuple(i for i in range(r.ndim) if i != ax)
    rms = np.array([np.sqrt(np.mean(seg * seg)) for seg in segs])
    shape = [1] * r.ndim
    shape[ax] = r.shape[ax]
    del other
    return np.repeat(rms, sizes).reshape(shape)


def _lowp_bound(r: np.ndarray, groups) -> np.ndarray:
    return LOWP_TOL * np.abs(r) + np.maximum(LOWP_FLOOR * _group_rms(r, groups), 1e-30)


def parity_error(actual, ref, dtype_name: str, groups=None) -> tuple[float, float]:
    """Return ``(err, bound)`` for the parity bar of ``dtype_name``: for fp32 the max-abs error and
    its bound; for 16-bit dtypes the worst per-element ``|a - ref| / bound_i`` and 1.0."""
    a = to_np(actual)
    r = to_np(ref)
    assert a.shape == r.shape, f"shape {a.shape} != {r.shape}"
    if not a.size:
        return 0.0, 1.0
    diff = np.abs(a - r)
    if dtype_name == "f32":
        return float(np.max(diff)), FP32_TOL * max(1.0, float(np.max(np.abs(r))))
    return float(np.max(diff / _lowp_bound(r, groups))), 1.0


def assert_parity(actual, ref, dtype_name: str, what: str = "", groups=None) -> None:
    """``groups``: :func:`by_band` / :func:`by_index` for per-band outputs (the 16-bit floor is then
    taken per band)."""
    a = to_np(actual)
    assert np.all(np.isfinite(a)), f"{what}: non-finite values"
    err, bound = parity_error(actual, ref, dtype_name, groups)
    if dtype_name == "f32":
        scale = bound / FP32_TOL
        if scale > 1.0:
            F32_SCALED.append((what, scale))
        assert err <= bound, (f"{what}: max abs err {err:.3e} > bound {bound:.3e} = 1e-5 x max(1, max|ref|) with "
                              f"max|ref| = {float(np.max(np.abs(to_np(ref)))):.3e} (scale {scale:.3e}, {dtype_name})")
    else:
        r = to_np(ref)
        i = int(np.argmax(np.abs(a - r) / _lowp_bound(r, groups)))
        assert err <= bound, (f"{what}: element {np.unravel_index(i, r.shape)} = {a.flat[i]:.6g} vs {r.flat[i]:.6g} "
                              f"exceeds 2e-2 * (|ref| + rms_group(ref)) by {err:.2f}x ({dtype_name})")


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

"""CPU checks of the C ABI: the library loads, exports every symbol the header declares,
and validates arguments before touching a device (no GPU needed)."""

from __future__ import annotations

import ctypes
import re

import pytest

from pymsst_amd import _lib


def _header_names():
    text = re.sub(r"/\*.*?\*/", "", _lib.HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pmsst_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    try:
        return _lib.load_library()
    except _lib.FusedKernelUnavailable as exc:
        pytest.fail(f"libpymsst_amd.so is not built: {exc}")


def test_every_declared_symbol_is_exported(lib):
    names = _header_names()
    assert len(names) >= 15
    for name in names:
        assert hasattr(lib, name), name
    parsed = _lib.parse_header()
    assert sorted(parsed) == names


def test_abi_version_and_error_string(lib):
    assert lib.pmsst_abi_version() == 6
    assert isinstance(_lib.last_error(), str)


def test_workspace_queries(lib):
    assert lib.pmsst_rms_norm_backward_workspace_size(1000, 192) == 1024 * 192 * 4
    # [dgamma partials of 17 row tiles | dot partials, pitch F / 64 + NB + 1 | fp32 gs * gamma]
    dg = -(-17 * 4100 * 4 // 256) * 256
    dots = -(-1032 * (4100 // 64 + 62 + 1) * 4 // 256) * 256
    t = -(-1032 * 4100 * 4 // 256) * 256
    assert lib.pmsst_band_split_ragged_backward_workspace_size(1032, 4100, 62, 192) == dg + dots + t
    assert lib.pmsst_band_split_ragged_backward_workspace_size(0, 4100, 62, 192) == 0
    assert lib.pmsst_mask_estimator_final_backward_workspace_size(1032, 4100, 2) == -(-1032 * 8200 * 2 // 256) * 256
    assert lib.pmsst_mask_estimator_final_backward_workspace_size(0, 4100, 2) == 0
    assert lib.pmsst_grouped_linear_backward_workspace_size(1032, 62, 768) == 0
    # [g = T(dy W), 16-bit [M, F] | dots [M, NB] fp32 | dgamma partials of every 16 rows]
    g = -(-1032 * 4100 * 2 // 256) * 256
    dots = -(-1032 * 62 * 4 // 256) * 256
    parts = -(-65 * 4100 * 4 // 256) * 256
    assert lib.pmsst_band_split_mixed_backward_workspace_size(1032, 4100, 62) == g + dots + parts
    assert lib.pmsst_band_split_mixed_backward_workspace_size(0, 4100, 62) == 0


def test_argument_errors_need_no_device(lib):
    # null pointers / bad dtypes are rejected before any HIP call
    rc = lib.pmsst_rms_norm_forward(None, None, None, None, None, 4, 8, 0, None)
    assert rc == -1 and "null pointer" in _lib.last_error()
    rc = lib.pmsst_rms_norm_forward(None, None, None, None, None, 4, 8, 7, None)
    assert rc == -2 and "unsupported dtype" in _lib.last_error()
    dims = (ctypes.c_int64 * 2)(8, -1)
    rc = lib.pmsst_band_split_ragged_forward(None, 8, None, None, None, None, dims, 2, 4, 64, None, None, None, 2,
                                             None)
    assert rc == -1 and "dim_inputs must be positive" in _lib.last_error()


def test_dtype_codes():
    import torch

    assert _lib.dtype_code(torch.float32) == 0
    assert _lib.dtype_code(torch.float16) == 1
    assert _lib.dtype_code(torch.bfloat16) == 2
    with pytest.raises(_lib.PmsstError):
        _lib.dtype_code(torch.float64)

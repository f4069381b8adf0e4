"""GPU: the allocation-free RMSNorm backward (``pmsst_rms_norm_backward_from_input_noalloc``, dgamma
partials in a static device array) gives the same bits as the workspace entry point
``pmsst_rms_norm_backward_from_input`` it wraps, on two calls in a row (the second smaller, so it
runs over the partial rows the first call left behind), both called through the C ABI; a dim past
the array's capacity is refused before any launch."""

from __future__ import annotations

import ctypes

import pytest
import torch

from pymsst_amd import _lib

pytestmark = pytest.mark.gpu


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _case(lib, rows, dim, dtype, gamma_fp32, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, dim, generator=g).to(dtype).cuda()
    dy = torch.randn(rows, dim, generator=g).to(dtype).cuda()
    gamma = (1 + 0.1 * torch.randn(dim, generator=g)).to(torch.float32 if gamma_fp32 else dtype).cuda()
    inv = (1.0 / x.float().norm(dim=-1).clamp_min(1e-12)).contiguous()
    code = _lib.dtype_code(dtype)
    gcode = _lib.dtype_code(gamma.dtype)
    outs = []
    for noalloc in (False, True):
        dx = torch.empty_like(x)
        dg = torch.empty_like(gamma)
        if noalloc:
            rc = lib.pmsst_rms_norm_backward_from_input_noalloc(
                _ptr(dy), _ptr(x), _ptr(inv), _ptr(gamma), _ptr(dx), _ptr(dg), rows, dim, code, gcode, _stream())
        else:
            ws = torch.empty(lib.pmsst_rms_norm_backward_workspace_size(rows, dim), dtype=torch.uint8, device="cuda")
            rc = lib.pmsst_rms_norm_backward_from_input(
                _ptr(dy), _ptr(x), _ptr(inv), _ptr(gamma), _ptr(dx), _ptr(dg), rows, dim, code, gcode, _ptr(ws),
                ws.numel(), _stream())
        assert rc == 0, _lib.last_error()
        torch.cuda.synchronize()
        outs.append((dx, dg))
    (dx_ref, dg_ref), (dx, dg) = outs
    assert torch.equal(dx, dx_ref)
    assert torch.equal(dg, dg_ref)
    assert torch.isfinite(dg).all()


def test_noalloc_matches_workspace_entry_point_twice(hip_ext):
    lib = _lib.load_library()
    # first call: 117,552 rows x 512, all 1024 partial rows in use; second call: fewer
    # rows and columns, over the first call's leftovers
    _case(lib, 1896 * 62, 512, torch.bfloat16, True, 1)
    _case(lib, 1000, 192, torch.bfloat16, False, 2)
    _case(lib, 77, 1024, torch.float32, True, 3)


def test_noalloc_rejects_dims_past_the_scratch(hip_ext):
    lib = _lib.load_library()
    x = torch.zeros(4, 2048, device="cuda")
    inv = torch.ones(4, device="cuda")
    rc = lib.pmsst_rms_norm_backward_from_input_noalloc(_ptr(x), _ptr(x), _ptr(inv), _ptr(x), _ptr(x), _ptr(x), 4,
                                                        2048, 0, 0, _stream())
    assert rc == -1 and "outside [1, 1024]" in _lib.last_error()

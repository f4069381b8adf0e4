"""GPU parity: mask estimator final layer (per-band Linear + bias + GLU) and grouped linear.

Cases: the reference's direct-mode test (tests/test_training_smoke.py:574-615:
seed 11, M=4, NB=5, hidden 16, widths (3,4,2,5,6)); the BS-RoFormer 62-band
layout at cfg1 (hidden 256) and cfg2 (M=1032, hidden 768); mel-style widths;
grouped linear (the mask MLP's hidden layer, O=768) on strided views.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_parity, dt_name, to_np

pytestmark = pytest.mark.gpu

BSR_WIDTHS = tuple([8] * 24 + [16] * 12 + [48] * 8 + [96] * 8 + [192] * 8 + [512, 516])


def _offsets(dim_inputs):
    return torch.tensor(np.concatenate([[0], np.cumsum(dim_inputs)]), dtype=torch.long, device="cuda")


def _check(ext, dim_inputs, m, hidden, dtype, seed, direct=True):
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(seed)
    nb = len(dim_inputs)
    x = torch.randn(m, nb, hidden, generator=g).to(dtype).cuda()
    weights = [(torch.randn(2 * d, hidden, generator=g) / hidden**0.5).to(dtype).cuda() for d in dim_inputs]
    bias = (0.1 * torch.randn(2 * sum(dim_inputs), generator=g)).to(dtype).cuda()
    offs = _offsets(dim_inputs)
    fwd = ext.mask_estimator_final_direct_forward if direct else ext.mask_estimator_final_forward
    bwd = ext.mask_estimator_final_direct_backward if direct else ext.mask_estimator_final_backward
    out, pre, x_saved = fwd(x, weights, bias, list(dim_inputs), offs)
    npw = [to_np(w) for w in weights]
    r_out, r_pre = oracle.mask_estimator_final_forward(to_np(x), npw, to_np(bias), dim_inputs, dn)
    assert_parity(out, r_out, dn, "out")
    assert_parity(pre, r_pre, dn, "pre")
    gout = torch.randn(out.shape, generator=g).to(dtype).cuda()
    res = bwd(gout, x_saved, pre, weights, list(dim_inputs), offs)
    r_dx, r_db, r_dw = oracle.mask_estimator_final_backward(to_np(gout), to_np(x), to_np(pre), npw, dim_inputs, dn)
    assert_parity(res[0], r_dx, dn, "dx")
    assert_parity(res[1], r_db, dn, "dbias")
    for b in range(nb):
        assert res[2 + b].shape == (2 * dim_inputs[b], hidden)
    assert_parity(torch.cat([w.reshape(-1) for w in res[2:]]), np.concatenate([w.reshape(-1) for w in r_dw]), dn,
                  "dW")


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("direct", [True, False])
def test_reference_direct_case(hip_ext, dtype, direct):
    _check(hip_ext, (3, 4, 2, 5, 6), 4, 16, dtype, 11, direct)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bsr_cfg1(hip_ext, dtype):
    _check(hip_ext, BSR_WIDTHS, 130, 256, dtype, 2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bsr_cfg2(hip_ext, dtype):
    _check(hip_ext, BSR_WIDTHS, 1032, 768, dtype, 3)


def test_mel_style_widths(hip_ext):
    r = np.random.default_rng(5)
    widths = tuple(int(4 * w) for w in r.integers(6, 131, size=12))
    _check(hip_ext, widths, 77, 100, torch.bfloat16, 6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("has_bias", [True, False])
def test_grouped_linear(hip_ext, dtype, has_bias):
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(9)
    full = torch.randn(3, 43, 62, 200, generator=g).to(dtype).cuda()
    x = full[..., :192].reshape(129, 62, 192)
    w = (torch.randn(62, 768, 192, generator=g) / 192**0.5).to(dtype).cuda()
    b = (0.1 * torch.randn(62, 768, generator=g)).to(dtype).cuda() if has_bias else None
    out = hip_ext.grouped_linear_forward(x, w, b)
    ref = oracle.grouped_linear_forward(to_np(x), to_np(w), to_np(b) if has_bias else None, dn)
    assert_parity(out, ref, dn, "grouped linear")
    # strided view without a copy: the band-split group pattern
    xv = full[..., :192]
    assert not xv.is_contiguous()
    out2 = hip_ext.grouped_linear_forward(xv.reshape(129, 62, 192), w, b)
    assert torch.equal(out2, out)


def test_empty_rows(hip_ext):
    dims = (4, 8)
    x = torch.empty(0, 2, 32, device="cuda")
    weights = [torch.randn(2 * d, 32, device="cuda") for d in dims]
    bias = torch.randn(24, device="cuda")
    out, pre, xs = hip_ext.mask_estimator_final_forward(x, weights, bias, list(dims), _offsets(dims))
    assert out.shape == (0, 12) and pre.shape == (0, 24)
    res = hip_ext.mask_estimator_final_backward(out, xs, pre, weights, list(dims), _offsets(dims))
    assert res[0].shape == (0, 2, 32)
    assert all(torch.count_nonzero(t).item() == 0 for t in res[1:])

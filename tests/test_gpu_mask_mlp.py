"""GPU parity: the one-pass depth-2 mask MLP forward (``pmsst_mask_mlp_forward``) against the oracle.

``oracle.mask_mlp_forward`` / ``oracle.mask_mlp_hidden`` restate the reference's grouped MLP
(fr.py:332-369: grouped Linear, ``inference_tanh``, final Linear + GLU) with its rounding points.
Cases: the BS-RoFormer 62-band layout at configs[0] (dim 64, hidden 256), configs[1] (M=1032, dim
192, hidden 768) in bf16 and fp16, configs[4]'s dim 512 / hidden 2048 on a row sample, the 60-band
mel layout on a row sample, and a small ragged layout with a partial row tile and bands that end
inside a 16-output group.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_parity, by_band, by_index, dt_name, to_np

pytestmark = pytest.mark.gpu

BSR_WIDTHS = tuple([8] * 24 + [16] * 12 + [48] * 8 + [96] * 8 + [192] * 8 + [512, 516])


def _mel_widths():
    from pymsst_amd.core.mel_band_roformer import mel_band_bins

    return tuple(4 * len(b) for b in mel_band_bins(44100, 2048, 60))


def _inputs(dims, m, dim, hidden, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    nb = len(dims)
    x = torch.randn(m, nb, dim, generator=g).to(dtype).cuda()
    w1 = (torch.randn(nb, hidden, dim, generator=g) / dim**0.5).to(dtype).cuda()
    b1 = (0.1 * torch.randn(nb, hidden, generator=g)).to(dtype).cuda()
    w2s = [(torch.randn(2 * d, hidden, generator=g) / hidden**0.5).to(dtype) for d in dims]
    w2 = torch.cat([w.reshape(-1) for w in w2s]).cuda()
    b2 = (0.1 * torch.randn(2 * sum(dims), generator=g)).to(dtype).cuda()
    return x, w1, b1, w2, w2s, b2


CASES = [
    pytest.param(BSR_WIDTHS, 1032, 192, 768, torch.bfloat16, id="configs1-bf16"),
    pytest.param(BSR_WIDTHS, 1032, 192, 768, torch.float16, id="configs1-fp16"),
    pytest.param(BSR_WIDTHS, 130, 64, 256, torch.bfloat16, id="configs0-bf16"),
    pytest.param(BSR_WIDTHS, 300, 512, 2048, torch.bfloat16, id="configs4-dims-bf16"),
    pytest.param("mel", 700, 192, 768, torch.bfloat16, id="mel60-bf16"),
    pytest.param((4, 8, 12, 400, 64, 128, 4), 77, 128, 96, torch.float16, id="ragged-fp16"),
]


@pytest.mark.parametrize("dims,m,dim,hidden,dtype", CASES)
def test_mask_mlp_forward_vs_oracle(hip_ext, dims, m, dim, hidden, dtype):
    dims = _mel_widths() if dims == "mel" else dims
    dn = dt_name(dtype)
    print(f"mask_mlp_forward dims={len(dims)} bands m={m} dim={dim} hidden={hidden} {dn}", flush=True)
    assert hip_ext.mask_mlp_supported(dim, hidden, dims, dtype)
    x, w1, b1, w2, w2s, b2 = _inputs(dims, m, dim, hidden, dtype, seed=31)
    out, pre, hid = hip_ext.mask_mlp_forward(x, w1, b1, w2, b2, dims, save_hidden=True)
    torch.cuda.synchronize()
    xn, w1n, b1n = to_np(x), to_np(w1), to_np(b1)
    r_h = oracle.mask_mlp_hidden(xn, w1n, b1n, dn)
    assert_parity(hid, r_h, dn, "hidden", by_index(1))
    r_out, r_pre = oracle.mask_estimator_final_forward(r_h, [to_np(w) for w in w2s], to_np(b2), dims, dn)
    assert_parity(pre, r_pre, dn, "pre", by_band(1, [2 * d for d in dims]))
    assert_parity(out, r_out, dn, "out", by_band(1, dims))
    # without the hidden output the kernel computes the same values
    out2, pre2, none = hip_ext.mask_mlp_forward(x, w1, b1, w2, b2, dims, save_hidden=False)
    assert none is None
    assert torch.equal(out2, out) and torch.equal(pre2, pre)


def test_mask_mlp_forward_matches_two_kernel_path(hip_ext):
    """The hidden layer equals the grouped-linear tanh kernel's output except where the two
    accumulation orders round z to different neighbours (rare, at most 2 ulps of h)."""
    dims, m, dim, hidden, dtype = BSR_WIDTHS, 1032, 192, 768, torch.bfloat16
    x, w1, b1, w2, _, b2 = _inputs(dims, m, dim, hidden, dtype, seed=5)
    _, _, hid = hip_ext.mask_mlp_forward(x, w1, b1, w2, b2, dims, save_hidden=True)
    h2 = hip_ext.grouped_linear_forward_act(x, w1, b1, activation="tanh")
    diff = (hid.float() - h2.float()).abs()
    assert (diff <= h2.float().abs() * 2.0**-6 + 1e-6).all()
    assert (diff > 0).float().mean().item() < 1e-3


@pytest.mark.parametrize("m,groups,i,o,dtype", [
    (1032, 62, 192, 768, torch.bfloat16),
    (77, 5, 128, 96, torch.float16),
    (300, 7, 256, 64, torch.bfloat16),
    (1, 3, 192, 768, torch.bfloat16),
    (257, 9, 64, 256, torch.float16),
])
def test_grouped_dx_register_kernel_vs_oracle(hip_ext, m, groups, i, o, dtype):
    """The grouped linear's input gradient on glin_dx_kernel (16-bit, in_features 64-256): full and
    partial row tiles, a single row, and the mask MLP's configs[1] hidden layer."""
    dn = dt_name(dtype)
    print(f"grouped dx m={m} groups={groups} i={i} o={o} {dn}", flush=True)
    g = torch.Generator().manual_seed(41)
    x = torch.randn(m, groups, i, generator=g).to(dtype).cuda()
    w = (torch.randn(groups, o, i, generator=g) / o**0.5).to(dtype).cuda()
    dy = torch.randn(m, groups, o, generator=g).to(dtype).cuda()
    dx, dw, db = hip_ext.grouped_linear_backward(dy, x, w, True)
    rdx, rdw, rdb = oracle.grouped_linear_backward(to_np(dy), to_np(x), to_np(w), True, dn)
    assert_parity(dx, rdx, dn, "dx", by_index(1))
    assert_parity(dw, rdw, dn, "dW", by_index(0))
    assert_parity(db, rdb, dn, "db", by_index(0))

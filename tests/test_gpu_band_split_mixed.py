"""GPU parity: the band split of an fp32 input with a 16-bit projection (the fused band split under
autocast, where the input is the fp32 STFT: fr.py:827-857 runs the reference kernels in x's dtype).

Forward and backward through the C ABI against ``oracle.band_split_mixed_*`` at the configs[2]
(62 bands, M = 1032, dim 192), configs[4] (M = 1896, dim 512) and configs[3] (60 mel bands,
M = 2760) shapes, the reference's odd ragged widths (scalar paths), a row pitch wider than F and an
empty batch.  ``inv_norm`` is fp32 arithmetic and meets the fp32 bar; the other outputs pass through
a 16-bit rounding (the projection's input u, the Linear's input gradient g), so a 1-ulp difference
there moves them by 2^-8 relative: they meet the 16-bit bar, per band.
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


def _case(ext, dims, m, o, dtype, seed, pitch_extra=0):
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(seed)
    f = sum(dims)
    # STFT-like magnitudes: Laplace(0, 0.05) with a few loud low bins
    lap = torch.distributions.Laplace(0.0, 0.05)
    torch.manual_seed(seed)
    xfull = lap.sample((m, f + pitch_extra))
    xfull[:, :64] *= 20.0
    if m > 1:
        xfull[1, : dims[0]] = 0.0  # a zero band row
    xfull = xfull.cuda()
    x = xfull[:, :f]
    gamma = (1 + 0.1 * torch.randn(f, generator=g)).cuda()
    w = torch.cat([(torch.randn(o, d, generator=g) / d**0.5).reshape(-1) for d in dims]).to(dtype).cuda()
    b = (0.1 * torch.randn(len(dims) * o, generator=g)).to(dtype).cuda()
    out, feats, inv = ext.band_split_mixed_forward(x, gamma, w, b, dims, dtype)
    off = np.concatenate([[0], np.cumsum(dims)])
    npg = [to_np(gamma)[off[k]:off[k + 1]] for k in range(len(dims))]
    npw = [to_np(w)[o * off[k]:o * off[k + 1]].reshape(o, dims[k]) for k in range(len(dims))]
    npb = [to_np(b)[o * k:o * (k + 1)] for k in range(len(dims))]
    r_out, r_feats, r_inv = oracle.band_split_mixed_forward(to_np(x), npg, npw, npb, dims, dn)
    assert out.dtype == dtype and feats.dtype == dtype and inv.dtype == torch.float32
    assert_parity(inv, r_inv, "f32", "inv_norm")
    assert_parity(feats, r_feats, dn, "features", by_band(1, dims))
    assert_parity(out, r_out, dn, "out", by_index(1))
    dy = torch.randn(out.shape, generator=g).to(dtype).cuda()
    dx, dg, dw, db = ext.band_split_mixed_backward(dy, x, feats, inv, gamma, w, dims, True)
    assert dx.dtype == torch.float32 and dg.dtype == torch.float32 and dw.dtype == dtype and db.dtype == dtype
    r_dx, r_dg, r_dw, r_db = oracle.band_split_mixed_backward(to_np(dy), to_np(x), to_np(feats), to_np(inv), npg, npw,
                                                              dims, dn)
    assert_parity(dx, r_dx, dn, "dx", by_band(1, dims))
    assert_parity(dg, np.concatenate(r_dg), dn, "dgamma", by_band(0, dims))
    assert_parity(dw, np.concatenate([v.reshape(-1) for v in r_dw]), dn, "dW", by_band(0, [o * d for d in dims]))
    assert_parity(db.reshape(len(dims), o), np.stack(r_db), dn, "dbias", by_index(0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mixed_configs2(hip_ext, dtype):
    _case(hip_ext, BSR_WIDTHS, 1032, 192, dtype, 31)


def test_mixed_configs4(hip_ext):
    _case(hip_ext, BSR_WIDTHS, 1896, 512, torch.bfloat16, 32)


def test_mixed_mel_configs3(hip_ext):
    _case(hip_ext, _mel_widths(), 2760, 192, torch.bfloat16, 33)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mixed_odd_widths_and_pitch(hip_ext, dtype):
    # the reference's ragged widths (scalar loads), then 4-aligned widths read through a wider row pitch
    _case(hip_ext, (3, 5, 2, 7), 5, 4, dtype, 7)
    _case(hip_ext, (8, 64, 132, 4), 300, 64, dtype, 34, pitch_extra=12)


def test_mixed_empty_batch(hip_ext):
    dims = (8, 16)
    x = torch.empty(0, 24, device="cuda")
    gamma = torch.ones(24, device="cuda")
    w = torch.randn(4 * 24, device="cuda").bfloat16()
    b = torch.zeros(8, device="cuda").bfloat16()
    out, feats, inv = hip_ext.band_split_mixed_forward(x, gamma, w, b, dims, torch.bfloat16)
    assert out.shape == (0, 2, 4) and feats.shape == (0, 24)
    dx, dg, dw, db = hip_ext.band_split_mixed_backward(torch.empty(0, 2, 4, device="cuda").bfloat16(), x, feats, inv,
                                                       gamma, w, dims, True)
    torch.cuda.synchronize()
    assert dx.shape == (0, 24) and torch.all(dg == 0) and torch.all(dw == 0) and torch.all(db == 0)


def test_mixed_rejects_wrong_dtypes(hip_ext):
    x = torch.randn(4, 24, device="cuda")
    w = torch.randn(4 * 24, device="cuda").bfloat16()
    with pytest.raises(RuntimeError, match="float32"):
        hip_ext.band_split_mixed_forward(x.bfloat16(), torch.ones(24, device="cuda"), w, None, (8, 16), torch.bfloat16)
    with pytest.raises(RuntimeError, match="projection dtype"):
        hip_ext.band_split_mixed_forward(x, torch.ones(24, device="cuda"), w.float(), None, (8, 16), torch.float32)

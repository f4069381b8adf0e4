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
    # row tiles one wave shorter than the block (224 + 33 rows at dim 192, 96 + 44 at dim 512)
    pytest.param(BSR_WIDTHS, 257, 192, 768, torch.bfloat16, id="row-tile-224-bf16"),
    pytest.param(BSR_WIDTHS, 140, 512, 2048, torch.float16, id="row-tile-96-dim512-fp16"),
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
    (1100, 62, 192, 768, torch.bfloat16),  # 48-row waves, the last tile's third wave part-filled
    (1160, 62, 192, 768, torch.float16),   # 48-row waves, an 8-row last tile
    (77, 5, 128, 96, torch.float16),
    (300, 7, 256, 64, torch.bfloat16),
    (1, 3, 192, 768, torch.bfloat16),
    (257, 9, 64, 256, torch.float16),
])
def test_grouped_dx_register_kernel_vs_oracle(hip_ext, m, groups, i, o, dtype):
    """The grouped linear's input gradient on glin_dx_kernel (16-bit, in_features 64-256): full and
    partial row tiles, a single row, and the mask MLP's configs[1] hidden layer; at in_features 192
    both block forms (32-row waves at m = 1, 48-row waves at m >= 1032, chosen by the launcher)."""
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


APPLY_CASES = [
    # dims, batch, frames, dim, hidden, dtype, stems, stem, channels, zero_dc
    pytest.param(BSR_WIDTHS, 4, 258, 192, 768, torch.bfloat16, 4, 2, 2, False, id="configs1-bf16-stem2"),
    pytest.param(BSR_WIDTHS, 4, 258, 192, 768, torch.float16, 4, 0, 2, True, id="configs1-fp16-stem0-zdc"),
    pytest.param(BSR_WIDTHS, 2, 65, 64, 256, torch.bfloat16, 1, 0, 2, True, id="configs0-bf16-zdc"),
    pytest.param(BSR_WIDTHS, 1, 300, 512, 2048, torch.bfloat16, 1, 0, 2, False, id="configs4-dims-bf16"),
    pytest.param((4, 8, 12, 400, 64, 128, 4), 7, 11, 128, 96, torch.float16, 3, 1, 2, False, id="ragged-fp16"),
    pytest.param((4, 8, 12, 400, 64, 128, 4), 7, 11, 128, 96, torch.bfloat16, 2, 1, 1, True, id="ragged-mono-zdc"),
]


def _complex_product_bound(spec, mask_ri):
    """One-ulp-scale bound for re/im of ``spec * m`` computed in fp32 with or without fused
    multiply-adds: 2^-22 (|re s||re m| + |im s||im m|) per component, componentwise."""
    sr, si = spec.real.abs(), spec.imag.abs()
    mr, mi = mask_ri[..., 0].abs(), mask_ri[..., 1].abs()
    return torch.stack([sr * mr + si * mi, sr * mi + si * mr], dim=-1) * 2.0**-22


@pytest.mark.parametrize("dims,b,t,dim,hidden,dtype,stems,stem,channels,zero_dc", APPLY_CASES)
def test_mask_mlp_forward_apply_matches_mlp_then_apply(hip_ext, dims, b, t, dim, hidden, dtype, stems, stem,
                                                       channels, zero_dc):
    """The mask MLP with the mask product in its epilogue (``pmsst_mask_mlp_forward_apply``) writes
    stem ``stem`` of the iSTFT-layout estimate equal to ``mask_mlp_forward`` followed by
    ``mask_apply_forward`` (each pinned to the oracle above and in test_gpu_mask_apply.py), within
    one fp32 rounding of the complex product; pre and hidden are bit-identical to
    ``mask_mlp_forward``'s, and the other stems' slices of the estimate are not written."""
    dn = dt_name(dtype)
    m, total = b * t, sum(dims)
    fc = total // 2
    f = fc // channels
    print(f"mask_mlp_forward_apply bands={len(dims)} b={b} t={t} dim={dim} hidden={hidden} {dn} stems={stems} "
          f"stem={stem} channels={channels} zero_dc={zero_dc}", flush=True)
    x, w1, b1, w2, w2s, b2 = _inputs(dims, m, dim, hidden, dtype, seed=17 + stem)
    g = torch.Generator().manual_seed(23)
    spec = torch.complex(torch.randn(b, fc, t, generator=g), torch.randn(b, fc, t, generator=g)).cuda()
    sentinel = complex(7.0, -3.0)
    est = torch.full((b * stems * channels, f, t), sentinel, dtype=torch.complex64, device="cuda")
    pre, hid = hip_ext.mask_mlp_forward_apply(x, w1, b1, w2, b2, dims, spec, est, stem, channels, zero_dc,
                                              save_hidden=True)
    out_r, pre_r, hid_r = hip_ext.mask_mlp_forward(x, w1, b1, w2, b2, dims, save_hidden=True)
    torch.cuda.synchronize()
    assert torch.equal(pre, pre_r) and torch.equal(hid, hid_r)
    mask = torch.zeros(b, stems, t, total, dtype=dtype, device="cuda")
    mask[:, stem] = out_r.view(b, t, total)
    want = hip_ext.mask_apply_forward(spec, mask, channels, zero_dc).view(b, stems, channels, f, t)
    got = est.view(b, stems, channels, f, t)
    others = [s for s in range(stems) if s != stem]
    assert (got[:, others] == sentinel).all(), "stems other than `stem` were written"
    got_s, want_s = torch.view_as_real(got[:, stem]), torch.view_as_real(want[:, stem])
    # mask[b, t, (f*C + c)*2 + {0,1}] -> [b, c, f, t, 2], the estimate's layout
    m_ri = mask[:, stem].float().view(b, t, f, channels, 2).permute(0, 3, 2, 1, 4)
    s_l = spec.view(b, f, channels, t).permute(0, 2, 1, 3)
    bound = _complex_product_bound(s_l, m_ri)
    diff = (got_s - want_s).abs()
    assert torch.isfinite(got_s).all()
    assert (diff <= bound).all(), f"max excess {(diff - bound).max().item():.3e}"
    if zero_dc:
        assert (got_s[:, :, 0] == 0).all()
    # the estimate against the oracle's product of the spectrum and the kernel's rounded mask
    ref = oracle.mask_apply_forward(spec.cpu().numpy(), mask.float().cpu().numpy(), channels, zero_dc)
    ref = ref.reshape(b, stems, channels, f, t)[:, stem]
    ref_ri = np.stack([ref.real, ref.imag], axis=-1)
    assert_parity(got_s, ref_ri, "f32", "est")
    # without the hidden output: same estimate and pre-activation
    est2 = torch.full_like(est, sentinel)
    pre2, none = hip_ext.mask_mlp_forward_apply(x, w1, b1, w2, b2, dims, spec, est2, stem, channels, zero_dc)
    assert none is None and torch.equal(pre2, pre) and torch.equal(est2, est)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("zero_dc", [False, True])
def test_mask_apply_grad_mask_matches_backward(hip_ext, dtype, zero_dc):
    """``mask_apply_grad_mask`` (no mask argument) returns ``mask_apply_backward``'s mask gradient."""
    b, s, c, f, t = 2, 4, 2, 1025, 67
    g = torch.Generator().manual_seed(3)
    spec = torch.complex(torch.randn(b, f * c, t, generator=g), torch.randn(b, f * c, t, generator=g)).cuda()
    mask = torch.randn(b, s, t, 2 * f * c, generator=g).to(dtype).cuda()
    grad_est = torch.complex(torch.randn(b * s * c, f, t, generator=g), torch.randn(b * s * c, f, t, generator=g)).cuda()
    want, _ = hip_ext.mask_apply_backward(grad_est, spec, mask, c, zero_dc, need_spec_grad=False)
    got = hip_ext.mask_apply_grad_mask(grad_est, spec, s, c, dtype, zero_dc)
    assert got.dtype == dtype and got.shape == want.shape
    assert torch.equal(got, want)
    gm, _ = oracle.mask_apply_backward(grad_est.cpu().numpy(), spec.cpu().numpy(), mask.float().cpu().numpy(), c, zero_dc)
    assert_parity(got, gm, dt_name(dtype), "grad_mask")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_mask_mlp_apply_autograd_matches_two_functions(hip_ext, dtype):
    """``_FusedMaskMLPApply`` (masks never stored) against the stems' ``_FusedMaskMLP`` outputs stacked
    and multiplied in by ``_FusedMaskApply``: the estimate within one fp32 rounding of the product,
    the input and parameter gradients to the 16-bit bar (both run the same backward kernels)."""
    from pymsst_amd import fused_roformer as fr

    dims, b, t, dim, hidden, stems, channels = BSR_WIDTHS, 2, 129, 192, 768, 2, 2
    total = sum(dims)
    fc = total // 2
    g = torch.Generator().manual_seed(9)
    spec = torch.complex(torch.randn(b, fc, t, generator=g), torch.randn(b, fc, t, generator=g)).cuda()
    x0 = torch.randn(b * t, len(dims), dim, generator=g).to(dtype).cuda()
    params = []
    for s in range(stems):
        _, w1, b1, w2, _, b2 = _inputs(dims, 1, dim, hidden, dtype, seed=100 + s)
        params += [p.clone().requires_grad_(True) for p in (w1, b1, w2, b2)]
    weight = torch.randn(b * stems * channels, fc // channels, t, 2, generator=g).cuda()

    def run(fused):
        x = x0.clone().requires_grad_(True)
        ps = [p.detach().clone().requires_grad_(True) for p in params]
        if fused:
            est = fr._FusedMaskMLPApply.apply(spec, x, channels, True, dims, hip_ext, *ps)
        else:
            outs = [fr._FusedMaskMLP.apply(x, *ps[4 * s: 4 * s + 4], hip_ext, dims) for s in range(stems)]
            mask = torch.stack([o.view(b, t, total) for o in outs], dim=1)
            est = fr._FusedMaskApply.apply(spec, mask, channels, True, hip_ext)
        (torch.view_as_real(est) * weight).sum().backward()
        torch.cuda.synchronize()
        return est.detach(), x.grad, [p.grad for p in ps]

    est_f, dx_f, gp_f = run(True)
    est_r, dx_r, gp_r = run(False)
    assert (torch.view_as_real(est_f) - torch.view_as_real(est_r)).abs().max().item() <= \
        2.0**-20 * torch.view_as_real(est_r).abs().max().item()
    dn = dt_name(dtype)
    assert_parity(dx_f, to_np(dx_r), dn, "dx", by_index(1))
    names = ("w1", "b1", "w2", "b2")
    for i, (gf, gr) in enumerate(zip(gp_f, gp_r)):
        assert_parity(gf, to_np(gr), dn, f"stem {i // 4} {names[i % 4]}")

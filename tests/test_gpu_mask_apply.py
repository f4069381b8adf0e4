"""GPU parity: the complex mask product in the iSTFT layout (``mask_apply_forward/backward``),
against the numpy oracle (itself pinned to torch's CPU complex autograd of the stock model's
product, permute and zero-DC fill in ``test_oracle_pinning.py``).

Cases: the configs[2] shape (B=4 x 4 stems, stereo, 1025 bins, 258 frames) with bf16 masks; fp32 and
fp16 masks; odd sizes that leave partial tiles in both directions; a mask view with a batch stride
larger than its stems (no copy); zero_dc on and off; the spectrum gradient on and off; and the
patched BS-RoFormer against the stock model (loss and gradients) with zero_dc on.  The estimate and
the spectrum gradient are fp32 (bar 1e-5); the mask gradient is stored in the mask dtype.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pymsst_amd import fused_roformer as fr
from pymsst_amd.workloads import WORKLOADS, workload_batch
from tests.conftest import assert_parity, dt_name

pytestmark = pytest.mark.gpu


def _ri(z):
    z = z.detach().cpu().numpy() if isinstance(z, torch.Tensor) else z
    return np.stack([np.real(z), np.imag(z)], axis=-1)


def _inputs(b, s, c, f, t, dtype, seed, stem_pad=0):
    g = torch.Generator().manual_seed(seed)
    spec = torch.complex(torch.randn(b, f * c, t, generator=g), torch.randn(b, f * c, t, generator=g))
    mask_full = torch.randn(b, s + stem_pad, t, 2 * f * c, generator=g).to(dtype).cuda()
    return spec.cuda(), mask_full[:, stem_pad:]


@pytest.mark.parametrize(
    "b,s,c,f,t,dtype",
    [
        (4, 4, 2, 1025, 258, torch.bfloat16),
        (2, 3, 2, 33, 70, torch.float32),
        (3, 2, 1, 40, 129, torch.float16),
        (1, 1, 1, 7, 5, torch.float32),
        (2, 1, 2, 1, 64, torch.bfloat16),
    ],
)
@pytest.mark.parametrize("zero_dc", [False, True])
def test_mask_apply_vs_oracle(hip_ext, b, s, c, f, t, dtype, zero_dc):
    spec, mask = _inputs(b, s, c, f, t, dtype, seed=b * 100 + f + t)
    est = hip_ext.mask_apply_forward(spec, mask, c, zero_dc)
    assert est.shape == (b * s * c, f, t) and est.dtype == torch.complex64
    want = oracle.mask_apply_forward(spec.cpu().numpy(), mask.float().cpu().numpy(), c, zero_dc)
    assert_parity(_ri(est), _ri(want), "f32", "est")
    g = torch.Generator().manual_seed(7)
    grad_est = torch.complex(torch.randn(est.shape, generator=g), torch.randn(est.shape, generator=g)).cuda()
    grad_mask, grad_spec = hip_ext.mask_apply_backward(grad_est, spec, mask, c, zero_dc, need_spec_grad=True)
    want_gm, want_gs = oracle.mask_apply_backward(grad_est.cpu().numpy(), spec.cpu().numpy(),
                                                  mask.float().cpu().numpy(), c, zero_dc)
    assert grad_mask.dtype == dtype and grad_mask.shape == mask.shape
    assert_parity(grad_mask, want_gm, dt_name(dtype), "grad_mask")
    assert_parity(_ri(grad_spec), _ri(want_gs), "f32", "grad_spec")
    gm_only, none = hip_ext.mask_apply_backward(grad_est, spec, mask, c, zero_dc, need_spec_grad=False)
    assert none is None
    assert torch.equal(gm_only, grad_mask)


def test_mask_apply_strided_stems_view(hip_ext):
    # a [B, S, T, 2FC] view of a tensor with one more stem: batch stride > S * T * 2FC, no copy
    spec, mask = _inputs(3, 2, 2, 17, 66, torch.bfloat16, seed=11, stem_pad=1)
    assert not mask.is_contiguous()
    est = hip_ext.mask_apply_forward(spec, mask, 2)
    want = oracle.mask_apply_forward(spec.cpu().numpy(), mask.float().cpu().numpy(), 2)
    assert_parity(_ri(est), _ri(want), "f32", "est (strided mask)")


def test_mask_apply_autograd_function(hip_ext):
    spec, mask = _inputs(2, 3, 2, 20, 40, torch.float32, seed=3)
    spec.requires_grad_(True)
    mask.requires_grad_(True)
    est = fr._FusedMaskApply.apply(spec, mask, 2, False, hip_ext)
    w = torch.randn(est.shape, dtype=torch.float32, device="cuda")
    torch.view_as_real(est)[..., 0].mul(w).sum().backward()
    s2 = spec.detach().cpu().to(torch.complex128).requires_grad_(True)
    m2 = mask.detach().cpu().double().requires_grad_(True)
    b, st, t = m2.shape[:3]
    ref = (s2.unsqueeze(1) * torch.view_as_complex(m2.reshape(b, st, t, -1, 2)).transpose(-1, -2))
    ref = ref.reshape(b, st, -1, 2, t).transpose(2, 3).reshape(b * st * 2, -1, t)
    torch.view_as_real(ref)[..., 0].mul(w.cpu().double()).sum().backward()
    assert_parity(mask.grad, m2.grad.numpy(), "f32", "mask grad")
    assert_parity(_ri(spec.grad), _ri(s2.grad.numpy()), "f32", "spec grad")


def test_patched_model_matches_stock_with_zero_dc(monkeypatch, hip_ext):
    for key, value in fr.RUNTIME_PRESETS["hip_full"].items():
        monkeypatch.setenv(key, value)
    wl = WORKLOADS["bsr_tiny"]
    target, mixture = workload_batch(wl, seed=1, device="cuda")
    results = []
    try:
        for fused in (False, True):
            model = wl.build_model("cuda", seed=4)
            model.zero_dc = True
            model.train()
            fr.restore_stock_implementations(model)
            if fused:
                status = fr.apply_roformer_fused_training_backend(model, "hip", extension=hip_ext,
                                                                  rms_norm_mode="fast")
                assert status.patched_mask_apply
            loss = model(mixture, target)
            loss.backward()
            torch.cuda.synchronize()
            results.append((float(loss.detach()), {n: p.grad.detach().clone() for n, p in model.named_parameters()
                                                   if p.grad is not None}))
            fr.restore_stock_implementations(model)
    finally:
        fr.restore_stock_implementations()
    (ls, gs), (lf, gf) = results
    assert abs(lf - ls) <= 1e-5 * abs(ls), (lf, ls)
    for name, ref in gs.items():
        diff = (gf[name] - ref).abs().max().item()
        assert diff <= 1e-5 * max(1.0, ref.abs().max().item()), f"{name}: {diff:.3e}"

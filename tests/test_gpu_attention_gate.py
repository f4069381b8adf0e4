"""GPU parity: attention output gate (gate Linear + sigmoid + scale of the SDPA output), fwd + bwd.

Cases: the reference op signature (``attention_gate_forward/backward`` on ``[M,H,Dh]``,
fused_band_split.cpp:536-587) at the BS-RoFormer head layout (8 x 64, dim 192) and the
configs[0] layout (4 x 32, dim 64) in every dtype; shapes that take the generic kernels
(odd heads/head dims, 32 heads); the in-place ``[B,N,H,Dh]`` path on the transposed SDPA
output with the gradient written in the ``[B,H,N,Dh]`` layout; a row count that needs more
than one row chunk per dW block; no rows; the autograd Function.  Bars are those of ``conftest.py``.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from tests.conftest import assert_parity, dt_name, to_np

pytestmark = pytest.mark.gpu


def _inputs(m, h, dh, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    attn = torch.randn(m, h, dh, generator=g).to(dtype).cuda()
    x = torch.randn(m, d, generator=g).to(dtype).cuda()
    w = (torch.randn(h, d, generator=g) / d**0.5).to(dtype).cuda()
    b = (0.5 * torch.randn(h, generator=g)).to(dtype).cuda()
    gout = torch.randn(m, h * dh, generator=g).to(dtype).cuda()
    return attn, x, w, b, gout


def _check_ref_api(ext, m, h, dh, d, dtype, seed):
    dn = dt_name(dtype)
    attn, x, w, b, gout = _inputs(m, h, dh, d, dtype, seed)
    out, gate, sa, sx = ext.attention_gate_forward(attn, x, w, b)
    assert out.shape == (m, h * dh) and gate.shape == (m, h)
    r_out, r_gate = oracle.attention_gate_forward(to_np(attn), to_np(x), to_np(w), to_np(b), dn)
    assert_parity(gate, r_gate, dn, "gate")
    assert_parity(out, r_out, dn, "out")
    ga, gx, gw, gb = ext.attention_gate_backward(gout, sa, sx, w, gate)
    # backward from the kernel's own stored gate (the saved tensor of the op)
    r = oracle.attention_gate_backward(to_np(gout), to_np(attn), to_np(x), to_np(w), to_np(gate), dn)
    assert ga.shape == attn.shape and gx.shape == x.shape and gw.shape == w.shape and gb.shape == b.shape
    assert_parity(ga, r[0], dn, "grad_attn")
    assert_parity(gx, r[1], dn, "grad_x")
    assert_parity(gw, r[2], dn, "grad_weight")
    assert_parity(gb, r[3], dn, "grad_bias")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1000, 8, 64, 192), (130, 4, 32, 64), (77, 8, 64, 512), (9, 2, 64, 16)])
def test_reference_op_fast_shapes(hip_ext, dtype, shape):
    _check_ref_api(hip_ext, *shape, dtype, 31)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(37, 3, 5, 7), (50, 32, 64, 96), (21, 8, 20, 33), (16, 1, 64, 70)])
def test_reference_op_generic_shapes(hip_ext, dtype, shape):
    _check_ref_api(hip_ext, *shape, dtype, 32)


def test_many_rows_multiple_rows_per_chunk(hip_ext):
    # 140000 rows > 2048 chunks of 64 rows: the dW chunk height doubles
    _check_ref_api(hip_ext, 140000, 2, 64, 24, torch.float32, 33)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_bnhd_views_in_place(hip_ext, dtype):
    """The transposed SDPA output is read in place and grad_attn is written as [B,H,N,Dh]."""
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(34)
    bsz, n, h, dh, d = 4, 258, 8, 64, 192
    attn_bhnd = torch.randn(bsz, h, n, dh, generator=g).to(dtype).cuda()
    attn = attn_bhnd.transpose(1, 2)
    assert not attn.is_contiguous()
    x = torch.randn(bsz * n, d, generator=g).to(dtype).cuda()
    w = (torch.randn(h, d, generator=g) / d**0.5).to(dtype).cuda()
    b = (0.5 * torch.randn(h, generator=g)).to(dtype).cuda()
    out, gate, sa, sx = hip_ext.attention_gate_forward_bnhd(attn, x, w, b)
    a3 = to_np(attn).reshape(bsz * n, h, dh)
    r_out, r_gate = oracle.attention_gate_forward(a3, to_np(x), to_np(w), to_np(b), dn)
    assert_parity(out, r_out, dn, "out")
    assert_parity(gate, r_gate, dn, "gate")
    # same values as the reference-signature op on a contiguous copy
    out2, gate2, _, _ = hip_ext.attention_gate_forward(attn.reshape(bsz * n, h, dh), x, w, b)
    assert torch.equal(out, out2) and torch.equal(gate, gate2)
    gout = torch.randn(bsz * n, h * dh, generator=g).to(dtype).cuda()
    ga, gx, gw, gb = hip_ext.attention_gate_backward_bnhd(gout, sa, sx, w, gate)
    assert ga.shape == attn.shape and ga.transpose(1, 2).is_contiguous()
    r = oracle.attention_gate_backward(to_np(gout), a3, to_np(x), to_np(w), to_np(gate), dn)
    assert_parity(ga.reshape(bsz * n, h, dh), r[0], dn, "grad_attn")
    assert_parity(gx, r[1], dn, "grad_x")
    assert_parity(gw, r[2], dn, "grad_weight")
    assert_parity(gb, r[3], dn, "grad_bias")
    # dense [B,N,H,Dh] gradient (the flash-attention layout): same values, other storage order
    ga2, gx2, gw2, gb2 = hip_ext.attention_gate_backward_bnhd(gout, sa, sx, w, gate, out_layout="bnhd")
    assert ga2.shape == attn.shape and ga2.is_contiguous()
    assert torch.equal(ga2, ga) and torch.equal(gx2, gx) and torch.equal(gw2, gw) and torch.equal(gb2, gb)


def test_flash_layout_attention_copies_nothing(hip_ext):
    """16-bit attention block on the fused path: q/k/v from the qkv rotary in dense [B,N,H,D], SDPA on
    their [B,H,N,D] views, the gate on its output; no aten::clone runs in forward or backward."""
    from torch.profiler import ProfilerActivity, profile

    from pymsst_amd.core import transformer
    from pymsst_amd.fused_roformer import _FusedAttentionGate, _FusedQKVRotary

    g = torch.Generator().manual_seed(35)
    bsz, n, h, dh, d = 8, 62, 8, 64, 192
    qkv = torch.randn(bsz, n, 3 * h * dh, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    pos = torch.arange(n, dtype=torch.float32)[:, None] / (10000 ** (torch.arange(0, dh, 2) / dh))[None]
    cos = pos.cos().repeat_interleave(2, -1).view(1, n, 1, dh).to(torch.bfloat16).cuda()
    sin = pos.sin().repeat_interleave(2, -1).view(1, n, 1, dh).to(torch.bfloat16).cuda()
    x = torch.randn(bsz, n, d, generator=g).to(torch.bfloat16).cuda().requires_grad_()
    w = (torch.randn(h, d, generator=g) / d**0.5).to(torch.bfloat16).cuda().requires_grad_()
    b = torch.randn(h, generator=g).to(torch.bfloat16).cuda().requires_grad_()

    def block(layout):
        q, k, v = _FusedQKVRotary.apply(qkv, cos[..., ::2], sin[..., ::2], h, hip_ext, layout)
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        if layout == "bnhd":
            out = transformer._sdpa(q, k, v, 0.0).transpose(1, 2)
        else:
            out = transformer._sdpa(q.contiguous(), k.contiguous(), v.contiguous(), 0.0).transpose(1, 2)
        gated = _FusedAttentionGate.apply(out, x, w, b, hip_ext)
        (gated.float() * torch.linspace(-1, 1, gated.shape[-1], device="cuda")).sum().backward()
        grads = [t.grad for t in (qkv, x, w, b)]
        for t in (qkv, x, w, b):
            t.grad = None
        return gated.detach(), grads

    ref_out, ref_grads = block("bhnd")
    torch.cuda.synchronize()
    with profile(activities=[ProfilerActivity.CPU]) as prof:
        out, grads = block("bnhd")
        torch.cuda.synchronize()
    clones = [e for e in prof.events() if e.name == "aten::clone"]
    assert not clones, [e.name for e in clones]
    # the layouts change the storage order only: same values, to bf16 rounding of the attention
    assert torch.allclose(out.float(), ref_out.float(), rtol=2e-2, atol=2e-2)
    for got, want in zip(grads, ref_grads):
        err = (got.float() - want.float()).norm() / want.float().norm()
        assert err < 2e-2, err


def test_no_rows(hip_ext):
    attn = torch.empty(0, 8, 64, device="cuda")
    x = torch.empty(0, 192, device="cuda")
    w = torch.randn(8, 192, device="cuda")
    b = torch.randn(8, device="cuda")
    out, gate, sa, sx = hip_ext.attention_gate_forward(attn, x, w, b)
    assert out.shape == (0, 512) and gate.shape == (0, 8)
    ga, gx, gw, gb = hip_ext.attention_gate_backward(out, sa, sx, w, gate)
    assert ga.shape == (0, 8, 64) and gx.shape == (0, 192)
    assert torch.count_nonzero(gw).item() == 0 and torch.count_nonzero(gb).item() == 0


def test_argument_errors(hip_ext):
    attn = torch.randn(4, 8, 64, device="cuda")
    with pytest.raises(RuntimeError, match="attn heads must match weight"):
        hip_ext.attention_gate_forward(attn, torch.randn(4, 16, device="cuda"), torch.randn(7, 16, device="cuda"),
                                       torch.randn(7, device="cuda"))
    with pytest.raises(RuntimeError, match="x dtype must match attn"):
        hip_ext.attention_gate_forward(attn, torch.randn(4, 16, device="cuda").half(), torch.randn(8, 16, device="cuda"),
                                       torch.randn(8, device="cuda"))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_autograd_function(hip_ext, dtype):
    from pymsst_amd.fused_roformer import _FusedAttentionGate

    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(35)
    bsz, n, h, dh, d = 2, 62, 8, 64, 192
    attn = torch.randn(bsz, h, n, dh, generator=g).to(dtype).cuda().transpose(1, 2).requires_grad_()
    x = torch.randn(bsz, n, d, generator=g).to(dtype).cuda().requires_grad_()
    w = (torch.randn(h, d, generator=g) / d**0.5).to(dtype).cuda().requires_grad_()
    b = (0.5 * torch.randn(h, generator=g)).to(dtype).cuda().requires_grad_()
    out = _FusedAttentionGate.apply(attn, x, w, b, hip_ext)
    assert out.shape == (bsz, n, h * dh)
    a3 = to_np(attn).reshape(bsz * n, h, dh)
    r_out, r_gate = oracle.attention_gate_forward(a3, to_np(x).reshape(bsz * n, d), to_np(w), to_np(b), dn)
    assert_parity(out.reshape(bsz * n, -1), r_out, dn, "out")
    gout = torch.randn(out.shape, generator=g).to(dtype).cuda()
    out.backward(gout)
    r = oracle.attention_gate_backward(to_np(gout).reshape(bsz * n, -1), a3, to_np(x).reshape(bsz * n, d), to_np(w),
                                       r_gate, dn)
    assert attn.grad.shape == attn.shape
    assert_parity(attn.grad.reshape(bsz * n, h, dh), r[0], dn, "grad_attn")
    assert_parity(x.grad.reshape(bsz * n, d), r[1], dn, "grad_x")
    assert_parity(w.grad, r[2], dn, "grad_weight")
    assert_parity(b.grad, r[3], dn, "grad_bias")

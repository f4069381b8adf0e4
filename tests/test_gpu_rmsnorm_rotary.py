"""GPU parity: RMSNorm (plain / fp32-gamma / mixed / saved-input), rotary and fused q/k norm+rotary.

Each case calls the HIP kernels through the C ABI (via ``HipFusedExtension``)
and compares with the float64 oracle on the same seeded inputs, to the bars in
``conftest.py``.  Shapes cover the reference configs (dim 64/192/512, head dim
32/64), the guarded scalar path (dims not a multiple of the pack width), empty
inputs, a single row, and all-zero rows (inv_norm = 1e12).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_parity, dt_name, to_np

pytestmark = pytest.mark.gpu

DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _rand(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype).cuda()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("rows,dim", [(1, 64), (257, 192), (1031, 512), (130, 64), (77, 100), (33, 8), (5, 6)])
def test_rms_norm_plain(hip_ext, dtype, rows, dim):
    dn = dt_name(dtype)
    x = _rand((rows, dim), dtype, 1)
    if rows > 3:
        x[3].zero_()
    gamma = (1 + 0.1 * _rand((dim,), torch.float32, 2)).to(dtype)
    out, normed, inv = hip_ext.rms_norm_forward(x, gamma)
    r_out, r_normed, r_inv = oracle.rms_norm_forward(to_np(x), to_np(gamma), dn, "plain")
    assert_parity(out, r_out, dn, "out")
    assert_parity(normed, r_normed, dn, "normed")
    assert_parity(inv.clamp(max=1e6), np.minimum(r_inv, 1e6), "f32", "inv_norm")
    dy = _rand((rows, dim), dtype, 3)
    dx, dg = hip_ext.rms_norm_backward(dy, normed, inv, gamma)
    r_dx, r_dg = oracle.rms_norm_backward(to_np(dy), to_np(normed), to_np(inv), to_np(gamma), dn, "plain")
    if rows > 3:
        # zero row: dx = inv * gn * sqrt(D) with inv = 1e12 -- compared relative to its own scale
        keep = [i for i in range(rows) if i != 3]
        assert_parity(dx[keep], r_dx[keep], dn, "dx")
        a3, r3 = to_np(dx[3]), r_dx[3]
        # fp16 overflows to inf here (1e12 * g): both sides must agree on which entries are infinite
        assert np.array_equal(np.isinf(a3), np.isinf(r3))
        assert np.array_equal(a3[np.isinf(a3)], r3[np.isinf(r3)])
        fin = np.isfinite(r3)
        if fin.any():
            rel = np.max(np.abs(a3[fin] - r3[fin])) / max(np.max(np.abs(r3[fin])), 1e-30)
            assert rel <= (1e-5 if dn == "f32" else 2e-2), f"zero-row dx rel err {rel}"
    else:
        assert_parity(dx, r_dx, dn, "dx")
    assert_parity(dg, r_dg, dn, "dgamma")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,dim", [(1000, 192), (64, 64), (17, 100)])
def test_rms_norm_fp32_gamma_and_mixed(hip_ext, dtype, rows, dim):
    dn = dt_name(dtype)
    x = _rand((rows, dim), dtype, 11)
    gamma = 1 + 0.1 * _rand((dim,), torch.float32, 12)
    out, normed, inv = hip_ext.rms_norm_forward_fp32_gamma(x, gamma)
    assert out.dtype == dtype and normed.dtype == dtype
    r_out, r_normed, _ = oracle.rms_norm_forward(to_np(x), to_np(gamma), dn, "fp32_gamma")
    assert_parity(out, r_out, dn, "fp32g out")
    assert_parity(normed, r_normed, dn, "fp32g normed")
    dy = _rand((rows, dim), dtype, 13)
    dx, dg = hip_ext.rms_norm_backward_fp32_gamma(dy, normed, inv, gamma)
    assert dg.dtype == torch.float32
    r_dx, r_dg = oracle.rms_norm_backward(to_np(dy), to_np(normed), to_np(inv), to_np(gamma), dn, "fp32_gamma")
    assert_parity(dx, r_dx, dn, "fp32g dx")
    assert_parity(dg, r_dg, "f32" if dn == "f32" else dn, "fp32g dgamma")

    out, normed, inv = hip_ext.rms_norm_forward_mixed(x, gamma)
    assert out.dtype == torch.float32 and normed.dtype == torch.float32
    r_out, r_normed, _ = oracle.rms_norm_forward(to_np(x), to_np(gamma), dn, "mixed")
    assert_parity(out, r_out, "f32", "mixed out")
    assert_parity(normed, r_normed, "f32", "mixed normed")
    dy32 = _rand((rows, dim), torch.float32, 14)
    dx, dg = hip_ext.rms_norm_backward_mixed(dy32, normed, inv, gamma, x.new_empty(0))
    assert dx.dtype == dtype
    r_dx, r_dg = oracle.rms_norm_backward(to_np(dy32), to_np(normed), to_np(inv), to_np(gamma), dn, "mixed")
    assert_parity(dx, r_dx, dn, "mixed dx")
    assert_parity(dg, r_dg, "f32", "mixed dgamma")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("gamma_fp32", [False, True])
def test_rms_norm_lean_roundtrip(hip_ext, dtype, gamma_fp32):
    dn = dt_name(dtype)
    rows, dim = 2049, 192
    x = _rand((rows, dim), dtype, 21)
    gamma = 1 + 0.1 * _rand((dim,), torch.float32, 22)
    if not gamma_fp32:
        gamma = gamma.to(dtype)
    out, inv = hip_ext.rms_norm_forward_lean(x, gamma)
    mode = "fp32_gamma" if gamma_fp32 and dtype != torch.float32 else "plain"
    r_out, _, _ = oracle.rms_norm_forward(to_np(x), to_np(gamma), dn, mode)
    assert_parity(out, r_out, dn, "lean out")
    dy = _rand((rows, dim), dtype, 23)
    dx, dg = hip_ext.rms_norm_backward_from_input(dy, x, inv, gamma)
    gdt = "f32" if gamma.dtype == torch.float32 else dn
    r_dx, r_dg = oracle.rms_norm_backward_lean(to_np(dy), to_np(x), to_np(inv), to_np(gamma), dn, gdt)
    assert_parity(dx, r_dx, dn, "lean dx")
    assert_parity(dg, r_dg, gdt, "lean dgamma")


def test_rms_norm_empty_and_large(hip_ext):
    x = torch.empty(0, 192, device="cuda", dtype=torch.bfloat16)
    gamma = torch.ones(192, device="cuda", dtype=torch.bfloat16)
    out, normed, inv = hip_ext.rms_norm_forward(x, gamma)
    assert out.shape == (0, 192) and inv.shape == (0,)
    dx, dg = hip_ext.rms_norm_backward(out, normed, inv, gamma)
    assert dx.shape == (0, 192)
    assert torch.count_nonzero(dg).item() == 0
    # the cfg3 transformer shape: 63,984 rows x 192, fp32 (the dtype of the residual stream under autocast)
    rows, dim = 63984, 192
    x = _rand((rows, dim), torch.float32, 31)
    gamma = 1 + 0.1 * _rand((dim,), torch.float32, 32)
    out, normed, inv = hip_ext.rms_norm_forward(x, gamma)
    dy = _rand((rows, dim), torch.float32, 33)
    dx, dg = hip_ext.rms_norm_backward(dy, normed, inv, gamma)
    # size-independent properties: ||normed|| = sqrt(D) per row; dx is orthogonal to normed (scale invariance)
    nrm = normed.double().norm(dim=-1)
    assert torch.allclose(nrm, torch.full_like(nrm, dim**0.5), rtol=1e-5)
    ortho = (dx.double() * x.double()).sum(-1).abs().max().item()
    assert ortho <= 1e-4 * dx.double().abs().max().item() * x.double().abs().max().item() * dim**0.5
    # dgamma against a float64 torch reduction of the same inputs
    ref_dg = (dy.double() * normed.double()).sum(0)
    assert_parity(dg, ref_dg, "f32", "large dgamma")


def test_rms_norm_rejects_bad_args(hip_ext):
    x = torch.randn(4, 8, device="cuda")
    with pytest.raises(RuntimeError, match="gamma dimension must match"):
        hip_ext.rms_norm_forward(x, torch.ones(7, device="cuda"))
    with pytest.raises(RuntimeError, match="gamma dtype must match x"):
        hip_ext.rms_norm_forward(x, torch.ones(8, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="gamma must be float32"):
        hip_ext.rms_norm_forward_mixed(x.bfloat16(), torch.ones(8, device="cuda", dtype=torch.bfloat16))
    with pytest.raises(RuntimeError, match="not supported"):
        hip_ext.rms_norm_forward(torch.randn(2, 1001, device="cuda"), torch.ones(1001, device="cuda"))


def _tables(n, d, dtype, sliced=True):
    c, s = oracle.rotary_tables(n, d)
    c = torch.from_numpy(c).to(dtype).cuda()
    s = torch.from_numpy(s).to(dtype).cuda()
    if sliced:
        # the reference passes cos[..., ::2] of the pairwise-repeated [1,N,1,D] table (fused_roformer.py:727)
        c = c.repeat_interleave(2, dim=-1).reshape(1, n, 1, d)[..., ::2]
        s = s.repeat_interleave(2, dim=-1).reshape(1, n, 1, d)[..., ::2]
    else:
        c = c.reshape(1, n, 1, d // 2)
        s = s.reshape(1, n, 1, d // 2)
    return c, s


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(3, 65, 4, 32), (2, 62, 8, 64), (5, 7, 3, 6), (1, 1, 1, 2)])
@pytest.mark.parametrize("sliced", [True, False])
def test_rotary(hip_ext, dtype, shape, sliced):
    dn = dt_name(dtype)
    b, n, h, d = shape
    t = _rand(shape, dtype, 41)
    cos, sin = _tables(n, d, dtype, sliced)
    out = hip_ext.rotary_forward(t, cos, sin)
    r = oracle.rotary_forward(to_np(t), to_np(cos).reshape(n, d // 2), to_np(sin).reshape(n, d // 2), dn)
    assert_parity(out, r, dn, "rotary fwd")
    g = _rand(shape, dtype, 42)
    dt_ = hip_ext.rotary_backward(g, cos, sin)
    r = oracle.rotary_backward(to_np(g), to_np(cos).reshape(n, d // 2), to_np(sin).reshape(n, d // 2), dn)
    assert_parity(dt_, r, dn, "rotary bwd")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(3, 65, 4, 32), (2, 62, 8, 64), (5, 7, 3, 6)])
def test_rotary_strided_qkv_view_and_bhnd_output(hip_ext, dtype, shape):
    """q/k read in place from a fused qkv projection ([B, N, 3*H*D] viewed as [B, N, 3, H, D] and
    unbound, as Attention does) and written as the [B,N,H,D]-shaped view of a dense [B,H,N,D]
    buffer; the backward takes the transposed gradient SDPA hands back."""
    dn = dt_name(dtype)
    b, n, h, d = shape
    qkv = _rand((b, n, 3 * h * d), dtype, 43)
    q, k, _ = qkv.view(b, n, 3, h, d).unbind(dim=2)
    assert not q.is_contiguous()
    cos, sin = _tables(n, d, dtype, True)
    cn, sn = to_np(cos).reshape(n, d // 2), to_np(sin).reshape(n, d // 2)
    for t in (q, k):
        for layout in ("bnhd", "bhnd"):
            out = hip_ext.rotary_forward(t, cos, sin, out_layout=layout)
            assert out.shape == (b, n, h, d)
            if layout == "bhnd":
                assert out.transpose(1, 2).is_contiguous()
            assert_parity(out, oracle.rotary_forward(to_np(t), cn, sn, dn), dn, f"rotary fwd {layout}")
    g = _rand((b, h, n, d), dtype, 44).transpose(1, 2)  # SDPA-style gradient, bhnd memory
    dt_ = hip_ext.rotary_backward(g, cos, sin)
    assert dt_.is_contiguous()
    assert_parity(dt_, oracle.rotary_backward(to_np(g), cn, sn, dn), dn, "rotary bwd strided")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(2, 7, 3, 16), (248, 258, 8, 64), (1032, 62, 8, 64), (3, 5, 2, 6)])
def test_rotary_qkv_split_forward_backward(hip_ext, dtype, shape):
    """One launch splits a fused qkv projection into rotated q, rotated k and v (dense [B,H,N,D] or
    dense [B,N,H,D] storage); the backward writes the qkv gradient (q, k rotated back, v copied) in one launch."""
    dn = dt_name(dtype)
    b, n, h, d = shape
    qkv = _rand((b, n, 3 * h * d), dtype, 45)
    cos, sin = _tables(n, d, dtype, True)
    cn, sn = to_np(cos).reshape(n, d // 2), to_np(sin).reshape(n, d // 2)
    q, k, v = hip_ext.rotary_qkv_forward(qkv, h, cos, sin)
    parts = qkv.view(b, n, 3, h, d).unbind(2)
    for name, out, src, rot in (("q", q, parts[0], True), ("k", k, parts[1], True), ("v", v, parts[2], False)):
        assert out.shape == (b, n, h, d) and out.transpose(1, 2).is_contiguous()
        if rot:
            assert_parity(out, oracle.rotary_forward(to_np(src), cn, sn, dn), dn, f"qkv fwd {name}")
        else:
            assert torch.equal(out, src)
    # dense [B,N,H,D] outputs: the same values
    for out, dense in zip((q, k, v), hip_ext.rotary_qkv_forward(qkv, h, cos, sin, out_layout="bnhd")):
        assert dense.shape == (b, n, h, d) and dense.is_contiguous() and torch.equal(dense, out)
    gq, gk, gv = (_rand((b, h, n, d), dtype, 46 + i).transpose(1, 2) for i in range(3))
    dqkv = hip_ext.rotary_qkv_backward(gq, gk, gv, cos, sin)
    assert dqkv.shape == qkv.shape and dqkv.is_contiguous()
    dparts = dqkv.view(b, n, 3, h, d).unbind(2)
    assert_parity(dparts[0], oracle.rotary_backward(to_np(gq), cn, sn, dn), dn, "qkv bwd q")
    assert_parity(dparts[1], oracle.rotary_backward(to_np(gk), cn, sn, dn), dn, "qkv bwd k")
    assert torch.equal(dparts[2], gv)
    # same values as the single-tensor ops
    assert torch.equal(q, hip_ext.rotary_forward(parts[0], cos, sin))
    assert torch.equal(dparts[1], hip_ext.rotary_backward(gk, cos, sin))


def test_fused_qkv_rotary_autograd(hip_ext):
    from pymsst_amd.fused_roformer import _FusedQKVRotary

    b, n, h, d = 4, 62, 8, 64
    qkv = _rand((b, n, 3 * h * d), torch.float32, 47).requires_grad_()
    cos, sin = _tables(n, d, torch.float32, True)
    q, k, v = _FusedQKVRotary.apply(qkv, cos, sin, h, hip_ext)
    loss = (q * 1.5).sum() + (k * k).sum() + (v * 0.5).sum()
    loss.backward()
    cn, sn = to_np(cos).reshape(n, d // 2), to_np(sin).reshape(n, d // 2)
    gq = torch.full_like(q, 1.5)
    gk = 2 * k.detach()
    expect = torch.cat([
        torch.from_numpy(oracle.rotary_backward(to_np(gq), cn, sn, "f32")).float().cuda().reshape(b, n, 1, h, d),
        torch.from_numpy(oracle.rotary_backward(to_np(gk), cn, sn, "f32")).float().cuda().reshape(b, n, 1, h, d),
        torch.full((b, n, 1, h, d), 0.5, device="cuda"),
    ], dim=2).reshape(b, n, -1)
    assert_parity(qkv.grad, to_np(expect), "f32", "dqkv")


def test_rotary_microbench_shape_roundtrip(hip_ext):
    # cfg2 q/k shape; forward then backward is the identity up to rounding (rotation is orthogonal)
    shape = (248, 258, 8, 64)
    t = _rand(shape, torch.float32, 51)
    cos, sin = _tables(258, 64, torch.float32)
    back = hip_ext.rotary_backward(hip_ext.rotary_forward(t, cos, sin), cos, sin)
    assert (back - t).abs().max().item() <= 1e-5
    nr = hip_ext.rotary_forward(t, cos, sin).double().norm(dim=-1)
    assert torch.allclose(nr, t.double().norm(dim=-1), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("gamma_fp32", [False, True])
@pytest.mark.parametrize("shape", [(4, 65, 4, 32), (6, 258, 8, 64), (2, 3, 1, 128)])
def test_rms_norm_rotary_fused(hip_ext, dtype, gamma_fp32, shape):
    dn = dt_name(dtype)
    b, n, h, d = shape
    x = _rand(shape, dtype, 61)
    gamma = 1 + 0.1 * _rand((d,), torch.float32, 62)
    if not gamma_fp32:
        gamma = gamma.to(dtype)
    cos, sin = _tables(n, d, dtype)
    out, inv = hip_ext.rms_norm_rotary_forward(x, gamma, cos, sin)
    cn, sn = to_np(cos).reshape(n, d // 2), to_np(sin).reshape(n, d // 2)
    r_out, r_inv = oracle.rms_norm_rotary_forward(to_np(x), to_np(gamma), cn, sn, dn)
    assert_parity(out, r_out, dn, "norm-rot out")
    assert_parity(inv, r_inv.reshape(-1), "f32", "norm-rot inv")
    dy = _rand(shape, dtype, 63)
    dx, dg = hip_ext.rms_norm_rotary_backward(dy, x, inv, gamma, cos, sin)
    gdt = "f32" if gamma.dtype == torch.float32 else dn
    r_dx, r_dg = oracle.rms_norm_rotary_backward(to_np(dy), to_np(x), to_np(inv), to_np(gamma), cn, sn, dn, gdt)
    assert_parity(dx, r_dx, dn, "norm-rot dx")
    assert_parity(dg, r_dg, gdt, "norm-rot dgamma")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("gamma_fp32", [False, True])
@pytest.mark.parametrize("shape", [(4, 65, 4, 32), (248, 258, 8, 64), (2, 3, 1, 128)])
def test_rms_norm_rotary_pair_equals_single(hip_ext, dtype, gamma_fp32, shape):
    """q and k in one launch each way (the configs[1] microbench op): every output bit for bit the
    single-tensor op's, dgamma included (the pair's column sums run over the same partial rows)."""
    b, n, h, d = shape
    q, k = _rand(shape, dtype, 71), _rand(shape, dtype, 72)
    gq = 1 + 0.1 * _rand((d,), torch.float32, 73)
    gk = 1 + 0.1 * _rand((d,), torch.float32, 74)
    if not gamma_fp32:
        gq, gk = gq.to(dtype), gk.to(dtype)
    cos, sin = _tables(n, d, dtype)
    qo, ko, iq, ik = hip_ext.rms_norm_rotary_pair_forward(q, k, gq, gk, cos, sin)
    sq, siq = hip_ext.rms_norm_rotary_forward(q, gq, cos, sin)
    sk, sik = hip_ext.rms_norm_rotary_forward(k, gk, cos, sin)
    assert torch.equal(qo, sq) and torch.equal(ko, sk) and torch.equal(iq, siq) and torch.equal(ik, sik)
    dq_, dk_ = _rand(shape, dtype, 75), _rand(shape, dtype, 76)
    dq, dk, dgq, dgk = hip_ext.rms_norm_rotary_pair_backward(dq_, dk_, q, k, iq, ik, gq, gk, cos, sin)
    sdq, sdgq = hip_ext.rms_norm_rotary_backward(dq_, q, siq, gq, cos, sin)
    sdk, sdgk = hip_ext.rms_norm_rotary_backward(dk_, k, sik, gk, cos, sin)
    assert torch.equal(dq, sdq) and torch.equal(dk, sdk)
    assert torch.equal(dgq, sdgq) and torch.equal(dgk, sdgk)

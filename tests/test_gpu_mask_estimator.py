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
from tests.conftest import assert_parity, by_band, by_index, dt_name, to_np

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
    two = [2 * d for d in dim_inputs]
    assert_parity(out, r_out, dn, "out", by_band(1, dim_inputs))
    assert_parity(pre, r_pre, dn, "pre", by_band(1, two))
    gout = torch.randn(out.shape, generator=g).to(dtype).cuda()
    res = bwd(gout, x_saved, pre, weights, list(dim_inputs), offs)
    # one kernel serves both reference modes with the grouped mode's rounding point: dpre is stored in
    # the tensor dtype before the dx / dW products (.cu:2343-2344)
    r_dx, r_db, r_dw = oracle.mask_estimator_final_backward(to_np(gout), to_np(x), to_np(pre), npw, dim_inputs, dn,
                                                            grad_pre_dt=dn)
    assert_parity(res[0], r_dx, dn, "dx", by_index(1))
    assert_parity(res[1], r_db, dn, "dbias", by_band(0, two))
    for b in range(nb):
        assert res[2 + b].shape == (2 * dim_inputs[b], hidden)
    assert_parity(torch.cat([w.reshape(-1) for w in res[2:]]), np.concatenate([w.reshape(-1) for w in r_dw]), dn,
                  "dW", by_band(0, [t * hidden for t in two]))
    if direct:
        # the direct mode's own rounding (.cu:2585-2704): dx and dbias from the fp32 dpre, dW from the
        # 16-bit grad_pre; the kernels' 16-bit dpre meets it per element, at the same bars
        d_dx, d_db, d_dw = oracle.mask_estimator_final_backward(to_np(gout), to_np(x), to_np(pre), npw, dim_inputs, dn)
        assert_parity(res[0], d_dx, dn, "dx (direct-mode oracle)", by_index(1))
        assert_parity(res[1], d_db, dn, "dbias (direct-mode oracle)", by_band(0, two))
        assert_parity(torch.cat([w.reshape(-1) for w in res[2:]]), np.concatenate([w.reshape(-1) for w in d_dw]), dn,
                      "dW (direct-mode oracle)", by_band(0, [t * hidden for t in two]))


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


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m,hidden", [(77, 200), (64, 768), (1, 144), (300, 216), (130, 256), (3, 384)])
def test_register_direct_forward_classes(hip_ext, dtype, m, hidden):
    """16-bit forward and backward with every width a multiple of 4 (the DMA-ring kernels when
    hidden % 8 == 0, and for dx when hidden % 128 == 0): narrow and wide bands, partial first K
    chunks of the forward (hidden % 32 != 0) and of dx (2 I_b % 32 != 0), M not a multiple of
    the row tiles."""
    widths = (4, 8, 12, 16, 20, 24, 32, 36, 48, 96, 100, 516, 8, 4)
    _check(hip_ext, widths, m, hidden, dtype, 17 + m)


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


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(129, 62, 192, 768), (37, 3, 6, 10), (130, 62, 64, 256), (65, 4, 512, 2048),
                                   (100, 100, 192, 776),
                                   # 16-bit dx on 48-row waves with row tiles of 144 (7 x 144 + 25) and
                                   # 176 rows (15 x 176 + 120) instead of the block's 192
                                   (1033, 62, 192, 768), (2760, 60, 192, 768)])
def test_grouped_linear_tanh_forward_and_backward(hip_ext, dtype, shape):
    """Mask-MLP hidden layer: grouped linear with the tanh epilogue, and the grouped-linear backward
    (dx, dW, db) against the oracle; odd widths (6 -> 10) take the unaligned paths.  At 100 groups of
    192 -> 776 the 16-bit dW takes 192 output columns per block (fewer rounds of resident blocks than
    128) with a last column tile of 8."""
    dn = dt_name(dtype)
    m, groups, i, o = shape
    g = torch.Generator().manual_seed(21)
    x = torch.randn(m, groups, i, generator=g).to(dtype).cuda()
    w = (torch.randn(groups, o, i, generator=g) / i**0.5).to(dtype).cuda()
    b = (0.1 * torch.randn(groups, o, generator=g)).to(dtype).cuda()
    out = hip_ext.grouped_linear_forward_act(x, w, b, activation="tanh")
    assert_parity(out, oracle.grouped_linear_forward(to_np(x), to_np(w), to_np(b), dn, act="tanh"), dn, "tanh fwd")
    plain = hip_ext.grouped_linear_forward(x, w, b)
    assert torch.allclose(torch.tanh(plain.float()), out.float(), atol=2e-2 if dtype != torch.float32 else 1e-6)
    dy = torch.randn(m, groups, o, generator=g).to(dtype).cuda()
    for has_bias in (True, False):
        dx, dw, db = hip_ext.grouped_linear_backward(dy, x, w, has_bias)
        rdx, rdw, rdb = oracle.grouped_linear_backward(to_np(dy), to_np(x), to_np(w), has_bias, dn)
        assert_parity(dx, rdx, dn, "dx")
        assert_parity(dw, rdw, dn, "dW")
        if has_bias:
            assert_parity(db, rdb, dn, "db")
        else:
            assert db is None


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_mask_final_backward_with_tanh_input(hip_ext, dtype):
    dn = dt_name(dtype)
    dims = BSR_WIDTHS
    m, hidden = 130, 256
    g = torch.Generator().manual_seed(22)
    h = torch.tanh(torch.randn(m, len(dims), hidden, generator=g)).to(dtype).cuda()
    w_all = torch.cat([(torch.randn(2 * d, hidden, generator=g) / hidden**0.5).reshape(-1) for d in dims])
    w_all = w_all.to(dtype).cuda()
    bias = (0.1 * torch.randn(2 * sum(dims), generator=g)).to(dtype).cuda()
    out, pre = hip_ext.mask_estimator_final_forward_packed(h, w_all, bias, dims)
    gout = torch.randn(out.shape, generator=g).to(dtype).cuda()
    dz, db, dw = hip_ext.mask_estimator_final_backward_packed(gout, h, pre, w_all, dims, input_activation="tanh")
    npw, off = [], 0
    for d in dims:
        npw.append(to_np(w_all[off : off + 2 * d * hidden]).reshape(2 * d, hidden))
        off += 2 * d * hidden
    r_dz, r_db, r_dw = oracle.mask_estimator_final_backward(to_np(gout), to_np(h), to_np(pre), npw, dims, dn,
                                                            input_act="tanh", grad_pre_dt=dn)
    assert_parity(dz, r_dz, dn, "dz", by_index(1))
    assert_parity(db, r_db, dn, "dbias", by_band(0, [2 * d for d in dims]))
    assert_parity(dw, np.concatenate([w.reshape(-1) for w in r_dw]), dn, "dW", by_band(0, [2 * d * hidden for d in dims]))
    dx0, _, _ = hip_ext.mask_estimator_final_backward_packed(gout, h, pre, w_all, dims)
    assert torch.allclose((dx0.float() * (1 - h.float() ** 2)), dz.float(), rtol=2e-2, atol=2e-2 * dz.abs().max().item())


@pytest.mark.parametrize("dtype,m,dim", [(torch.float32, 65, 64), (torch.bfloat16, 1032, 192)])
def test_fused_mask_mlp_autograd_vs_oracle(hip_ext, dtype, m, dim):
    """The whole depth-2 mask MLP through the autograd Function the patch layer uses."""
    from pymsst_amd.fused_roformer import _FusedMaskMLP

    dn = dt_name(dtype)
    dims = BSR_WIDTHS
    nb, hid = len(dims), 4 * dim
    g = torch.Generator().manual_seed(23)
    x = torch.randn(m, nb, dim, generator=g).to(dtype).cuda().requires_grad_()
    w1 = (torch.randn(nb, hid, dim, generator=g) / dim**0.5).to(dtype).cuda().requires_grad_()
    b1 = (0.1 * torch.randn(nb, hid, generator=g)).to(dtype).cuda().requires_grad_()
    w2s = [(torch.randn(2 * d, hid, generator=g) / hid**0.5).to(dtype) for d in dims]
    w2 = torch.cat([w.reshape(-1) for w in w2s]).cuda().requires_grad_()
    b2 = (0.1 * torch.randn(2 * sum(dims), generator=g)).to(dtype).cuda().requires_grad_()
    out = _FusedMaskMLP.apply(x, w1, b1, w2, b2, hip_ext, dims)
    npw2 = [to_np(w) for w in w2s]
    ref = oracle.mask_mlp_forward(to_np(x), to_np(w1), to_np(b1), npw2, to_np(b2), dims, dn)
    assert_parity(out, ref, dn, "mlp out", by_band(1, dims))
    gout = torch.randn(out.shape, generator=g).to(dtype).cuda()
    out.backward(gout)
    r = oracle.mask_mlp_backward(to_np(gout), to_np(x), to_np(w1), to_np(b1), npw2, to_np(b2), dims, dn)
    assert_parity(x.grad, r[0], dn, "dx", by_index(1))
    assert_parity(w1.grad, r[1], dn, "dW1", by_index(0))
    assert_parity(b1.grad, r[2], dn, "db1", by_index(0))
    assert_parity(w2.grad, np.concatenate([w.reshape(-1) for w in r[3]]), dn, "dW2",
                  by_band(0, [2 * d * hid for d in dims]))
    assert_parity(b2.grad, r[4], dn, "db2", by_band(0, [2 * d for d in dims]))

"""GPU parity: band split (per-band RMSNorm + Linear), ragged and equal-width group ops, fwd + bwd.

Cases: the reference's own ragged test (tests/test_training_smoke.py:512-571: widths
(3,5,2,7), M=5, O=4, seed 7, fp16) plus its other dtypes; the BS-RoFormer 62-band
layout at the cfg1 (M=130, dim 64) and cfg2 (M=1032, dim 192) shapes; mel-style
ragged widths; strided group views with and without bias; the saved-input
backward; and an empty batch.  Bars are those of ``conftest.py``.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_parity, by_band, by_index, dt_name, to_np

pytestmark = pytest.mark.gpu

BSR_WIDTHS = tuple([8] * 24 + [16] * 12 + [48] * 8 + [96] * 8 + [192] * 8 + [512, 516])


def _params(dim_inputs, o, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    gammas = [(1 + 0.1 * torch.randn(d, generator=g)).to(dtype).cuda() for d in dim_inputs]
    weights = [(torch.randn(o, d, generator=g) / d**0.5).to(dtype).cuda() for d in dim_inputs]
    biases = [(0.1 * torch.randn(o, generator=g)).to(dtype).cuda() for _ in dim_inputs]
    return gammas, weights, biases


def _offsets(dim_inputs):
    return torch.tensor(np.concatenate([[0], np.cumsum(dim_inputs)]), dtype=torch.long, device="cuda")


def _check_ragged(ext, dim_inputs, m, o, dtype, seed, x_scale=1.0):
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(m, sum(dim_inputs), generator=g) * x_scale).to(dtype).cuda()
    gammas, weights, biases = _params(dim_inputs, o, dtype, seed + 1)
    offs = _offsets(dim_inputs)
    out, normed, inv = ext.band_split_ragged_forward(x, gammas, weights, biases, list(dim_inputs), offs)
    npx = to_np(x)
    npg = [to_np(v) for v in gammas]
    npw = [to_np(v) for v in weights]
    npb = [to_np(v) for v in biases]
    r_out, r_normed, r_inv = oracle.band_split_ragged_forward(npx, npg, npw, npb, dim_inputs, dn)
    assert_parity(out, r_out, dn, "out", by_index(1))
    assert_parity(normed, r_normed, dn, "normed", by_band(1, dim_inputs))
    assert_parity(inv, r_inv, "f32", "inv_norm")
    dy = torch.randn(out.shape, generator=g).to(dtype).cuda()
    res = ext.band_split_ragged_backward(dy, normed, inv, gammas, weights, list(dim_inputs), offs)
    nb = len(dim_inputs)
    r_dx, r_dg, r_dw, r_db = oracle.band_split_ragged_backward(
        to_np(dy), to_np(normed), to_np(inv), npg, npw, dim_inputs, dn
    )
    assert_parity(res[0], r_dx, dn, "dx", by_band(1, dim_inputs))
    assert_parity(torch.cat(res[1 : 1 + nb]), np.concatenate(r_dg), dn, "dgamma", by_band(0, dim_inputs))
    for b in range(nb):
        assert res[1 + nb + b].shape == (o, dim_inputs[b])
    assert_parity(torch.cat([w.reshape(-1) for w in res[1 + nb : 1 + 2 * nb]]),
                  np.concatenate([w.reshape(-1) for w in r_dw]), dn, "dW", by_band(0, [o * d for d in dim_inputs]))
    assert_parity(torch.stack(res[1 + 2 * nb :]), np.stack(r_db), dn, "dbias", by_index(0))
    return x, gammas, weights, biases, out, inv, dy


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
def test_reference_ragged_case(hip_ext, dtype):
    _check_ragged(hip_ext, (3, 5, 2, 7), 5, 4, dtype, 7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bsr_layout_cfg1(hip_ext, dtype):
    # cfg1: B=2 x T=65 rows, dim 64, STFT-scale inputs
    _check_ragged(hip_ext, BSR_WIDTHS, 130, 64, dtype, 3, x_scale=0.05)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_bsr_layout_cfg2(hip_ext, dtype):
    # cfg2: B=4 x T=258 rows, dim 192
    _check_ragged(hip_ext, BSR_WIDTHS, 1032, 192, dtype, 5)


@pytest.mark.parametrize("o", [192, 512, 100])
def test_mel_style_widths(hip_ext, o):
    r = np.random.default_rng(8)
    widths = tuple(int(4 * w) for w in r.integers(6, 131, size=20))
    _check_ragged(hip_ext, widths, 97, o, torch.bfloat16, 9)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_odd_widths_long_rows(hip_ext, dtype):
    # odd widths take the scalar (non-4-aligned) loads and stores of every kernel; 777 rows
    r = np.random.default_rng(12)
    widths = tuple(int(w) for w in r.integers(1, 90, size=13))
    _check_ragged(hip_ext, widths, 777, 100, dtype, 13)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_long_rows_from_normed(hip_ext, dtype):
    # 2500 rows, 40 outputs (O % 8 == 0, one ragged 64-wide output tile), from normed
    _check_ragged(hip_ext, (4, 68, 200, 12), 2500, 40, dtype, 14)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("dims,m,o", [(BSR_WIDTHS, 300, 192), ((8, 64, 132, 4), 4500, 64)])
def test_saved_input_backward(hip_ext, dtype, dims, m, o):
    # 4500 rows: the 16-bit dW kernel stages inv for its rows in LDS windows of 2048 rows
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(21)
    x = (0.05 * torch.randn(m, sum(dims), generator=g)).to(dtype).cuda()
    gammas, weights, biases = _params(dims, o, dtype, 22)
    ga = torch.cat(gammas)
    wa = torch.cat([w.reshape(-1) for w in weights])
    ba = torch.cat(biases)
    out, normed, inv = hip_ext.band_split_ragged_forward_packed(x, ga, wa, ba, dims, write_normed=False)
    assert normed is None
    r_out, _, _ = oracle.band_split_ragged_forward(to_np(x), [to_np(v) for v in gammas],
                                                   [to_np(v) for v in weights], [to_np(v) for v in biases], dims, dn)
    assert_parity(out, r_out, dn, "out", by_index(1))
    dy = torch.randn(out.shape, generator=g).to(dtype).cuda()
    dx, dg, dw, db = hip_ext.band_split_ragged_backward_packed(dy, x, True, inv, ga, wa, dims, True)
    r_dx, r_dg, r_dw, r_db = oracle.band_split_ragged_backward_lean(
        to_np(dy), to_np(x), to_np(inv), [to_np(v) for v in gammas], [to_np(v) for v in weights], dims, dn
    )
    assert_parity(dx, r_dx, dn, "dx", by_band(1, dims))
    assert_parity(dg, np.concatenate(r_dg), dn, "dgamma", by_band(0, dims))
    assert_parity(dw, np.concatenate([w.reshape(-1) for w in r_dw]), dn, "dW", by_band(0, [o * d for d in dims]))
    assert_parity(db, np.concatenate(r_db), dn, "dbias", by_band(0, [o] * len(dims)))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dims,m,o,has_bias", [((3, 5, 2, 7), 5, 4, True), (BSR_WIDTHS, 1032, 192, True),
                                               (BSR_WIDTHS, 130, 64, False), ((12, 520, 36), 77, 100, True)])
def test_backward_from_input_and_normed(hip_ext, dtype, dims, m, o, has_bias):
    """Backward from the saved input and from normed (one block per 64-wide input chunk, the row dots
    added up in the finish pass); against the oracle."""
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(31)
    x = (0.05 * torch.randn(m, sum(dims), generator=g)).to(dtype).cuda()
    gammas, weights, biases = _params(dims, o, dtype, 32)
    ga = torch.cat(gammas)
    wa = torch.cat([w.reshape(-1) for w in weights])
    ba = torch.cat(biases) if has_bias else None
    out, normed, inv = hip_ext.band_split_ragged_forward_packed(x, ga, wa, ba, dims, write_normed=True)
    dy = torch.randn(out.shape, generator=g).to(dtype).cuda()
    r_dx, r_dg, r_dw, r_db = oracle.band_split_ragged_backward_lean(
        to_np(dy), to_np(x), to_np(inv), [to_np(v) for v in gammas], [to_np(v) for v in weights], dims, dn
    )
    for saved, is_input in ((x, True), (normed, False)):
        dx, dg, dw, db = hip_ext.band_split_ragged_backward_packed(dy, saved, is_input, inv, ga, wa, dims, has_bias)
        tag = "x" if is_input else "normed"
        assert_parity(dx, r_dx, dn, f"dx from {tag}", by_band(1, dims))
        assert_parity(dg, np.concatenate(r_dg), dn, f"dgamma from {tag}", by_band(0, dims))
        assert_parity(dw, np.concatenate([w.reshape(-1) for w in r_dw]), dn, f"dW from {tag}",
                      by_band(0, [o * d for d in dims]))
        if has_bias:
            assert_parity(db, np.concatenate(r_db), dn, f"dbias from {tag}", by_band(0, [o] * len(dims)))


@pytest.mark.parametrize("has_bias", [True, False])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_group_view(hip_ext, has_bias, dtype):
    """fused_roformer.py:859-873: x[..., start:end].reshape(-1, G, I) is a strided view of the full row."""
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(31)
    full = torch.randn(2, 33, 4100, generator=g).to(dtype).cuda()
    start, gcount, width = 3584 - 8 * 192, 8, 192
    xv = full[..., start : start + gcount * width].reshape(-1, gcount, width)
    assert not xv.is_contiguous()
    gamma = (1 + 0.1 * torch.randn(gcount, width, generator=g)).to(dtype).cuda()
    weight = (torch.randn(gcount, 64, width, generator=g) / width**0.5).to(dtype).cuda()
    bias = (0.1 * torch.randn(gcount, 64, generator=g)).to(dtype).cuda() if has_bias else None
    out, normed, inv = hip_ext.band_split_forward(xv, gamma, weight, bias)
    r_out, r_normed, r_inv = oracle.band_split_forward(to_np(xv), to_np(gamma), to_np(weight),
                                                       to_np(bias) if has_bias else None, dn)
    assert_parity(out, r_out, dn, "out")
    assert_parity(normed, r_normed, dn, "normed")
    dy = torch.randn(out.shape, generator=g).to(dtype).cuda()
    for fn in (hip_ext.band_split_backward, hip_ext.band_split_backward_v2, hip_ext.band_split_backward_v3):
        dx, dgm, dw, db = fn(dy, normed, inv, gamma, weight, has_bias)
        r = oracle.band_split_backward(to_np(dy), to_np(normed), to_np(inv), to_np(gamma), to_np(weight), has_bias,
                                       dn)
        assert_parity(dx, r[0], dn, "dx")
        assert_parity(dgm, r[1], dn, "dgamma")
        assert_parity(dw, r[2], dn, "dW")
        if has_bias:
            assert_parity(db, r[3], dn, "db")
        else:
            assert db is None


def test_ragged_equals_groups_bitwise(hip_ext):
    """The ragged op and the equal-width group ops run the same kernel: results are bit-identical."""
    dims = BSR_WIDTHS
    g = torch.Generator().manual_seed(41)
    x = torch.randn(64, sum(dims), generator=g).cuda()
    gammas, weights, biases = _params(dims, 64, torch.float32, 42)
    out, normed, inv = hip_ext.band_split_ragged_forward(x, gammas, weights, biases, list(dims), _offsets(dims))
    start = 0
    for gstart, gend, width in ((0, 24, 8), (24, 36, 16), (36, 44, 48), (44, 52, 96), (52, 60, 192)):
        xv = x[:, start : start + (gend - gstart) * width].reshape(-1, gend - gstart, width)
        o2, n2, i2 = hip_ext.band_split_forward(
            xv, torch.stack(gammas[gstart:gend]), torch.stack(weights[gstart:gend]), torch.stack(biases[gstart:gend])
        )
        assert torch.equal(o2, out[:, gstart:gend])
        assert torch.equal(i2, inv[:, gstart:gend])
        start += (gend - gstart) * width


def test_empty_batch(hip_ext):
    dims = (8, 16)
    x = torch.empty(0, 24, device="cuda")
    gammas, weights, biases = _params(dims, 64, torch.float32, 1)
    out, normed, inv = hip_ext.band_split_ragged_forward(x, gammas, weights, biases, list(dims), _offsets(dims))
    assert out.shape == (0, 2, 64)
    res = hip_ext.band_split_ragged_backward(out, normed, inv, gammas, weights, list(dims), _offsets(dims))
    assert res[0].shape == (0, 24)
    assert all(torch.count_nonzero(t).item() == 0 for t in res[1:])


def test_rejects_bad_args(hip_ext):
    dims = (8, 16)
    gammas, weights, biases = _params(dims, 64, torch.float32, 1)
    x = torch.randn(4, 25, device="cuda")
    with pytest.raises(RuntimeError, match="x total dimension must match dim_inputs"):
        hip_ext.band_split_ragged_forward(x, gammas, weights, biases, list(dims), _offsets(dims))
    with pytest.raises(RuntimeError, match="gamma dtype must match x"):
        hip_ext.band_split_ragged_forward(x[:, :24].contiguous(), [g.half() for g in gammas], weights, biases,
                                          list(dims), _offsets(dims))

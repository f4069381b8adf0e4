"""GPU parity at the full kernel shapes of configs[4] (BS-RoFormer dim 512, hidden 2048, M = 1896) and
at the real 60-band Mel layout of configs[3] (F = 7916, M = 2760), against the float64 oracle.

configs[4] (B = 2, T = 948, 62 bands, 8 heads x 64):
* band split at O = 512 over the 62 bands, forward without the normed copy and the saved-input
  backward (the path the training step runs);
* the mask-MLP hidden layer: grouped linear 512 -> 2048 + tanh over 62 groups, and its backward;
* the mask final layer at H = 2048 (8-wave dx blocks) with the tanh input of the hidden layer;
* the fused qkv rotary at [124, 948, 8, 64] (time attention) and [1896, 62, 8, 64] (band attention);
* the attention output gate at D = 512 on 117,552 rows; RMSNorm at D = 512 on 117,552 rows.

band split and mask final on the 60 Slaney mel bands (38 widths, 24 to 520 features).

Each case runs in bf16 and fp32 (the bars of ``conftest.py``).  The band-split case with a bias that
dominates the output checks that the normalisation backward does not depend on the bias (its row
dots come from the fp32 gs, not from the stored output).  Inputs are seeded; the oracle runs on
the host.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from tests.conftest import assert_parity, by_band, by_index, dt_name, to_np

pytestmark = pytest.mark.gpu

BSR_WIDTHS = tuple([8] * 24 + [16] * 12 + [48] * 8 + [96] * 8 + [192] * 8 + [512, 516])
DTYPES = [torch.bfloat16, torch.float32]


def _mel_widths():
    from pymsst_amd.core.mel_band_roformer import mel_band_bins

    return tuple(4 * len(b) for b in mel_band_bins(44100, 2048, 60))


def _rand(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (scale * torch.randn(shape, generator=g)).to(dtype).cuda()


def _band_split_case(ext, widths, m, o, dtype, seed, bias_scale=0.1):
    """Packed forward (no normed copy) and the saved-input backward (the training path)."""
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(seed)
    F = sum(widths)
    x = (0.05 * torch.randn(m, F, generator=g)).to(dtype).cuda()
    gammas = [(1 + 0.1 * torch.randn(d, generator=g)).to(dtype) for d in widths]
    weights = [(torch.randn(o, d, generator=g) / d**0.5).to(dtype) for d in widths]
    biases = [(bias_scale * torch.randn(o, generator=g)).to(dtype) for _ in widths]
    ga = torch.cat(gammas).cuda()
    wa = torch.cat([w.reshape(-1) for w in weights]).cuda()
    ba = torch.cat(biases).cuda()
    out, normed, inv = ext.band_split_ragged_forward_packed(x, ga, wa, ba, widths, write_normed=False)
    assert normed is None
    npg = [to_np(v) for v in gammas]
    npw = [to_np(v) for v in weights]
    r_out, _, r_inv = oracle.band_split_ragged_forward(to_np(x), npg, npw, [to_np(v) for v in biases], widths, dn)
    assert_parity(out, r_out, dn, "out", by_index(1))
    assert_parity(inv, r_inv, "f32", "inv_norm")
    dy = torch.randn(out.shape, generator=g).to(dtype).cuda()
    dx, dg, dw, db = ext.band_split_ragged_backward_packed(dy, x, True, inv, ga, wa, widths, True)
    r_dx, r_dg, r_dw, r_db = oracle.band_split_ragged_backward_lean(to_np(dy), to_np(x), to_np(inv), npg, npw,
                                                                   widths, dn)
    assert_parity(dx, r_dx, dn, "dx", by_band(1, widths))
    assert_parity(dg, np.concatenate(r_dg), dn, "dgamma", by_band(0, widths))
    assert_parity(dw, np.concatenate([w.reshape(-1) for w in r_dw]), dn, "dW", by_band(0, [o * d for d in widths]))
    assert_parity(db, np.concatenate(r_db), dn, "dbias", by_band(0, [o] * len(widths)))


@pytest.mark.parametrize("dtype", DTYPES)
def test_band_split_configs4(hip_ext, dtype):
    _band_split_case(hip_ext, BSR_WIDTHS, 1896, 512, dtype, 101)


@pytest.mark.parametrize("dtype", DTYPES)
def test_band_split_mel_configs3(hip_ext, dtype):
    _band_split_case(hip_ext, _mel_widths(), 2760, 192, dtype, 102)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_band_split_bias_dominates_output(hip_ext, dtype):
    """A bias several times the scale of (n * gamma) W^T: a backward that took its row dots from the
    stored 16-bit output minus the bias would lose them to cancellation here."""
    _band_split_case(hip_ext, BSR_WIDTHS, 1032, 192, dtype, 103, bias_scale=6.0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_grouped_linear_tanh_configs4(hip_ext, dtype):
    """Mask-MLP hidden layer at configs[4]: 62 groups, 512 -> 2048, tanh epilogue, M = 1896."""
    dn = dt_name(dtype)
    m, nb, i, o = 1896, 62, 512, 2048
    x = _rand((m, nb, i), 111, 1.0, dtype)
    w = _rand((nb, o, i), 112, 1.0 / i**0.5, dtype)
    b = _rand((nb, o), 113, 0.1, dtype)
    h = hip_ext.grouped_linear_forward_act(x, w, b, activation="tanh")
    r_h = oracle.grouped_linear_forward(to_np(x), to_np(w), to_np(b), dn, act="tanh")
    assert_parity(h, r_h, dn, "hidden", by_index(1))
    dz = _rand((m, nb, o), 114, 1.0, dtype)
    dx, dw, db = hip_ext.grouped_linear_backward(dz, x, w, has_bias=True)
    r_dx, r_dw, r_db = oracle.grouped_linear_backward(to_np(dz), to_np(x), to_np(w), True, dn)
    assert_parity(dx, r_dx, dn, "dx", by_index(1))
    assert_parity(dw, r_dw, dn, "dW", by_index(0))
    assert_parity(db, r_db, dn, "dbias", by_index(0))


def _mask_final_case(ext, widths, m, hidden, dtype, seed, tanh_in):
    dn = dt_name(dtype)
    g = torch.Generator().manual_seed(seed)
    nb = len(widths)
    x = torch.randn(m, nb, hidden, generator=g)
    if tanh_in:
        x = torch.tanh(x)
    x = x.to(dtype).cuda()
    weights = [(torch.randn(2 * d, hidden, generator=g) / hidden**0.5).to(dtype) for d in widths]
    bias = (0.1 * torch.randn(2 * sum(widths), generator=g)).to(dtype).cuda()
    wa = torch.cat([w.reshape(-1) for w in weights]).cuda()
    out, pre = ext.mask_estimator_final_forward_packed(x, wa, bias, widths)
    npw = [to_np(w) for w in weights]
    r_out, r_pre = oracle.mask_estimator_final_forward(to_np(x), npw, to_np(bias), widths, dn)
    two = [2 * d for d in widths]
    assert_parity(out, r_out, dn, "out", by_band(1, widths))
    assert_parity(pre, r_pre, dn, "pre", by_band(1, two))
    gout = torch.randn(out.shape, generator=g).to(dtype).cuda()
    dx, db, dw = ext.mask_estimator_final_backward_packed(gout, x, pre, wa, widths,
                                                          input_activation="tanh" if tanh_in else None)
    r_dx, r_db, r_dw = oracle.mask_estimator_final_backward(to_np(gout), to_np(x), to_np(pre), npw, widths, dn,
                                                            input_act="tanh" if tanh_in else None, grad_pre_dt=dn)
    assert_parity(dx, r_dx, dn, "dx", by_index(1))
    assert_parity(db, r_db, dn, "dbias", by_band(0, two))
    assert_parity(dw, np.concatenate([w.reshape(-1) for w in r_dw]), dn, "dW", by_band(0, [t * hidden for t in two]))


@pytest.mark.parametrize("dtype", DTYPES)
def test_mask_final_configs4(hip_ext, dtype):
    _mask_final_case(hip_ext, BSR_WIDTHS, 1896, 2048, dtype, 121, tanh_in=True)


@pytest.mark.parametrize("dtype", DTYPES)
def test_mask_final_mel_configs3(hip_ext, dtype):
    _mask_final_case(hip_ext, _mel_widths(), 2760, 768, dtype, 122, tanh_in=True)


def _tables(n, d, dtype):
    c, s = oracle.rotary_tables(n, d)
    c = torch.from_numpy(c).to(dtype).cuda().repeat_interleave(2, dim=-1).reshape(1, n, 1, d)[..., ::2]
    s = torch.from_numpy(s).to(dtype).cuda().repeat_interleave(2, dim=-1).reshape(1, n, 1, d)[..., ::2]
    return c, s


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(124, 948, 8, 64), (1896, 62, 8, 64)])
def test_rotary_qkv_configs4(hip_ext, dtype, shape):
    dn = dt_name(dtype)
    b, n, h, d = shape
    qkv = _rand((b, n, 3 * h * d), 131, 1.0, dtype)
    cos, sin = _tables(n, d, dtype)
    cn, sn = to_np(cos).reshape(n, d // 2), to_np(sin).reshape(n, d // 2)
    q, k, v = hip_ext.rotary_qkv_forward(qkv, h, cos, sin)
    parts = qkv.view(b, n, 3, h, d).unbind(2)
    assert_parity(q, oracle.rotary_forward(to_np(parts[0]), cn, sn, dn), dn, "q")
    assert_parity(k, oracle.rotary_forward(to_np(parts[1]), cn, sn, dn), dn, "k")
    assert torch.equal(v, parts[2])
    del q, k, v
    gq, gk, gv = (_rand((b, h, n, d), 132 + i, 1.0, dtype).transpose(1, 2) for i in range(3))
    dqkv = hip_ext.rotary_qkv_backward(gq, gk, gv, cos, sin)
    dparts = dqkv.view(b, n, 3, h, d).unbind(2)
    assert_parity(dparts[0], oracle.rotary_backward(to_np(gq), cn, sn, dn), dn, "dq")
    assert_parity(dparts[1], oracle.rotary_backward(to_np(gk), cn, sn, dn), dn, "dk")
    assert torch.equal(dparts[2], gv)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(124, 948), (1896, 62)])
def test_attention_gate_configs4(hip_ext, dtype, shape):
    """Gate on the transposed SDPA output ([B, H, N, Dh] memory) at D = 512, 117,552 rows."""
    dn = dt_name(dtype)
    b, n = shape
    h, dh, dim = 8, 64, 512
    attn = _rand((b, h, n, dh), 141, 1.0, dtype).transpose(1, 2)
    x = _rand((b * n, dim), 142, 1.0, dtype)
    w = _rand((h, dim), 143, 1.0 / dim**0.5, dtype)
    bias = _rand((h,), 144, 0.5, dtype)
    out, gate = hip_ext.attention_gate_forward_bnhd(attn, x, w, bias)[:2]
    a3 = to_np(attn).reshape(b * n, h, dh)
    r_out, r_gate = oracle.attention_gate_forward(a3, to_np(x), to_np(w), to_np(bias), dn)
    assert_parity(gate, r_gate, dn, "gate")
    assert_parity(out, r_out, dn, "out")
    gout = _rand((b * n, h * dh), 145, 1.0, dtype)
    ga, gx, gw, gb = hip_ext.attention_gate_backward_bnhd(gout, attn, x, w, gate)
    r = oracle.attention_gate_backward(to_np(gout), a3, to_np(x), to_np(w), to_np(gate), dn)
    assert_parity(ga.reshape(b * n, h, dh), r[0], dn, "grad_attn")
    assert_parity(gx, r[1], dn, "grad_x")
    assert_parity(gw, r[2], dn, "grad_weight")
    assert_parity(gb, r[3], dn, "grad_bias")


@pytest.mark.parametrize("dtype", DTYPES)
def test_rms_norm_configs4(hip_ext, dtype):
    """The axial blocks' RMSNorm at D = 512 on M * 62 = 117,552 rows, fp32 gamma ("fast" mode), with the
    saved-input backward."""
    dn = dt_name(dtype)
    rows, dim = 1896 * 62, 512
    x = _rand((rows, dim), 151, 1.0, dtype)
    gamma = 1 + _rand((dim,), 152, 0.1)
    out, inv = hip_ext.rms_norm_forward_lean(x, gamma)
    r_out, _, r_inv = oracle.rms_norm_forward(to_np(x), to_np(gamma), dn, "fp32_gamma")
    assert_parity(out, r_out, dn, "out")
    assert_parity(inv, r_inv, "f32", "inv_norm")
    dy = _rand((rows, dim), 153, 1.0, dtype)
    dx, dg = hip_ext.rms_norm_backward_from_input(dy, x, inv, gamma)
    r_dx, r_dg = oracle.rms_norm_backward_lean(to_np(dy), to_np(x), to_np(inv), to_np(gamma), dn, "f32")
    assert_parity(dx, r_dx, dn, "dx")
    assert_parity(dg, r_dg, "f32", "dgamma")

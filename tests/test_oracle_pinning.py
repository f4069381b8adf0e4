"""Pin the float64 oracle (``oracle/``) against independent computations (CPU only).

Each oracle function is compared with torch float64 autograd of the closed-form
module (``tests/torch_reference.py``), with complex multiplication, with
invariants, and at the reference tests' own seeded shapes.  A planted-mistake
test shows the checks fail when a term of the hand-derived backward is dropped.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from oracle import round_to
from tests import torch_reference as tr

TOL = 1e-10  # float64 vs float64


def _t(a, grad=False):
    return torch.tensor(np.asarray(a), dtype=torch.float64, requires_grad=grad)


def _rng(seed):
    return np.random.default_rng(seed)


def _close(a, b, tol=TOL, what=""):
    a = np.asarray(a, dtype=np.float64)
    b = b.detach().numpy() if isinstance(b, torch.Tensor) else np.asarray(b, dtype=np.float64)
    scale = max(1.0, float(np.max(np.abs(b))) if b.size else 1.0)
    err = float(np.max(np.abs(a - b))) if a.size else 0.0
    assert err <= tol * scale, f"{what}: {err:.3e}"


# ------------------------------------------------------------------ RMSNorm


@pytest.mark.parametrize("rows,dim", [(7, 64), (5, 192), (3, 5), (1, 1)])
def test_rms_norm_forward_backward_vs_autograd(rows, dim):
    r = _rng(rows * 1000 + dim)
    x = r.standard_normal((rows, dim))
    x[0] *= 1e-3
    gamma = 1 + 0.1 * r.standard_normal(dim)
    dy = r.standard_normal((rows, dim))
    out, normed, inv = oracle.rms_norm_forward(x, gamma, "f64")
    tx, tg = _t(x, True), _t(gamma, True)
    ref = tr.rms_norm(tx, tg)
    _close(out, ref, what="out")
    ref.backward(_t(dy))
    dx, dg = oracle.rms_norm_backward(dy, normed, inv, gamma, "f64")
    _close(dx, tx.grad, what="dx")
    _close(dg, tg.grad, what="dgamma")
    # saved-input variant
    dx2, dg2 = oracle.rms_norm_backward_lean(dy, x, inv, gamma, "f64")
    _close(dx2, tx.grad, what="lean dx")
    _close(dg2, tg.grad, what="lean dgamma")


def test_rms_norm_invariants_and_zero_row():
    r = _rng(3)
    x = r.standard_normal((6, 32))
    x[2] = 0.0
    gamma = np.ones(32)
    out, normed, inv = oracle.rms_norm_forward(x, gamma, "f64")
    norms = np.linalg.norm(normed, axis=-1)
    assert np.allclose(np.delete(norms, 2), math.sqrt(32), rtol=1e-12)
    assert np.all(normed[2] == 0) and inv[2] == 1e12
    # scale invariance f(alpha x) = f(x)
    out2, _, _ = oracle.rms_norm_forward(3.7 * x, gamma, "f64")
    assert np.allclose(out, out2, atol=1e-12)
    # zero-row backward: dx = inv * dy * gamma * sqrt(D)  (autograd of F.normalize's eps clamp)
    dy = r.standard_normal((6, 32))
    tx, tg = _t(x, True), _t(gamma, True)
    tr.rms_norm(tx, tg).backward(_t(dy))
    dx, _ = oracle.rms_norm_backward(dy, normed, inv, gamma, "f64")
    rel = np.max(np.abs(dx[2] - tx.grad[2].numpy())) / np.max(np.abs(tx.grad[2].numpy()))
    assert rel < 1e-6


def test_rms_norm_mode_dtypes():
    r = _rng(4)
    x = oracle.round_to(r.standard_normal((4, 16)), "bf16")
    gamma = 1 + 0.1 * r.standard_normal(16)
    out, normed, _ = oracle.rms_norm_forward(x, gamma, "bf16", "mixed")
    # mixed writes fp32, so it keeps more precision than bf16 rounding
    assert np.any(oracle.round_to(out, "bf16") != out)
    outb, _, _ = oracle.rms_norm_forward(x, gamma, "bf16", "fp32_gamma")
    assert np.all(oracle.round_to(outb, "bf16") == outb)


def test_planted_mistake_in_oracle_backward_is_caught(monkeypatch):
    """Drop the projection term of the RMSNorm backward: the autograd check must fail."""
    r = _rng(5)
    x = r.standard_normal((4, 16))
    gamma = 1 + 0.1 * r.standard_normal(16)
    dy = r.standard_normal((4, 16))
    _, normed, inv = oracle.rms_norm_forward(x, gamma, "f64")

    def broken(grad_out, normed, inv_norm, gamma, dt, mode="plain", acc=np.float64):
        scale = math.sqrt(grad_out.shape[-1])
        dx = inv_norm[:, None] * (grad_out * gamma * scale)  # missing "- n * dot / scale"
        return dx, np.sum(grad_out * normed, axis=0)

    tx, tg = _t(x, True), _t(gamma, True)
    tr.rms_norm(tx, tg).backward(_t(dy))
    dx_bad, _ = broken(dy, normed, inv, gamma, "f64")
    with pytest.raises(AssertionError):
        _close(dx_bad, tx.grad, what="planted")


# ------------------------------------------------------------------ rotary


@pytest.mark.parametrize("shape", [(2, 5, 3, 8), (1, 65, 4, 32), (1, 3, 1, 2)])
def test_rotary_vs_complex_multiply_and_autograd(shape):
    b, n, h, d = shape
    r = _rng(n * d)
    t = r.standard_normal(shape)
    cos, sin = oracle.rotary_tables(n, d)
    out = oracle.rotary_forward(t, cos, sin, "f64")
    tt = _t(t, True)
    ref = tr.rotary(tt, _t(cos), _t(sin))
    _close(out, ref, what="fwd")
    g = r.standard_normal(shape)
    ref.backward(_t(g))
    _close(oracle.rotary_backward(g, cos, sin, "f64"), tt.grad, what="bwd")


def test_rotary_tables_and_relative_position():
    n, d = 16, 8
    cos, sin = oracle.rotary_tables(n, d, theta=10000.0)
    # closed form: angle(n, p) = n * 10000^(-2p/d)
    ang = np.arange(n)[:, None] * (10000.0 ** (-np.arange(0, d, 2) / d))[None, :]
    assert np.allclose(cos, np.cos(ang)) and np.allclose(sin, np.sin(ang))
    # q(m).k(n) depends only on m - n
    r = _rng(9)
    q = r.standard_normal(d)
    k = r.standard_normal(d)
    qs = oracle.rotary_forward(np.tile(q, (1, n, 1, 1)), cos, sin, "f64")[0, :, 0]
    ks = oracle.rotary_forward(np.tile(k, (1, n, 1, 1)), cos, sin, "f64")[0, :, 0]
    dots = qs @ ks.T
    for delta in range(-3, 4):
        diag = np.diagonal(dots, offset=delta)
        assert np.allclose(diag, diag[0], atol=1e-10)
    # norm preservation
    assert np.allclose(np.linalg.norm(qs, axis=-1), np.linalg.norm(q))


@pytest.mark.parametrize("shape", [(2, 5, 3, 8), (1, 9, 2, 64)])
def test_rms_norm_rotary_vs_autograd(shape):
    b, n, h, d = shape
    r = _rng(d + n)
    x = r.standard_normal(shape)
    x[0, 0, 0] = 0.0
    gamma = 1 + 0.1 * r.standard_normal(d)
    cos, sin = oracle.rotary_tables(n, d)
    out, inv = oracle.rms_norm_rotary_forward(x, gamma, cos, sin, "f64")
    tx, tg = _t(x, True), _t(gamma, True)
    ref = tr.rotary(tr.rms_norm(tx, tg), _t(cos), _t(sin))
    _close(out, ref, what="fwd")
    g = r.standard_normal(shape)
    ref.backward(_t(g))
    dx, dg = oracle.rms_norm_rotary_backward(g, x, inv, gamma, cos, sin, "f64", "f64")
    keep = np.ones(shape, bool)
    keep[0, 0, 0] = False
    _close(dx[keep], tx.grad.numpy()[keep], what="dx")
    _close(dg, tg.grad, what="dgamma")


# ------------------------------------------------------------------ band split


@pytest.mark.parametrize("m,g,i,o,bias", [(5, 3, 8, 4, True), (4, 2, 16, 6, False), (3, 1, 7, 5, True)])
def test_band_split_group_vs_autograd(m, g, i, o, bias):
    r = _rng(m * g * i * o)
    x = r.standard_normal((m, g, i))
    gamma = 1 + 0.1 * r.standard_normal((g, i))
    w = r.standard_normal((g, o, i)) / math.sqrt(i)
    b = r.standard_normal((g, o)) if bias else None
    out, normed, inv = oracle.band_split_forward(x, gamma, w, b, "f64")
    tx, tg, tw = _t(x, True), _t(gamma, True), _t(w, True)
    tb = _t(b, True) if bias else None
    ref = tr.band_split_group(tx, tg, tw, tb)
    _close(out, ref, what="out")
    dy = r.standard_normal((m, g, o))
    ref.backward(_t(dy))
    dx, dg, dw, db = oracle.band_split_backward(dy, normed, inv, gamma, w, bias, "f64")
    _close(dx, tx.grad, what="dx")
    _close(dg, tg.grad, what="dgamma")
    _close(dw, tw.grad, what="dW")
    if bias:
        _close(db, tb.grad, what="db")
    else:
        assert db is None


@pytest.mark.parametrize("dim_inputs,m,o,seed", [((3, 5, 2, 7), 5, 4, 7), ((8, 8, 16, 48), 6, 12, 1)])
def test_band_split_ragged_vs_autograd(dim_inputs, m, o, seed):
    """Widths/seed of the reference's ragged test (tests/test_training_smoke.py:512-571)."""
    r = _rng(seed)
    x = r.standard_normal((m, sum(dim_inputs)))
    gammas = [1 + 0.1 * r.standard_normal(d) for d in dim_inputs]
    weights = [r.standard_normal((o, d)) for d in dim_inputs]
    biases = [r.standard_normal(o) for _ in dim_inputs]
    out, normed, inv = oracle.band_split_ragged_forward(x, gammas, weights, biases, dim_inputs, "f64")
    tx = _t(x, True)
    tg = [_t(v, True) for v in gammas]
    tw = [_t(v, True) for v in weights]
    tb = [_t(v, True) for v in biases]
    ref = tr.band_split_ragged(tx, tg, tw, tb, dim_inputs)
    _close(out, ref, what="out")
    dy = r.standard_normal((m, len(dim_inputs), o))
    ref.backward(_t(dy))
    dx, dgs, dws, dbs = oracle.band_split_ragged_backward(dy, normed, inv, gammas, weights, dim_inputs, "f64")
    _close(dx, tx.grad, what="dx")
    for k in range(len(dim_inputs)):
        _close(dgs[k], tg[k].grad, what=f"dgamma{k}")
        _close(dws[k], tw[k].grad, what=f"dW{k}")
        _close(dbs[k], tb[k].grad, what=f"db{k}")
    dx2, dgs2, dws2, dbs2 = oracle.band_split_ragged_backward_lean(dy, x, inv, gammas, weights, dim_inputs, "f64")
    _close(dx2, tx.grad, what="lean dx")
    # ragged == concatenation of single-band group results (the reference asserts this kernel vs kernel)
    off = np.cumsum((0,) + tuple(dim_inputs))
    for k, d in enumerate(dim_inputs):
        ob, _, _ = oracle.band_split_forward(
            x[:, None, off[k] : off[k + 1]], gammas[k][None], weights[k][None], biases[k][None], "f64"
        )
        _close(out[:, k], ob[:, 0], what="ragged==group")


@pytest.mark.parametrize("dt,tdt", [("bf16", torch.bfloat16), ("f16", torch.float16)])
@pytest.mark.parametrize("dim_inputs,m,o,seed", [((3, 5, 2, 7), 5, 4, 7), ((8, 8, 16, 48), 6, 12, 1)])
def test_band_split_mixed_vs_autocast_autograd(dim_inputs, m, o, seed, dt, tdt):
    """The fp32-input band split with a 16-bit projection against torch float64 autograd of the stock
    module under autocast (RMSNorm in fp32, nn.Linear on 16-bit operands), where the rounding of the
    projection's input and of its input gradient comes from the casts' autograd, not from the oracle's
    formula.  A backward that skips the rounding of the Linear's input gradient is caught."""
    r = _rng(seed)
    x = round_to(0.05 * r.standard_normal((m, sum(dim_inputs))), "f32")
    x[0, : dim_inputs[0]] = 0.0  # a zero band row: inv = 1e12
    gammas = [round_to(1 + 0.1 * r.standard_normal(d), "f32") for d in dim_inputs]
    weights = [round_to(r.standard_normal((o, d)) / math.sqrt(d), dt) for d in dim_inputs]
    biases = [round_to(0.1 * r.standard_normal(o), dt) for _ in dim_inputs]
    out, feats, inv = oracle.band_split_mixed_forward(x, gammas, weights, biases, dim_inputs, dt)
    tx = _t(x, True)
    tg = [_t(v, True) for v in gammas]
    tw = [_t(v, True) for v in weights]
    tb = [_t(v, True) for v in biases]
    ref = tr.band_split_ragged_autocast(tx, tg, tw, tb, dim_inputs, tdt)
    eps16 = 2.0**-8 if dt == "bf16" else 2.0**-11
    # the only difference is fp32 (oracle) vs float64 (reference) rounding before the 16-bit roundings
    mism = np.abs(out - ref.detach().numpy()) > 1e-12
    assert mism.mean() < 0.02, mism.mean()
    _close(out, ref, tol=2 * eps16, what="out")
    dy = round_to(r.standard_normal((m, len(dim_inputs), o)), dt)
    ref.backward(_t(dy))
    dx, dgs, dws, dbs = oracle.band_split_mixed_backward(dy, x, feats, inv, gammas, weights, dim_inputs, dt)
    _close(dx, tx.grad, tol=1e-5, what="dx")
    off = np.cumsum((0,) + tuple(dim_inputs))
    for k in range(len(dim_inputs)):
        _close(dgs[k], tg[k].grad, tol=1e-5, what=f"dgamma{k}")
        _close(dws[k], tw[k].grad, tol=eps16, what=f"dW{k}")
        _close(dbs[k], tb[k].grad, tol=eps16, what=f"db{k}")
    # planted mistake: the Linear's input gradient left unrounded moves dx past the bar
    n_all = np.concatenate([x[:, off[k]:off[k + 1]] * inv[:, k:k + 1] * math.sqrt(d)
                            for k, d in enumerate(dim_inputs)], axis=1)
    bad = []
    for k, d in enumerate(dim_inputs):
        g = dy[:, k] @ weights[k]  # not rounded
        gn = g * gammas[k][None]
        nk = n_all[:, off[k]:off[k + 1]]
        dot = np.sum(gn * nk, axis=-1, keepdims=True)
        bad.append(inv[:, k:k + 1] * (gn * math.sqrt(d) - nk * dot / math.sqrt(d)))
    with pytest.raises(AssertionError):
        _close(np.concatenate(bad, axis=1), tx.grad, tol=1e-5, what="planted")


def test_mask_final_direct_mode_rounding_points():
    """The direct mode (.cu:2585-2704) and the grouped mode (.cu:2312-2367) share dbias (fp32 sums of the
    unrounded dpre) and dW (from the dpre stored in the tensor dtype); only dx differs: the direct mode
    multiplies the unrounded dpre, the grouped mode the stored one."""
    r = _rng(41)
    dims = (3, 8, 5)
    m, h = 7, 16
    x = round_to(r.standard_normal((m, len(dims), h)), "bf16")
    w = [round_to(r.standard_normal((2 * d, h)) / 4, "bf16") for d in dims]
    pre = round_to(r.standard_normal((m, 2 * sum(dims))), "bf16")
    g = round_to(r.standard_normal((m, sum(dims))), "bf16")
    dx_d, db_d, dw_d = oracle.mask_estimator_final_backward(g, x, pre, w, dims, "bf16")
    dx_g, db_g, dw_g = oracle.mask_estimator_final_backward(g, x, pre, w, dims, "bf16", grad_pre_dt="bf16")
    assert np.array_equal(db_d, db_g)
    assert all(np.array_equal(a, b) for a, b in zip(dw_d, dw_g))
    assert not np.array_equal(dx_d, dx_g)
    # the direct dx is the unrounded product: the f64 oracle (no rounding anywhere) rounded once
    dx_exact, _, _ = oracle.mask_estimator_final_backward(g, x, pre, w, dims, "f64")
    assert np.array_equal(dx_d, round_to(dx_exact, "bf16"))


# ------------------------------------------------------------------ grouped linear / mask estimator


def test_grouped_linear_vs_bmm_reference():
    r = _rng(12)
    x = r.standard_normal((2, 5, 3, 4))
    w = r.standard_normal((3, 6, 4))
    b = r.standard_normal((3, 6))
    out = oracle.grouped_linear_forward(x.reshape(-1, 3, 4), w, b, "f64")
    tx, tw, tb = _t(x, True), _t(w, True), _t(b, True)
    ref = tr.grouped_linear(tx, tw, tb)
    _close(out, ref.reshape(-1, 3, 6), what="fwd")
    dy = r.standard_normal((2, 5, 3, 6))
    ref.backward(_t(dy))
    dx, dw, db = oracle.grouped_linear_backward(dy.reshape(-1, 3, 6), x.reshape(-1, 3, 4), w, True, "f64")
    _close(dx, tx.grad.reshape(-1, 3, 4), what="dx")
    _close(dw, tw.grad, what="dW")
    _close(db, tb.grad, what="db")


def test_mask_final_vs_linear_glu_reference_shapes():
    """Seed/shapes of tests/test_training_smoke.py:574-615: M=4, NB=5, hidden 16, widths (3,4,2,5,6)."""
    r = _rng(11)
    dim_inputs = (3, 4, 2, 5, 6)
    m, nb, hid = 4, 5, 16
    x = r.standard_normal((m, nb, hid))
    weights = [r.standard_normal((2 * d, hid)) for d in dim_inputs]
    bias = r.standard_normal(2 * sum(dim_inputs))
    out, pre = oracle.mask_estimator_final_forward(x, weights, bias, dim_inputs, "f64")
    tx, tb = _t(x, True), _t(bias, True)
    tw = [_t(w, True) for w in weights]
    ref = tr.mask_final(tx, tw, tb, dim_inputs)
    _close(out, ref, what="out")
    g = r.standard_normal((m, sum(dim_inputs)))
    ref.backward(_t(g))
    dx, dbias, dws = oracle.mask_estimator_final_backward(g, x, pre, weights, dim_inputs, "f64")
    _close(dx, tx.grad, what="dx")
    _close(dbias, tb.grad, what="dbias")
    for k in range(nb):
        _close(dws[k], tw[k].grad, what=f"dW{k}")


def test_mask_mlp_vs_autograd():
    r = _rng(13)
    dim_inputs = (8, 16, 4)
    m, nb, dim, hid = 6, 3, 12, 20
    x = r.standard_normal((m, nb, dim))
    w1 = r.standard_normal((nb, hid, dim)) / math.sqrt(dim)
    b1 = r.standard_normal((nb, hid))
    w2 = [r.standard_normal((2 * d, hid)) / math.sqrt(hid) for d in dim_inputs]
    b2 = r.standard_normal(2 * sum(dim_inputs))
    out = oracle.mask_mlp_forward(x, w1, b1, w2, b2, dim_inputs, "f64")
    tx, tw1, tb1, tb2 = _t(x, True), _t(w1, True), _t(b1, True), _t(b2, True)
    tw2 = [_t(w, True) for w in w2]
    ref = tr.mask_mlp(tx, tw1, tb1, tw2, tb2, dim_inputs)
    _close(out, ref, what="out")
    g = r.standard_normal((m, sum(dim_inputs)))
    ref.backward(_t(g))
    dx, dw1, db1, dw2, db2 = oracle.mask_mlp_backward(g, x, w1, b1, w2, b2, dim_inputs, "f64")
    _close(dx, tx.grad, what="dx")
    _close(dw1, tw1.grad, what="dW1")
    _close(db1, tb1.grad, what="db1")
    _close(db2, tb2.grad, what="db2")
    for k in range(nb):
        _close(dw2[k], tw2[k].grad, what=f"dW2_{k}")


def test_round_to_matches_torch_casts():
    r = _rng(14)
    a = r.standard_normal(10000) * 10 ** r.uniform(-6, 6, 10000)
    for name, dt in (("bf16", torch.bfloat16), ("f16", torch.float16), ("f32", torch.float32)):
        ref = torch.tensor(a, dtype=torch.float32).to(dt).double().numpy() if name != "f32" else a.astype(np.float32)
        got = oracle.round_to(a, name)
        if name == "f16":
            ref = a.astype(np.float32).astype(np.float16).astype(np.float64)
        assert np.array_equal(got, np.asarray(ref, dtype=np.float64)), name


def test_tanh_hidden_pieces_compose_to_mask_mlp_autograd():
    """The pieces the fused mask MLP runs (grouped linear + tanh epilogue, final layer, final
    backward with the tanh input, grouped-linear backward) chain to torch autograd of the MLP."""
    r = _rng(14)
    dim_inputs = (4, 8, 12, 4)
    m, nb, dim, hid = 5, 4, 6, 10
    x = r.standard_normal((m, nb, dim))
    w1 = r.standard_normal((nb, hid, dim)) / math.sqrt(dim)
    b1 = r.standard_normal((nb, hid))
    w2 = [r.standard_normal((2 * d, hid)) / math.sqrt(hid) for d in dim_inputs]
    b2 = r.standard_normal(2 * sum(dim_inputs))
    h = oracle.grouped_linear_forward(x, w1, b1, "f64", act="tanh")
    out, pre = oracle.mask_estimator_final_forward(h, w2, b2, dim_inputs, "f64")
    tx, tw1, tb1, tb2 = _t(x, True), _t(w1, True), _t(b1, True), _t(b2, True)
    tw2 = [_t(w, True) for w in w2]
    ref = tr.mask_mlp(tx, tw1, tb1, tw2, tb2, dim_inputs)
    _close(out, ref, what="out")
    g = r.standard_normal((m, sum(dim_inputs)))
    ref.backward(_t(g))
    dz, db2, dw2 = oracle.mask_estimator_final_backward(g, h, pre, w2, dim_inputs, "f64", input_act="tanh")
    dx, dw1, db1 = oracle.grouped_linear_backward(dz, x, w1, True, "f64")
    _close(dx, tx.grad, what="dx")
    _close(dw1, tw1.grad, what="dW1")
    _close(db1, tb1.grad, what="db1")
    _close(db2, tb2.grad, what="db2")
    for k in range(nb):
        _close(dw2[k], tw2[k].grad, what=f"dW2_{k}")
    # without the tanh factor the chain must fail (guards against a dropped 1 - h^2 term)
    dz_bad, _, _ = oracle.mask_estimator_final_backward(g, h, pre, w2, dim_inputs, "f64")
    dx_bad, _, _ = oracle.grouped_linear_backward(dz_bad, x, w1, True, "f64")
    assert np.max(np.abs(dx_bad - tx.grad.numpy())) > 1e-3


@pytest.mark.parametrize("m,h,dh,d", [(7, 8, 64, 192), (5, 4, 32, 64), (3, 3, 5, 7)])
def test_attention_gate_vs_autograd(m, h, dh, d):
    r = _rng(15)
    attn = r.standard_normal((m, h, dh))
    x = r.standard_normal((m, d))
    w = r.standard_normal((h, d)) / math.sqrt(d)
    b = r.standard_normal(h)
    out, gate = oracle.attention_gate_forward(attn, x, w, b, "f64")
    ta, tx, tw, tb = _t(attn, True), _t(x, True), _t(w, True), _t(b, True)
    ref = tr.attention_gate(ta, tx, tw, tb)
    _close(out, ref, what="out")
    g = r.standard_normal((m, h * dh))
    ref.backward(_t(g))
    ga, gx, gw, gb = oracle.attention_gate_backward(g, attn, x, w, gate, "f64")
    _close(ga, ta.grad, what="grad_attn")
    _close(gx, tx.grad, what="grad_x")
    _close(gw, tw.grad, what="grad_weight")
    _close(gb, tb.grad, what="grad_bias")


def test_attention_gate_rounding_points():
    """bf16: the stored gate (not the fp32 sigmoid) scales attn, and the stored gate
    pre-activation gradient feeds grad_x/grad_weight/grad_bias.  A planted variant that
    rounds only the outputs differs from the oracle on these inputs, so the check has teeth."""
    r = _rng(16)
    m, h, dh, d = 64, 8, 64, 192
    attn = oracle.round_to(r.standard_normal((m, h, dh)), "bf16")
    x = oracle.round_to(r.standard_normal((m, d)), "bf16")
    w = oracle.round_to(r.standard_normal((h, d)) / math.sqrt(d), "bf16")
    b = oracle.round_to(r.standard_normal(h), "bf16")
    out, gate = oracle.attention_gate_forward(attn, x, w, b, "bf16")
    # the stored gate is a bf16 value and out is exactly round(attn * gate)
    assert np.array_equal(gate, oracle.round_to(gate, "bf16"))
    assert np.array_equal(out, oracle.round_to((attn * gate[:, :, None]).reshape(m, -1), "bf16"))
    exact = oracle.sigmoid(x @ w.T + b)
    planted = oracle.round_to((attn * exact[:, :, None]).reshape(m, -1), "bf16")
    assert not np.array_equal(planted, out)
    g = oracle.round_to(r.standard_normal((m, h * dh)), "bf16")
    ga, gx, gw, gb = oracle.attention_gate_backward(g, attn, x, w, gate, "bf16")
    gpre = oracle.round_to((g.reshape(m, h, dh) * attn).sum(2) * gate * (1 - gate), "bf16")
    assert np.array_equal(gb, oracle.round_to(gpre.sum(0), "bf16"))
    unrounded = ((g.reshape(m, h, dh) * attn).sum(2) * gate * (1 - gate)).sum(0)
    assert not np.array_equal(oracle.round_to(unrounded, "bf16"), gb)


def test_band_rows_gather_scatter_vs_torch_index_ops():
    """The Mel-band gather / averaged scatter against torch index_select / scatter_add_ (the library
    routines the stock model uses), an all-ones mask averaging to ones on covered rows, and the
    scatter being the gather's adjoint (<gather(x), y> = <x, scatter(y)>)."""
    r = _rng(17)
    b, R, t = 2, 11, 5
    rows = np.array([0, 1, 2, 2, 3, 4, 5, 5, 6, 8, 9, 10, 10])  # rows 2, 5, 10 twice; row 7 never
    x = r.standard_normal((b, R, t, 2))
    got = oracle.band_rows_gather(x, rows)
    ref = torch.from_numpy(x).index_select(1, torch.from_numpy(rows)).permute(0, 2, 1, 3).numpy()
    _close(got, torch.from_numpy(ref), what="gather")
    y = r.standard_normal((b, t, rows.size, 2))
    vals = torch.from_numpy(y).permute(0, 2, 1, 3)
    idx = torch.from_numpy(rows).view(1, -1, 1, 1).expand(b, -1, t, 2)
    summed = torch.zeros(b, R, t, 2, dtype=torch.float64).scatter_add_(1, idx, vals)
    counts = torch.bincount(torch.from_numpy(rows), minlength=R).clamp(min=1).double()
    _close(oracle.band_rows_scatter(y, rows, R, mean=False), summed, what="scatter sum")
    _close(oracle.band_rows_scatter(y, rows, R, mean=True), summed / counts.view(1, -1, 1, 1), what="scatter mean")
    ones = oracle.band_rows_scatter(np.ones((b, t, rows.size, 2)), rows, R, mean=True)
    covered = np.bincount(rows, minlength=R) > 0
    assert np.allclose(ones[:, covered], 1.0) and np.allclose(ones[:, ~covered], 0.0)
    lhs = (oracle.band_rows_gather(x, rows) * y).sum()
    rhs = (x * oracle.band_rows_scatter(y, rows, R, mean=False)).sum()
    assert abs(lhs - rhs) <= 1e-9 * max(1.0, abs(lhs))


@pytest.mark.parametrize("zero_dc", [False, True])
def test_mask_apply_vs_torch_complex_autograd(zero_dc):
    """The stock model's mask product and iSTFT permute in torch (CPU complex autograd) against the
    oracle, plus an explicit-loop check of the layout on the same inputs."""
    g = torch.Generator().manual_seed(5)
    b, s, c, f, t = 2, 3, 2, 5, 7
    spec = torch.complex(torch.randn(b, f * c, t, generator=g, dtype=torch.float64),
                         torch.randn(b, f * c, t, generator=g, dtype=torch.float64)).requires_grad_(True)
    mask = torch.randn(b, s, t, f * c * 2, generator=g, dtype=torch.float64, requires_grad=True)
    m = torch.view_as_complex(mask.reshape(b, s, t, f * c, 2)).transpose(-1, -2)
    est = (spec.unsqueeze(1) * m).reshape(b, s, f, c, t).transpose(2, 3).reshape(b * s * c, f, t)
    if zero_dc:
        est = est.index_fill(1, torch.zeros(1, dtype=torch.long), 0.0)
    ge = torch.complex(torch.randn(est.shape, generator=g, dtype=torch.float64),
                       torch.randn(est.shape, generator=g, dtype=torch.float64))
    (est * ge.conj()).real.sum().backward()   # d/d(est) of Re<est, ge> is ge
    ri = lambda z: np.stack([np.real(z), np.imag(z)], axis=-1)  # noqa: E731  (compare re and im)
    got = oracle.mask_apply_forward(spec.detach().numpy(), mask.detach().numpy(), c, zero_dc)
    _close(ri(got), ri(est.detach().numpy()), what="est")
    gm, gs = oracle.mask_apply_backward(ge.numpy(), spec.detach().numpy(), mask.detach().numpy(), c, zero_dc)
    _close(gm, mask.grad.numpy(), what="grad_mask")
    _close(ri(gs), ri(spec.grad.numpy()), what="grad_spec")
    sp, mk = spec.detach().numpy(), mask.detach().numpy()
    for (bi, si, ci, fi, ti) in [(0, 0, 0, 1, 0), (1, 2, 1, 4, 6), (1, 1, 0, 2, 3)]:
        r = fi * c + ci
        want = sp[bi, r, ti] * complex(mk[bi, si, ti, 2 * r], mk[bi, si, ti, 2 * r + 1])
        assert abs(got[(bi * s + si) * c + ci, fi, ti] - want) < 1e-12
    if zero_dc:
        assert np.all(got[:, 0, :] == 0) and np.all(gm.reshape(b, s, t, f, c, 2)[:, :, :, 0] == 0)


def test_grouped_mode_rounding_points_follow_torch_casts():
    """``grad_pre_dt`` stores dpre in bf16 before the dx / dW products while dbias sums the unrounded
    values (.cu:2343-2346), and the MLP hidden layer is bf16 after the linear and after tanh
    (fr.py:338-340): checked against torch's own bf16 casts at those points; leaving the rounding out
    of dx must show."""
    r = _rng(15)
    dim_inputs = (4, 8, 12)
    m, nb, hid = 9, 3, 32
    x = oracle.round_to(r.standard_normal((m, nb, hid)), "bf16")
    w = [oracle.round_to(r.standard_normal((2 * d, hid)) / math.sqrt(hid), "bf16") for d in dim_inputs]
    bias = oracle.round_to(0.1 * r.standard_normal(2 * sum(dim_inputs)), "bf16")
    _, pre = oracle.mask_estimator_final_forward(x, w, bias, dim_inputs, "bf16")
    g = oracle.round_to(r.standard_normal((m, sum(dim_inputs))), "bf16")
    dx, dbias, dws = oracle.mask_estimator_final_backward(g, x, pre, w, dim_inputs, "f64", grad_pre_dt="bf16")
    off = 0
    for b, d in enumerate(dim_inputs):
        p = torch.from_numpy(pre[:, 2 * off : 2 * off + 2 * d])
        left, gate = p[:, :d], p[:, d:]
        s = torch.sigmoid(gate)
        gb = torch.from_numpy(g[:, off : off + d])
        dpre = torch.cat([gb * s, gb * left * s * (1 - s)], dim=1)
        _close(dbias[2 * off : 2 * off + 2 * d], dpre.sum(0), what=f"dbias{b}")
        dpre16 = dpre.to(torch.bfloat16).double()
        _close(dx[:, b], dpre16 @ torch.from_numpy(w[b]), what=f"dx{b}")
        _close(dws[b], dpre16.t() @ torch.from_numpy(x[:, b]), what=f"dW{b}")
        off += d
    dx_exact, _, _ = oracle.mask_estimator_final_backward(g, x, pre, w, dim_inputs, "f64")
    assert np.max(np.abs(dx_exact - dx)) > 1e-4
    w1 = oracle.round_to(r.standard_normal((nb, 16, hid)) / 4, "bf16")
    b1 = oracle.round_to(r.standard_normal((nb, 16)), "bf16")
    h = oracle.mask_mlp_hidden(x, w1, b1, "bf16")
    z = torch.einsum("mgi,goi->mgo", torch.from_numpy(x), torch.from_numpy(w1)) + torch.from_numpy(b1)
    ref = torch.tanh(z.to(torch.bfloat16).double()).to(torch.bfloat16).double()
    assert np.array_equal(h, ref.numpy())

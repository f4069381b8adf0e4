"""numpy restatement of the reference's fused layer kernels (test infrastructure only).

Reference: baicai-1145/pymsst ``src/pymsst/training/cuda/fused_band_split.cu``
(``.cu`` below) and ``src/pymsst/training/fused_roformer.py`` (``fr.py``).

Conventions
-----------
* Inputs are float arrays holding values exactly representable in their
  storage dtype ``dt`` (one of ``"f32"``, ``"f16"``, ``"bf16"``).
* Arithmetic is float64 (``acc=np.float64``) or float32 when the oracle is
  timed as the CPU baseline (``acc=np.float32``).
* Every stored output is rounded to the storage dtype the reference kernel
  writes (``static_cast<scalar_t>``); ``inv_norm`` is always fp32
  (fused_band_split.cpp:342,459).
* Functions suffixed ``_lean`` / ``rms_norm_rotary_*`` / ``mask_mlp_*``
  restate fused variants this build adds; they are compositions of the
  reference functions above them, with the intermediate left unrounded.
"""

from __future__ import annotations

import math

import numpy as np

from .dtypes import round_to

__all__ = [
    "rms_norm_forward",
    "rms_norm_backward",
    "rms_norm_backward_lean",
    "rotary_forward",
    "rotary_backward",
    "rotary_tables",
    "rms_norm_rotary_forward",
    "rms_norm_rotary_backward",
    "band_split_forward",
    "band_split_backward",
    "band_split_ragged_forward",
    "band_split_ragged_backward",
    "band_split_ragged_backward_lean",
    "band_split_mixed_forward",
    "band_split_mixed_backward",
    "grouped_linear_forward",
    "grouped_linear_backward",
    "mask_estimator_final_forward",
    "mask_estimator_final_backward",
    "mask_mlp_hidden",
    "mask_mlp_forward",
    "mask_mlp_backward",
    "attention_gate_forward",
    "attention_gate_backward",
    "band_rows_gather",
    "band_rows_scatter",
    "mask_apply_forward",
    "mask_apply_backward",
    "sigmoid",
]

_EPS = 1.0e-12


def _f(a, acc):
    return np.asarray(a, dtype=acc)


def _inv_out(inv, dt):
    """``inv_norm`` is stored as fp32 by every reference kernel; kept exact when ``dt == "f64"``."""
    return round_to(inv, "f64" if dt == "f64" else "f32")


def _inv_norm(x, acc):
    """``inv = 1/max(sqrt(sum x^2), 1e-12)`` over the last axis (.cu:48-50)."""
    ss = np.sum(x * x, axis=-1)
    return 1.0 / np.maximum(np.sqrt(ss), acc(_EPS))


# --------------------------------------------------------------------------- RMSNorm


def rms_norm_forward(x, gamma, dt: str, mode: str = "plain", acc=np.float64):
    """RMSNorm forward over the last axis.

    Follows .cu:1210-1249 (``mode="plain"``: gamma in ``dt``),
    .cu:1399-1438 (``"fp32_gamma"``: gamma fp32, outputs in ``dt``) and
    .cu:1588-1627 (``"mixed"``: gamma fp32, ``out``/``normed`` fp32).

    ``n = x * inv * sqrt(D)``, ``out = n * gamma``; ``out`` is formed from the
    unrounded ``n`` (.cu:1244-1247).  Returns ``(out, normed, inv_norm)``.
    """
    x = _f(x, acc)
    gamma = _f(gamma, acc)
    dim = x.shape[-1]
    inv = _inv_norm(x, acc)
    n = x * inv[..., None] * acc(math.sqrt(dim))
    out_dt = "f32" if mode == "mixed" else dt
    out = round_to(n * gamma, out_dt)
    normed = round_to(n, out_dt)
    return out, normed, _inv_out(inv, dt)


def rms_norm_backward(grad_out, normed, inv_norm, gamma, dt: str, mode: str = "plain", acc=np.float64):
    """RMSNorm backward from saved ``normed``/``inv_norm``.

    Follows .cu:1251-1315 (plain), .cu:1440-1504 (fp32_gamma) and
    .cu:1629-1691 (mixed: ``grad_out``/``normed`` fp32, ``grad_x`` in ``dt``):
    ``gn = dy*gamma``, ``dot = sum(gn*normed)``,
    ``dx = inv*(gn*sqrt(D) - normed*dot/sqrt(D))``, ``dgamma = sum_rows dy*normed``.
    ``dgamma`` is stored in gamma's dtype (``dt`` for plain, fp32 otherwise).
    """
    dy = _f(grad_out, acc)
    n = _f(normed, acc)
    inv = _f(inv_norm, acc)
    gamma = _f(gamma, acc)
    dim = dy.shape[-1]
    scale = acc(math.sqrt(dim))
    gn = dy * gamma
    dot = np.sum(gn * n, axis=-1, keepdims=True)
    dx = inv.reshape(dot.shape) * (gn * scale - n * (dot / scale))
    dgamma = np.sum((dy * n).reshape(-1, dim), axis=0)
    g_dt = dt if mode == "plain" else "f32"
    return round_to(dx, dt), round_to(dgamma, g_dt)


def rms_norm_backward_lean(grad_out, x, inv_norm, gamma, dt: str, gamma_dt: str | None = None, acc=np.float64):
    """RMSNorm backward that recomputes ``n = x*inv*sqrt(D)`` from the saved input.

    Same algebra as :func:`rms_norm_backward` (.cu:1251-1315) with the saved
    ``normed`` replaced by its unrounded value; used by this build's
    ``_FusedRMSNorm`` fast path, which saves ``x`` instead of writing ``normed``.
    """
    x = _f(x, acc)
    dim = x.shape[-1]
    n = x * _f(inv_norm, acc).reshape(*x.shape[:-1], 1) * acc(math.sqrt(dim))
    mode = "plain" if (gamma_dt or dt) == dt else "fp32_gamma"
    return rms_norm_backward(grad_out, n, inv_norm, gamma, dt, mode, acc)


# --------------------------------------------------------------------------- rotary


def rotary_tables(seq_len: int, dim: int, theta: float = 10000.0):
    """RoFormer tables ``cos/sin[n, p] = cos/sin(n * theta**(-2p/dim))``, shape ``[N, dim/2]``.

    The reference passes ``cos[..., ::2]`` of the pairwise-repeated stock table
    (fr.py:727), i.e. one value per adjacent pair; table construction itself
    lives in pymss-core and is restated from the public RoFormer definition.
    """
    p = np.arange(0, dim, 2, dtype=np.float64)[: dim // 2]
    inv_freq = 1.0 / (theta ** (p / dim))
    ang = np.arange(seq_len, dtype=np.float64)[:, None] * inv_freq[None, :]
    return np.cos(ang), np.sin(ang)


def _rot(t, cos, sin, acc, sign):
    t = _f(t, acc)
    b, n, h, d = t.shape
    c = _f(cos, acc).reshape(1, n, 1, d // 2)
    s = _f(sin, acc).reshape(1, n, 1, d // 2) * sign
    e = t[..., 0::2]
    o = t[..., 1::2]
    out = np.empty_like(t)
    out[..., 0::2] = e * c - o * s
    out[..., 1::2] = o * c + e * s
    return out


def rotary_forward(t, cos, sin, dt: str, acc=np.float64):
    """Adjacent-pair rotation of ``t[B,N,H,D]`` (.cu:1076-1101):
    ``(e, o) -> (e*c - o*s, o*c + e*s)`` with ``c, s = cos/sin[n, pair]``."""
    return round_to(_rot(t, cos, sin, acc, 1.0), dt)


def rotary_backward(grad_out, cos, sin, dt: str, acc=np.float64):
    """Transpose rotation (.cu:1103-1128): ``(ge*c + go*s, -ge*s + go*c)``."""
    return round_to(_rot(grad_out, cos, sin, acc, -1.0), dt)


def rms_norm_rotary_forward(x, gamma, cos, sin, dt: str, acc=np.float64):
    """Fused q/k RMSNorm over the head dim followed by rotary, one rounding.

    Composition of .cu:1399-1438 (gamma in its own dtype) and .cu:1076-1101
    with ``n*gamma`` kept unrounded.  Returns ``(out, inv_norm)``.
    """
    x = _f(x, acc)
    dim = x.shape[-1]
    inv = _inv_norm(x, acc)
    y = x * inv[..., None] * acc(math.sqrt(dim)) * _f(gamma, acc)
    return round_to(_rot(y, cos, sin, acc, 1.0), dt), _inv_out(inv, dt)


def rms_norm_rotary_backward(grad_out, x, inv_norm, gamma, cos, sin, dt: str, gamma_dt: str, acc=np.float64):
    """Backward of :func:`rms_norm_rotary_forward`: ``g = rot^T(dy)`` then the
    RMSNorm backward of .cu:1251-1315 on ``g`` with ``n`` recomputed from ``x``."""
    g = _rot(grad_out, cos, sin, acc, -1.0)
    x = _f(x, acc)
    dim = x.shape[-1]
    inv = _f(inv_norm, acc).reshape(x.shape[:-1])
    n = x * inv[..., None] * acc(math.sqrt(dim))
    scale = acc(math.sqrt(dim))
    gn = g * _f(gamma, acc)
    dot = np.sum(gn * n, axis=-1, keepdims=True)
    dx = inv[..., None] * (gn * scale - n * (dot / scale))
    dgamma = np.sum((g * n).reshape(-1, dim), axis=0)
    return round_to(dx, dt), round_to(dgamma, gamma_dt)


# --------------------------------------------------------------------------- band split


def band_split_forward(x, gamma, weight, bias, dt: str, acc=np.float64):
    """Equal-width band group ``x[M,G,I]``, ``gamma[G,I]``, ``weight[G,O,I]``, ``bias[G,O]|None``.

    .cu:13-71 / fr.py:1265-1271: ``n = x*inv*sqrt(I)``,
    ``out = bias + sum_i (n*gamma)_i W_oi``.  Returns ``(out, normed, inv_norm)``.
    """
    x = _f(x, acc)
    dim_in = x.shape[-1]
    inv = _inv_norm(x, acc)
    n = x * inv[..., None] * acc(math.sqrt(dim_in))
    feat = n * _f(gamma, acc)[None]
    out = np.einsum("mgi,goi->mgo", feat, _f(weight, acc))
    if bias is not None:
        out = out + _f(bias, acc)[None]
    return round_to(out, dt), round_to(n, dt), _inv_out(inv, dt)


def band_split_backward(grad_out, normed, inv_norm, gamma, weight, has_bias: bool, dt: str, acc=np.float64):
    """Backward of :func:`band_split_forward` (.cu:125-247; v2/v3 .cu:314-587 compute the same values).

    ``gs = dy W``, ``gn = gs*gamma``, ``dx = inv*(gn*sqrt(I) - n*(gn.n)/sqrt(I))``,
    ``dW = sum_m dy (n*gamma)``, ``db = sum_m dy``, ``dgamma = sum_m gs*n``.
    Returns ``(dx, dgamma, dW, db|None)``.
    """
    dy = _f(grad_out, acc)
    n = _f(normed, acc)
    inv = _f(inv_norm, acc)
    gamma = _f(gamma, acc)
    weight = _f(weight, acc)
    dim_in = n.shape[-1]
    scale = acc(math.sqrt(dim_in))
    gs = np.einsum("mgo,goi->mgi", dy, weight)
    gn = gs * gamma[None]
    dot = np.sum(gn * n, axis=-1, keepdims=True)
    dx = inv[..., None] * (gn * scale - n * (dot / scale))
    dW = np.einsum("mgo,mgi->goi", dy, n * gamma[None])
    db = dy.sum(axis=0) if has_bias else None
    dgamma = np.sum(gs * n, axis=0)
    return (
        round_to(dx, dt),
        round_to(dgamma, dt),
        round_to(dW, dt),
        round_to(db, dt) if db is not None else None,
    )


def _offsets(dim_inputs):
    off = [0]
    for d in dim_inputs:
        off.append(off[-1] + int(d))
    return off


def band_split_ragged_forward(x, gammas, weights, biases, dim_inputs, dt: str, acc=np.float64):
    """Ragged band split over ``x[M,F]`` (.cu:589-652): band ``b`` spans
    ``offsets[b]:offsets[b+1]``.  Returns ``(out[M,NB,O], normed[M,F], inv[M,NB])``."""
    x = _f(x, acc)
    off = _offsets(dim_inputs)
    outs, normed, invs = [], [], []
    for b in range(len(dim_inputs)):
        xb = x[:, off[b] : off[b + 1]][:, None, :]
        o, n, i = band_split_forward(
            xb, _f(gammas[b], acc)[None], _f(weights[b], acc)[None], _f(biases[b], acc)[None], dt, acc
        )
        outs.append(o[:, 0])
        normed.append(n[:, 0])
        invs.append(i[:, 0])
    return np.stack(outs, axis=1), np.concatenate(normed, axis=1), np.stack(invs, axis=1)


def band_split_ragged_backward(grad_out, normed, inv_norm, gammas, weights, dim_inputs, dt: str, acc=np.float64):
    """Ragged backward (.cu:741-879).  Returns ``(dx[M,F], [dgamma_b], [dW_b], [db_b])``."""
    off = _offsets(dim_inputs)
    dy = _f(grad_out, acc)
    n = _f(normed, acc)
    inv = _f(inv_norm, acc)
    dxs, dgs, dws, dbs = [], [], [], []
    for b in range(len(dim_inputs)):
        dx, dg, dw, db = band_split_backward(
            dy[:, b : b + 1],
            n[:, off[b] : off[b + 1]][:, None, :],
            inv[:, b : b + 1],
            _f(gammas[b], acc)[None],
            _f(weights[b], acc)[None],
            True,
            dt,
            acc,
        )
        dxs.append(dx[:, 0])
        dgs.append(dg[0])
        dws.append(dw[0])
        dbs.append(db[0])
    return np.concatenate(dxs, axis=1), dgs, dws, dbs


def band_split_ragged_backward_lean(grad_out, x, inv_norm, gammas, weights, dim_inputs, dt: str, acc=np.float64):
    """Ragged backward with ``normed`` recomputed (unrounded) from the saved input ``x``:
    same algebra as .cu:741-879; used by this build's saved-input fast path."""
    x = _f(x, acc)
    inv = _f(inv_norm, acc)
    off = _offsets(dim_inputs)
    n = np.empty_like(x)
    for b in range(len(dim_inputs)):
        w = off[b + 1] - off[b]
        n[:, off[b] : off[b + 1]] = x[:, off[b] : off[b + 1]] * inv[:, b : b + 1] * math.sqrt(w)
    return band_split_ragged_backward(grad_out, n, inv_norm, gammas, weights, dim_inputs, dt, acc)


def band_split_mixed_forward(x, gammas, weights, biases, dim_inputs, dt: str, acc=np.float64):
    """The ragged band split of an fp32 input with a 16-bit projection: the call fr.py:827-857 makes under
    autocast (the STFT input is fp32, so the reference's norm runs in fp32, .cu:589-652), with the
    projection rounded where the stock module's autocast nn.Linear rounds it: its input
    ``u = dt(n * gamma)`` and weight in ``dt``, its output ``dt(u W^T + bias)``.

    ``x`` fp32 values, ``gammas`` fp32, ``weights`` / ``biases`` in ``dt``.
    Returns ``(out[M,NB,O] in dt, u[M,F] in dt, inv[M,NB] fp32)``."""
    x = _f(x, acc)
    off = _offsets(dim_inputs)
    outs, feats, invs = [], [], []
    for b in range(len(dim_inputs)):
        xb = x[:, off[b] : off[b + 1]]
        inv = _inv_norm(xb, acc)
        n = xb * inv[:, None] * acc(math.sqrt(off[b + 1] - off[b]))
        u = round_to(n * _f(gammas[b], acc)[None], dt)
        outs.append(round_to(u @ _f(weights[b], acc).T + _f(biases[b], acc)[None], dt))
        feats.append(u)
        invs.append(_inv_out(inv, "f32"))
    return np.stack(outs, axis=1), np.concatenate(feats, axis=1), np.stack(invs, axis=1)


def band_split_mixed_backward(grad_out, x, features, inv_norm, gammas, weights, dim_inputs, dt: str, acc=np.float64):
    """Backward of :func:`band_split_mixed_forward`: the stock autocast Linear's input gradient
    ``g = dt(dy W)``, then the fp32 RMSNorm backward of .cu:741-879 (``gn = g gamma``,
    ``dx = inv (gn sqrt(I) - n (gn . n) / sqrt(I))``, ``dgamma = sum_m g n``); ``dW = dt(dy^T u)``,
    ``db = dt(sum_m dy)``.  Returns ``(dx fp32, [dgamma_b] fp32, [dW_b] dt, [db_b] dt)``."""
    dy = _f(grad_out, acc)
    x = _f(x, acc)
    u = _f(features, acc)
    inv = _f(inv_norm, acc)
    off = _offsets(dim_inputs)
    dxs, dgs, dws, dbs = [], [], [], []
    for b in range(len(dim_inputs)):
        w = off[b + 1] - off[b]
        scale = acc(math.sqrt(w))
        xb = x[:, off[b] : off[b + 1]]
        n = xb * inv[:, b : b + 1] * scale
        g = round_to(dy[:, b] @ _f(weights[b], acc), dt)
        gn = g * _f(gammas[b], acc)[None]
        dot = np.sum(gn * n, axis=-1, keepdims=True)
        dxs.append(round_to(inv[:, b : b + 1] * (gn * scale - n * (dot / scale)), "f32"))
        dgs.append(round_to(np.sum(g * n, axis=0), "f32"))
        dws.append(round_to(dy[:, b].T @ u[:, off[b] : off[b + 1]], dt))
        dbs.append(round_to(dy[:, b].sum(axis=0), dt))
    return np.concatenate(dxs, axis=1), dgs, dws, dbs


# --------------------------------------------------------------------------- grouped linear


def grouped_linear_forward(x, weight, bias, dt: str, acc=np.float64, act: str | None = None):
    """``out[m,g,o] = bias[g,o] + sum_i x[m,g,i] W[g,o,i]`` (.cu:1005-1030; bmm form tts.py:28-37).

    ``act="tanh"`` applies the mask-MLP hidden activation (``inference_tanh``, fr.py:340) to the
    linear output rounded to ``dt`` (the reference's two steps, fr.py:338-340), then rounds again."""
    out = np.matmul(_f(x, acc).transpose(1, 0, 2), _f(weight, acc).transpose(0, 2, 1)).transpose(1, 0, 2)
    if bias is not None:
        out = out + _f(bias, acc)[None]
    if act == "tanh":
        out = np.tanh(round_to(out, dt))
    elif act is not None:
        raise ValueError(act)
    return round_to(out, dt)


def grouped_linear_backward(grad_out, x, weight, has_bias: bool, dt: str, acc=np.float64):
    """Backward of grouped linear (fr.py:1042-1048): ``dx = dy W``, ``dW = dy^T x``, ``db = sum_m dy``."""
    dy = _f(grad_out, acc)
    dyt = dy.transpose(1, 0, 2)  # [G, M, O]
    dx = np.matmul(dyt, _f(weight, acc)).transpose(1, 0, 2)
    dW = np.matmul(dyt.transpose(0, 2, 1), _f(x, acc).transpose(1, 0, 2))
    db = dy.sum(axis=0) if has_bias else None
    return round_to(dx, dt), round_to(dW, dt), (round_to(db, dt) if db is not None else None)


# --------------------------------------------------------------------------- mask estimator


def _gmm(a, b):
    """``out[m,g,o] = sum_i a[m,g,i] b[g,o,i]`` as one batched matmul over g."""
    return np.matmul(a.transpose(1, 0, 2), b.transpose(0, 2, 1)).transpose(1, 0, 2)


def sigmoid(z):
    """Logistic function in the overflow-free form 0.5 * (1 + tanh(z / 2))."""
    return 0.5 * (1.0 + np.tanh(0.5 * z))


def mask_estimator_final_forward(x, weights, bias, dim_inputs, dt: str, acc=np.float64):
    """Final per-band Linear ``H -> 2*I_b`` + bias + GLU (.cu:2515-2552 direct; .cu:2283-2310 grouped).

    ``x[M,NB,H]``; ``weights[b]`` is ``[2*I_b, H]``; ``bias`` is flat ``[2F]`` with band
    ``b`` at ``[2*off_b, 2*off_b + 2*I_b)``, left half first.
    ``pre = x W^T + bias`` (stored), ``out = left * sigmoid(gate)``.
    Returns ``(out[M,F], pre[M,2F])``.
    """
    x = _f(x, acc)
    bias = _f(bias, acc)
    off = _offsets(dim_inputs)
    outs, pres = [], []
    for b, d in enumerate(dim_inputs):
        p = x[:, b, :] @ _f(weights[b], acc).T + bias[2 * off[b] : 2 * off[b] + 2 * d]
        left, gate = p[:, :d], p[:, d:]
        outs.append(left * sigmoid(gate))
        pres.append(p)
    return round_to(np.concatenate(outs, axis=1), dt), round_to(np.concatenate(pres, axis=1), dt)


def mask_estimator_final_backward(grad_out, x, pre, weights, dim_inputs, dt: str, acc=np.float64,
                                  input_act: str | None = None, grad_pre_dt: str | None = None):
    """Backward of :func:`mask_estimator_final_forward` (.cu:2312-2367, .cu:2585-2704).

    From the saved ``pre``: ``dL = g*s``, ``dG = g*L*s*(1-s)`` with ``s = sigmoid(G)``;
    ``dbias = sum_m dpre``, ``dx_b = dpre_b W_b``, ``dW_b = dpre_b^T x_b``.
    ``grad_pre_dt``: the grouped mode stores ``dpre`` in the tensor dtype before its GEMMs
    (.cu:2343-2344, ``static_cast<scalar_t>``) while ``dbias`` sums the unrounded values
    (.cu:2345-2346); ``None`` is the direct mode: ``dx`` and ``dbias`` from the unrounded ``dpre``
    (.cu:2620-2635, 2645-2655), ``dW`` from the ``grad_pre`` it stored in the tensor dtype
    (.cu:2618-2619 written, .cu:2697-2700 read).
    ``input_act="tanh"``: ``x`` is a tanh output and the first result is the gradient of its
    pre-activation, ``dx * (1 - x^2)`` (chain rule through ``inference_tanh``).
    Returns ``(dx[M,NB,H], dbias[2F], [dW_b])``.
    """
    g = _f(grad_out, acc)
    x = _f(x, acc)
    pre = _f(pre, acc)
    off = _offsets(dim_inputs)
    dx = np.empty_like(x)
    dbias = []
    dws = []
    for b, d in enumerate(dim_inputs):
        p = pre[:, 2 * off[b] : 2 * off[b] + 2 * d]
        left, gate = p[:, :d], p[:, d:]
        s = sigmoid(gate)
        gb = g[:, off[b] : off[b] + d]
        dpre = np.concatenate([gb * s, gb * left * s * (1.0 - s)], axis=1)
        dbias.append(dpre.sum(axis=0))
        if grad_pre_dt is not None:
            dpre = round_to(dpre, grad_pre_dt)
        dx[:, b, :] = dpre @ _f(weights[b], acc)
        dpre_stored = dpre if grad_pre_dt is not None else round_to(dpre, dt)
        dws.append(round_to(dpre_stored.T @ x[:, b, :], dt))
    if input_act == "tanh":
        # dh in the tensor dtype (the stored product of the grouped form), then tanh's backward
        dx = round_to(dx, dt) * (1.0 - x * x)
    elif input_act is not None:
        raise ValueError(input_act)
    return round_to(dx, dt), round_to(np.concatenate(dbias), dt), dws


def mask_mlp_hidden(x, w1, b1, dt: str, acc=np.float64):
    """Hidden layer of the mask MLP as the reference computes it: the grouped linear's output in the
    tensor dtype (fr.py:338, .cu:1005-1030), then ``inference_tanh`` in that dtype (fr.py:340)."""
    z = round_to(_gmm(_f(x, acc), _f(w1, acc)) + _f(b1, acc)[None], dt)
    return round_to(np.tanh(z), dt)


def mask_mlp_forward(x, w1, b1, weights2, bias2, dim_inputs, dt: str, acc=np.float64):
    """Whole per-band mask MLP (depth 2): ``h = tanh(x_b W1_b^T + b1_b)`` (:func:`mask_mlp_hidden`,
    ``w1[NB,Hd,dim]``, ``b1[NB,Hd]``), then the final Linear + GLU of
    :func:`mask_estimator_final_forward` (fr.py:332-369).  Returns ``out[M,F]``."""
    h = mask_mlp_hidden(x, w1, b1, dt, acc)
    out, _ = mask_estimator_final_forward(h, weights2, bias2, dim_inputs, dt, acc)
    return out


def mask_mlp_backward(grad_out, x, w1, b1, weights2, bias2, dim_inputs, dt: str, acc=np.float64):
    """Backward of :func:`mask_mlp_forward` with ``h`` recomputed: the final layer's backward in its
    grouped form (``dpre`` stored in ``dt``, .cu:2343-2344) gives ``dh`` in ``dt``, the tanh backward
    ``dz = dh (1 - h^2)`` in ``dt`` (autograd of ``inference_tanh``), then the grouped linear's backward
    (fr.py:1042-1048).  Returns ``(dx[M,NB,dim], dW1[NB,Hd,dim], db1[NB,Hd], [dW2_b], dbias2[2F])``."""
    x = _f(x, acc)
    w1 = _f(w1, acc)
    h = mask_mlp_hidden(x, w1, b1, dt, acc)
    _, pre = mask_estimator_final_forward(h, weights2, bias2, dim_inputs, dt, acc)
    dz, dbias2, dws2 = mask_estimator_final_backward(grad_out, h, pre, weights2, dim_inputs, dt, acc,
                                                     input_act="tanh", grad_pre_dt=dt)
    dzt = dz.transpose(1, 0, 2)  # [G, M, Hd]
    dx = np.matmul(dzt, w1).transpose(1, 0, 2)
    dW1 = np.matmul(dzt.transpose(0, 2, 1), x.transpose(1, 0, 2))
    db1 = dz.sum(axis=0)
    return round_to(dx, dt), round_to(dW1, dt), round_to(db1, dt), dws2, dbias2


def attention_gate_forward(attn, x, weight, bias, dt: str, acc=np.float64):
    """Attention output gate (.cu:1777-1826; fr.py:1228-1250).

    ``attn[M,H,Dh]``, ``x[M,D]``, ``weight[H,D]``, ``bias[H]``.
    ``gate = sigmoid(x W^T + b)`` is stored in the storage dtype (.cu:1805) and the stored
    value scales the attention output: ``out[m, h*Dh + d] = attn[m,h,d] * gate[m,h]`` (.cu:1823).
    Returns ``(out[M, H*Dh], gate[M,H])``.
    """
    attn = _f(attn, acc)
    gate = round_to(sigmoid(_f(x, acc) @ _f(weight, acc).T + _f(bias, acc)), dt)
    out = attn * _f(gate, acc)[:, :, None]
    return round_to(out.reshape(attn.shape[0], -1), dt), gate


def attention_gate_backward(grad_out, attn, x, weight, gate, dt: str, acc=np.float64):
    """Backward of :func:`attention_gate_forward` (.cu:1828-1920, .cu:1973-2036).

    ``grad_attn = g * gate``; ``gpre = (sum_d g * attn) * gate * (1 - gate)`` stored in the
    storage dtype (.cu:1862) and used as stored for ``grad_x = gpre W``,
    ``grad_weight = gpre^T x`` and ``grad_bias = sum_m gpre``.
    Returns ``(grad_attn[M,H,Dh], grad_x[M,D], grad_weight[H,D], grad_bias[H])``.
    """
    attn = _f(attn, acc)
    m, h, dh = attn.shape
    g = _f(grad_out, acc).reshape(m, h, dh)
    gt = _f(gate, acc)
    grad_attn = g * gt[:, :, None]
    gpre = _f(round_to((g * attn).sum(axis=2) * gt * (1.0 - gt), dt), acc)
    grad_x = gpre @ _f(weight, acc)
    grad_w = gpre.T @ _f(x, acc)
    grad_b = gpre.sum(axis=0)
    return round_to(grad_attn, dt), round_to(grad_x, dt), round_to(grad_w, dt), round_to(grad_b, dt)


def band_rows_gather(x, rows, divisor=None):
    """Mel band gather (no reference counterpart; pymss-core's Mel-band model indexes the spectrum
    rows of each band in band order): ``x[B, R, T, 2]`` -> ``out[B, T, J, 2]``,
    ``out[b, t, j] = x[b, rows[j], t] / divisor[j]``.  float64 results."""
    x = np.asarray(x, dtype=np.float64)
    out = x[:, np.asarray(rows), :, :].transpose(0, 2, 1, 3)
    if divisor is not None:
        out = out / np.asarray(divisor, dtype=np.float64)[None, None, :, None]
    return out


def band_rows_scatter(x, rows, num_rows: int, mean: bool = True):
    """Overlap-averaged mask scatter (no reference counterpart; the Mel-band model's scatter_add
    + division by the number of bands per bin): ``x[B, T, J, 2]`` -> ``out[B, R, T, 2]`` with each
    row the sum (``mean``: the average) of the selections pointing at it; unselected rows are 0."""
    x = np.asarray(x, dtype=np.float64)
    rows = np.asarray(rows)
    b, t, j, _ = x.shape
    out = np.zeros((b, num_rows, t, 2))
    np.add.at(out, (slice(None), rows), x.transpose(0, 2, 1, 3))
    if mean:
        counts = np.bincount(rows, minlength=num_rows).astype(np.float64)
        out = out / np.maximum(counts, 1.0)[None, :, None, None]
    return out


def mask_apply_forward(spec, mask, channels: int, zero_dc: bool = False):
    """Complex mask application in the iSTFT layout (no reference kernel; the stock model's
    ``spec.unsqueeze(1) * mask`` followed by the permute the cached-zero iSTFT consumes,
    cuda_graph.py:140-158, with its optional zero-DC fill): ``spec`` complex ``[B, F*C, T]``,
    ``mask`` real ``[B, S, T, F*C*2]`` ((re, im) pairs) -> complex128 ``[B*S*C, F, T]``."""
    spec = np.asarray(spec, dtype=np.complex128)
    mask = np.asarray(mask, dtype=np.float64)
    b, fc, t = spec.shape
    s = mask.shape[1]
    f = fc // channels
    m = mask[..., 0::2] + 1j * mask[..., 1::2]                       # [B, S, T, FC]
    est = spec[:, None, :, :] * m.transpose(0, 1, 3, 2)              # [B, S, FC, T]
    est = est.reshape(b, s, f, channels, t).transpose(0, 1, 3, 2, 4)  # [B, S, C, F, T]
    if zero_dc:
        est = est.copy()
        est[:, :, :, 0, :] = 0
    return est.reshape(b * s * channels, f, t)


def mask_apply_backward(grad_est, spec, mask, channels: int, zero_dc: bool = False):
    """Gradients of :func:`mask_apply_forward` in PyTorch's complex convention (for a product
    ``est = spec * m`` the gradient of ``m`` is ``grad * conj(spec)``): returns
    ``(grad_mask [B, S, T, F*C*2] real (re, im) pairs, grad_spec complex [B, F*C, T])``."""
    spec = np.asarray(spec, dtype=np.complex128)
    mask = np.asarray(mask, dtype=np.float64)
    b, fc, t = spec.shape
    s = mask.shape[1]
    f = fc // channels
    g = np.asarray(grad_est, dtype=np.complex128).reshape(b, s, channels, f, t).copy()
    if zero_dc:
        g[:, :, :, 0, :] = 0
    g = g.transpose(0, 1, 3, 2, 4).reshape(b, s, fc, t)                 # [B, S, FC, T]
    gm = (g * np.conj(spec)[:, None]).transpose(0, 1, 3, 2)             # [B, S, T, FC]
    grad_mask = np.stack([gm.real, gm.imag], axis=-1).reshape(b, s, t, 2 * fc)
    m = (mask[..., 0::2] + 1j * mask[..., 1::2]).transpose(0, 1, 3, 2)  # [B, S, FC, T]
    grad_spec = (g * np.conj(m)).sum(axis=1)
    return grad_mask, grad_spec

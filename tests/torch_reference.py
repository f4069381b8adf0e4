"""Closed-form PyTorch statements of the stock modules on the path (float64, CPU, autograd).

These are the independent checks that pin the oracle: each one is written
with library routines (``F.normalize``, ``F.linear``, ``F.glu``, ``bmm``,
complex multiplication) exactly as the reference's pure-torch pieces and tests
state the math, and its gradients come from torch autograd rather than from a
hand-derived backward:

* RMSNorm: ``F.normalize(x, dim=-1) * sqrt(D) * gamma`` (fused_roformer.py:1267).
* Band split group: ``reference_band_split_group`` (fused_roformer.py:1265-1271).
* Grouped linear: ``_reference_grouped_linear`` bmm/baddbmm (tests/test_training_smoke.py:28-37).
* Mask final: per-band ``F.linear`` + ``F.glu`` (tests/test_training_smoke.py:574-615).
* Rotary: multiplication of ``t[2p] + i t[2p+1]`` by ``exp(i angle)``.
* Attention gate: the stock ``Attention`` tail, ``out * to_gates(x).sigmoid().unsqueeze(-1)``
  with ``to_gates = nn.Linear(dim, heads)`` (fused_roformer.py:776-824 patches it).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def rms_norm(x, gamma):
    return F.normalize(x, dim=-1) * (x.shape[-1] ** 0.5) * gamma


def rotary(t, cos, sin):
    """``t[B,N,H,D]``, ``cos/sin[N,D/2]``: complex multiply of adjacent pairs."""
    b, n, h, d = t.shape
    tc = torch.view_as_complex(t.reshape(b, n, h, d // 2, 2).contiguous())
    rot = torch.complex(cos, sin).reshape(1, n, 1, d // 2)
    return torch.view_as_real(tc * rot).reshape(b, n, h, d)


def band_split_group(x, gamma, weight, bias):
    dim_in = x.shape[-1]
    normalized = F.normalize(x, dim=-1) * (dim_in**0.5) * gamma.unsqueeze(0)
    out = torch.einsum("mgi,goi->mgo", normalized, weight)
    if bias is not None:
        out = out + bias.unsqueeze(0)
    return out


def band_split_ragged(x, gammas, weights, biases, dim_inputs):
    outs = []
    for xb, g, w, b in zip(x.split(list(dim_inputs), dim=-1), gammas, weights, biases):
        outs.append(F.linear(rms_norm(xb, g), w, b))
    return torch.stack(outs, dim=-2)


class _AutocastCast(torch.autograd.Function):
    """An fp32 tensor entering a 16-bit autocast op, in float64: forward rounds to fp32 then to
    ``dtype``; backward hands back the gradient the op produced, which is in ``dtype`` too."""

    @staticmethod
    def forward(ctx, t, dtype):
        ctx.dtype = dtype
        return t.float().to(dtype).double()

    @staticmethod
    def backward(ctx, grad):
        return grad.to(ctx.dtype).double(), None


class _OutputCast(torch.autograd.Function):
    """The 16-bit output of an autocast op, in float64: forward rounds, backward passes through."""

    @staticmethod
    def forward(ctx, t, dtype):
        return t.float().to(dtype).double()

    @staticmethod
    def backward(ctx, grad):
        return grad, None


def band_split_ragged_autocast(x, gammas, weights, biases, dim_inputs, dtype):
    """The stock band split under autocast in ``dtype``: RMSNorm in fp32 on the fp32 input, then the
    per-band nn.Linear on ``dtype`` operands (its input and weight cast by autocast) with a ``dtype``
    output.  ``weights`` / ``biases`` hold ``dtype`` values."""
    outs = []
    for xb, g, w, b in zip(x.split(list(dim_inputs), dim=-1), gammas, weights, biases):
        u = _AutocastCast.apply(rms_norm(xb, g), dtype)
        outs.append(_OutputCast.apply(F.linear(u, w, b), dtype))
    return torch.stack(outs, dim=-2)


def grouped_linear(x, weight, bias):
    group_count, _, in_features = weight.shape
    leading = x.shape[:-2]
    xt = x.reshape(-1, group_count, in_features).transpose(0, 1)
    wt = weight.transpose(1, 2)
    if bias is None:
        out = torch.bmm(xt, wt)
    else:
        out = torch.baddbmm(bias.unsqueeze(1).expand(-1, xt.shape[1], -1), xt, wt)
    return out.transpose(0, 1).reshape(*leading, group_count, -1)


def mask_final(x, weights, bias, dim_inputs):
    outs = []
    start = 0
    for b, d in enumerate(dim_inputs):
        pre = F.linear(x[:, b, :], weights[b], bias[2 * start : 2 * start + 2 * d])
        outs.append(F.glu(pre, dim=-1))
        start += d
    return torch.cat(outs, dim=-1)


def mask_mlp(x, w1, b1, weights2, bias2, dim_inputs):
    h = torch.tanh(grouped_linear(x, w1, b1))
    return mask_final(h, weights2, bias2, dim_inputs)


def attention_gate(attn, x, weight, bias):
    """``attn[M,H,Dh] * sigmoid(F.linear(x, weight, bias))[..., None]`` flattened to ``[M, H*Dh]``."""
    gates = torch.sigmoid(F.linear(x, weight, bias))
    return (attn * gates.unsqueeze(-1)).reshape(attn.shape[0], -1)

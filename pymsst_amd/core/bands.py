"""Band split front end and mask estimator (stock PyTorch restatement).

Names and contracts follow the pymss-core module the reference patches
(``pymss_core.modules.bs_roformer.bands``; call sites fused_roformer.py:256-707):

* ``grouped_linear(x[..., G, I], weight[G, O, I], bias[G, O] | None) -> [..., G, O]``
  with bmm/baddbmm semantics (tests/test_training_smoke.py:28-37);
* ``inference_tanh`` (fused_roformer.py:340,538);
* ``BandSplit``: per-band ``RMSNorm(I_b) -> Linear(I_b, dim)``; ``_dim_offsets``
  (NB+1 prefix sums), ``_dim_groups`` (contiguous runs of equal width,
  ``(start, end, width)``), ``_get_group_params(start, end, device, dtype)``
  returning stacked ``(gamma[G,I], weight[G,O,I], bias[G,O] | None)``,
  ``_forward_grouped`` (patched per instance at fused_roformer.py:265-268);
* ``MaskEstimator``: per band ``MLP(dim -> 2*I_b) + GLU``; ``_band_groupable_layers``,
  ``_layer_grouping_plan``, ``_get_layer_group_params``, ``_indices_tensor`` and
  ``_forward_layer_grouped_mlp`` (patched at fused_roformer.py:332-375,527-589).

State-dict keys match the per-band module layout: ``to_features.{b}.0.gamma``,
``to_features.{b}.1.weight/bias`` and ``to_freqs.{b}.0.{layer}.weight/bias``.
"""

from __future__ import annotations

import os

import torch
import torch.nn.functional as F
from torch import nn

from .transformer import RMSNorm

CORE_GROUPED_TRAIN_ENV = "PYMSS_CORE_EXPERIMENTAL_TRAIN_GROUPED_BANDS"


def _grouped_in_training() -> bool:
    return os.environ.get(CORE_GROUPED_TRAIN_ENV, "").lower() in {"1", "true", "yes", "on"}


def inference_tanh(x: torch.Tensor) -> torch.Tensor:
    return torch.tanh(x)


class _GroupedLinearBmm(torch.autograd.Function):
    """bmm / baddbmm grouped Linear with an explicit backward.

    Autograd's own bmm backward multiplies by transposed views of the saved operands
    (``grad @ W^T``, ``X^T @ grad``); 16-bit batched GEMMs whose right operand is such a
    transposed view have faulted GPUs of this platform, so every product here, forward and
    backward, takes contiguous operands.
    """

    @staticmethod
    def forward(ctx, x, weight, bias):
        groups, out_features, in_features = weight.shape
        lead = x.shape[:-2]
        # the dtype autocast would give bmm / baddbmm; the backward computes in it too
        dt = torch.get_autocast_dtype(x.device.type) if torch.is_autocast_enabled(x.device.type) else x.dtype
        ctx.dtypes = (x.dtype, weight.dtype, bias.dtype if bias is not None else None)
        xt = x.reshape(-1, groups, in_features).transpose(0, 1).to(dt).contiguous()  # [G, M, I]
        wc = weight.to(dt)
        wt = wc.transpose(1, 2).contiguous()                                         # [G, I, O]
        with torch.autocast(x.device.type, enabled=False):
            out = torch.bmm(xt, wt) if bias is None else torch.baddbmm(bias.to(dt).unsqueeze(1), xt, wt)
        ctx.save_for_backward(xt, wc)
        ctx.lead = lead
        return out.transpose(0, 1).reshape(*lead, groups, out_features)

    @staticmethod
    def backward(ctx, grad_out):
        xt, wc = ctx.saved_tensors
        groups, out_features, in_features = wc.shape
        x_dt, w_dt, b_dt = ctx.dtypes
        g = grad_out.to(xt.dtype).reshape(-1, groups, out_features).transpose(0, 1).contiguous()  # [G, M, O]
        grad_x = torch.bmm(g, wc.contiguous())                                                    # [G, M, I]
        grad_w = torch.bmm(g.transpose(1, 2).contiguous(), xt)                                     # [G, O, I]
        grad_b = g.sum(dim=1).to(b_dt) if b_dt is not None else None
        grad_x = grad_x.transpose(0, 1).reshape(*ctx.lead, groups, in_features).to(x_dt)
        return grad_x, grad_w.to(w_dt), grad_b


def grouped_linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """Per-group Linear over the second-to-last axis via one batched GEMM (bmm / baddbmm semantics,
    tests/test_training_smoke.py:28-37).  Operands of every product are contiguous (see
    ``_GroupedLinearBmm``)."""
    return _GroupedLinearBmm.apply(x, weight, bias)


def _prefix(widths):
    off = [0]
    for w in widths:
        off.append(off[-1] + int(w))
    return off


def _equal_runs(widths):
    runs, start = [], 0
    for i in range(1, len(widths) + 1):
        if i == len(widths) or widths[i] != widths[start]:
            runs.append((start, i, int(widths[start])))
            start = i
    return runs


def _stack_params(tensors, device, dtype):
    return torch.stack([t.to(device=device, dtype=dtype) for t in tensors], dim=0)


class BandSplit(nn.Module):
    def __init__(self, dim: int, dim_inputs):
        super().__init__()
        self.dim = dim
        self.dim_inputs = tuple(int(d) for d in dim_inputs)
        self.to_features = nn.ModuleList([nn.Sequential(RMSNorm(d), nn.Linear(d, dim)) for d in self.dim_inputs])
        self._dim_offsets = _prefix(self.dim_inputs)
        self._dim_groups = _equal_runs(self.dim_inputs)
        self._group_cache: dict = {}

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """``x[..., F]`` -> ``[..., NB, dim]``."""
        if not self.training or _grouped_in_training():
            return self._forward_grouped(x)
        return self._forward_bands(x)

    def _forward_bands(self, x: torch.Tensor) -> torch.Tensor:
        outs = [net(part) for part, net in zip(x.split(list(self.dim_inputs), dim=-1), self.to_features)]
        return torch.stack(outs, dim=-2)

    def _get_group_params(self, start: int, end: int, device, dtype):
        key = (start, end, device.type, device.index, dtype)
        if not self.training:
            hit = self._group_cache.get(key)
            if hit is not None:
                return hit
        nets = self.to_features[start:end]
        gamma = _stack_params([n[0].gamma for n in nets], device, dtype)
        weight = _stack_params([n[1].weight for n in nets], device, dtype)
        bias = _stack_params([n[1].bias for n in nets], device, dtype) if nets[0][1].bias is not None else None
        out = (gamma, weight, bias)
        if not self.training:
            self._group_cache[key] = out
        return out

    def _forward_grouped(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        outs = []
        for start, end, width in self._dim_groups:
            part = x[..., self._dim_offsets[start] : self._dim_offsets[end]].reshape(*lead, end - start, width)
            gamma, weight, bias = self._get_group_params(start, end, x.device, x.dtype)
            normed = F.normalize(part, dim=-1) * (width**0.5) * gamma
            outs.append(grouped_linear(normed, weight, bias))
        return torch.cat(outs, dim=-2)

    def train(self, mode: bool = True):
        self._group_cache.clear()
        return super().train(mode)


def MLP(dim_in: int, dim_out: int, dim_hidden: int | None = None, depth: int = 1) -> nn.Sequential:
    """``Linear -> Tanh -> ... -> Linear`` with ``depth`` Linear layers."""
    dim_hidden = dim_hidden or dim_in
    dims = (dim_in, *((dim_hidden,) * (depth - 1)), dim_out)
    layers = []
    for i, (a, b) in enumerate(zip(dims[:-1], dims[1:])):
        layers.append(nn.Linear(a, b))
        if i < len(dims) - 2:
            layers.append(nn.Tanh())
    return nn.Sequential(*layers)


class MaskEstimator(nn.Module):
    def __init__(self, dim: int, dim_inputs, depth: int, mlp_expansion_factor: int = 4):
        super().__init__()
        self.dim = dim
        self.dim_inputs = tuple(int(d) for d in dim_inputs)
        hidden = dim * mlp_expansion_factor
        self.to_freqs = nn.ModuleList(
            [nn.Sequential(MLP(dim, d * 2, dim_hidden=hidden, depth=depth), nn.GLU(dim=-1)) for d in self.dim_inputs]
        )
        self._dim_offsets = _prefix(self.dim_inputs)
        self._dim_total = self._dim_offsets[-1]
        self._group_cache: dict = {}
        self._layer_group_cache: dict = {}
        self._packed_layer_group_cache: dict = {}
        self._index_cache: dict = {}

    # ---------------------------------------------------------------- grouping plan
    def _band_groupable_layers(self):
        """Per band: ``[(kind, module)]`` with kind ``"linear"`` or ``"tanh"``."""
        out = []
        for seq in self.to_freqs:
            out.append([("linear", m) if isinstance(m, nn.Linear) else ("tanh", m) for m in seq[0]])
        return out

    def _layer_grouping_plan(self):
        """``[(kind, groups)]``; for linear layers ``groups = [((in, out), band_indices), ...]``."""
        layers = self._band_groupable_layers()
        if not layers or any(len(l) != len(layers[0]) for l in layers):
            return None
        plan = []
        for li in range(len(layers[0])):
            kinds = {band[li][0] for band in layers}
            if len(kinds) != 1:
                return None
            kind = kinds.pop()
            if kind == "tanh":
                plan.append(("tanh", None))
                continue
            groups: dict = {}
            for b, band in enumerate(layers):
                lin = band[li][1]
                groups.setdefault((lin.in_features, lin.out_features), []).append(b)
            plan.append(("linear", [(sig, tuple(idx)) for sig, idx in groups.items()]))
        return plan

    def _indices_tensor(self, indices, device):
        key = (tuple(indices), device.type, device.index)
        hit = self._index_cache.get(key)
        if hit is None:
            with torch.inference_mode(False):  # cached for training steps too
                hit = torch.as_tensor(indices, dtype=torch.long, device=device)
            self._index_cache[key] = hit
        return hit

    def _get_layer_group_params(self, layer_index, signature, indices, device, dtype):
        key = (layer_index, signature, tuple(indices), device.type, device.index, dtype)
        if not self.training:
            hit = self._layer_group_cache.get(key)
            if hit is not None:
                return hit
        layers = self._band_groupable_layers()
        lins = [layers[b][layer_index][1] for b in indices]
        weight = _stack_params([l.weight for l in lins], device, dtype)
        bias = _stack_params([l.bias for l in lins], device, dtype) if lins[0].bias is not None else None
        if not self.training:
            self._layer_group_cache[key] = (weight, bias)
        return weight, bias

    def _get_group_params(self, start, end, device, dtype):
        """All layers of bands ``[start, end)`` stacked: ``(("linear", W, b) | ("tanh", None, None), ...)``."""
        layers = self._band_groupable_layers()
        out = []
        for li, (kind, _) in enumerate(layers[start]):
            if kind == "tanh":
                out.append(("tanh", None, None))
                continue
            w, b = self._get_layer_group_params(li, None, tuple(range(start, end)), device, dtype)
            out.append(("linear", w, b))
        return tuple(out)

    # ---------------------------------------------------------------- forward
    def _forward_layer_grouped_mlp(self, x: torch.Tensor):
        plan = self._layer_grouping_plan()
        if plan is None:
            return None
        h = x
        for li, (kind, groups) in enumerate(plan):
            if kind == "tanh":
                h = inference_tanh(h)
                continue
            last = li == len(plan) - 1
            if len(groups) == 1 and not last:
                (sig, idx), = groups
                w, b = self._get_layer_group_params(li, sig, idx, x.device, x.dtype)
                h = grouped_linear(h, w, b)
                continue
            if not last:
                out_dims = {sig[1] for sig, _ in groups}
                if len(out_dims) != 1:
                    return None
                nxt = None
                for sig, idx in groups:
                    w, b = self._get_layer_group_params(li, sig, idx, x.device, x.dtype)
                    y = grouped_linear(h.index_select(-2, self._indices_tensor(idx, x.device)), w, b)
                    if nxt is None:
                        nxt = y.new_empty(*h.shape[:-1], y.shape[-1])
                    nxt.index_copy_(-2, self._indices_tensor(idx, x.device), y)
                h = nxt
                continue
            outs = [None] * len(self.to_freqs)
            for sig, idx in groups:
                w, b = self._get_layer_group_params(li, sig, idx, x.device, x.dtype)
                y = F.glu(grouped_linear(h.index_select(-2, self._indices_tensor(idx, x.device)), w, b), dim=-1)
                for pos, band in zip(idx, y.unbind(dim=-2)):
                    outs[pos] = band
            return torch.cat(outs, dim=-1)
        return None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """``x[..., NB, dim]`` -> ``[..., F]`` (per-band GLU outputs concatenated)."""
        out = self._forward_layer_grouped_mlp(x)
        if out is not None:
            return out
        return torch.cat([mlp(xb) for xb, mlp in zip(x.unbind(dim=-2), self.to_freqs)], dim=-1)

    def train(self, mode: bool = True):
        self._group_cache.clear()
        self._layer_group_cache.clear()
        self._packed_layer_group_cache.clear()
        return super().train(mode)

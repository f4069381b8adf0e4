"""Per-band parameters kept in one flat storage per kind, read in place by the kernels.

A band module owns many small parameters of one kind -- the 62 band-split Linear weights, the 62
RMSNorm gammas, the first-layer weights of the 62 mask MLPs -- and the kernels want each kind as one
band-major buffer (the ``[O, I_b]`` matrices back to back).  Stacking or concatenating them every
step costs one copy per parameter kind per step, plus a cast under autocast.

:class:`FlatParams` moves the parameters of one kind into a single flat storage once and re-points
each ``nn.Parameter`` at its slice (``param.data`` becomes a view), so the parameters, their names in
the state dict and the optimizer's view of them are unchanged while their bytes are contiguous.
:meth:`FlatParams.flat` hands that storage to autograd as one tensor in the compute dtype (at most
one cast per optimizer step, cached on the version counters of the parameters and the storage) whose
backward splits the flat gradient back into per-parameter gradients.  Writes through ``param.data``
bypass every version counter: after them, :meth:`FlatParams.invalidate` (or :func:`invalidate_casts` on
the module) drops the cached casts.  :meth:`FlatParams.group` does the same for a
contiguous run of equal-shaped parameters, stacked ``[G, ...]`` without a copy.

If a parameter stops being a view of the storage (``module.to(...)`` after packing, a state dict
loaded with ``assign=True``), :func:`pack` builds a new storage on the next call.
"""

from __future__ import annotations

from typing import Sequence

import torch
from torch import nn

__all__ = ["FlatParams", "pack", "band_split_packs", "mask_layer_packs", "invalidate_casts"]


class FlatParams:
    """Parameters ``params[i]`` stored at ``[starts[i], starts[i] + numel_i)`` of one flat tensor."""

    def __init__(self, params: Sequence[nn.Parameter]):
        params = list(params)
        if not params:
            raise ValueError("FlatParams needs at least one parameter")
        dev, dt = params[0].device, params[0].dtype
        if any(p.device != dev or p.dtype != dt for p in params):
            raise ValueError("packed parameters must share one device and dtype")
        self.params = params
        self.shapes = [tuple(p.shape) for p in params]
        self.sizes = [p.numel() for p in params]
        self.starts = [0]
        for n in self.sizes:
            self.starts.append(self.starts[-1] + n)
        # a pack first built under torch.inference_mode() (a validation pass) must still hold normal
        # tensors: the parameters are re-pointed at this storage for good, and training saves them
        with torch.inference_mode(False):
            storage = torch.empty(self.starts[-1], device=dev, dtype=dt)
            with torch.no_grad():
                for p, a, n in zip(params, self.starts, self.sizes):
                    storage[a : a + n].copy_(p.detach().reshape(-1))
            for p, a, n, shape in zip(params, self.starts, self.sizes, self.shapes):
                p.data = storage[a : a + n].view(shape)
        self.storage = storage
        self._casts: dict = {}

    def intact(self) -> bool:
        """Every parameter is still the view of the storage it was packed into."""
        base = self.storage.data_ptr()
        esz = self.storage.element_size()
        for p, a, shape in zip(self.params, self.starts, self.shapes):
            if (p.device != self.storage.device or p.dtype != self.storage.dtype or p.data_ptr() != base + a * esz
                    or tuple(p.shape) != shape):
                return False
        return True

    def _values(self, dtype: torch.dtype) -> torch.Tensor:
        """The storage in ``dtype``: the storage itself, or a cast cached until the values change.

        The cache key holds the version counters of the storage and of every parameter: an in-place
        update of a parameter (the optimizer step, ``load_state_dict``) or of the storage bumps one of
        them.  A write through ``param.data`` bumps none; code that writes that way calls
        :meth:`invalidate` afterwards.  The cast is made outside inference mode, so one made during an
        inference-mode validation pass can serve the next training step."""
        if dtype == self.storage.dtype:
            return self.storage.detach()
        key = (dtype, self.storage._version, tuple(p._version for p in self.params))
        hit = self._casts.get(dtype)
        if hit is None or hit[0] != key:
            with torch.inference_mode(False):
                hit = (key, self.storage.detach().to(dtype))
            self._casts = {dtype: hit}
        return hit[1]

    def invalidate(self) -> None:
        """Drop the cached casts (after writes that bypass the version counters, such as ``p.data.copy_``)."""
        self._casts = {}

    def flat(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        """All parameters as one flat tensor in ``dtype`` (default: theirs), differentiable with respect
        to each parameter."""
        return _FlatView.apply(self, 0, len(self.params), dtype or self.storage.dtype, *self.params)

    def group(self, start: int, end: int, dtype: torch.dtype | None = None) -> torch.Tensor:
        """Parameters ``[start, end)`` (equal shapes) stacked as ``[end - start, *shape]`` without a copy."""
        shape = self.shapes[start]
        if any(s != shape for s in self.shapes[start:end]):
            raise ValueError("group() needs parameters of one shape")
        t = _FlatView.apply(self, start, end, dtype or self.storage.dtype, *self.params[start:end])
        return t.view(end - start, *shape)


class _FlatView(torch.autograd.Function):
    """Forward: slice ``[starts[a], starts[b])`` of the (cast) storage; backward: that slice's gradient
    split into the parameters' shapes and dtype."""

    @staticmethod
    def forward(ctx, pack: FlatParams, a: int, b: int, dtype: torch.dtype, *params):
        ctx.pack, ctx.a, ctx.b = pack, a, b
        return pack._values(dtype)[pack.starts[a] : pack.starts[b]].view(-1)

    @staticmethod
    def backward(ctx, grad):
        pack, a, b = ctx.pack, ctx.a, ctx.b
        g = grad.to(pack.storage.dtype).contiguous()
        grads = [v.view(s) for v, s in zip(g.split(pack.sizes[a:b]), pack.shapes[a:b])]
        return (None, None, None, None, *grads)


def pack(module: nn.Module, key: str, params: Sequence[nn.Parameter]) -> FlatParams:
    """The module's :class:`FlatParams` for ``key``, built (or rebuilt) when missing or no longer intact."""
    packs = module.__dict__.setdefault("_pymsst_packs", {})
    params = list(params)
    hit = packs.get(key)
    same = hit is not None and len(hit.params) == len(params) and all(a is b for a, b in zip(hit.params, params))
    if not same or not hit.intact():
        hit = packs[key] = FlatParams(params)
    return hit


def band_split_packs(module) -> tuple[FlatParams, FlatParams, FlatParams | None]:
    """``(gamma, weight, bias | None)`` packs of a ``BandSplit``: band-major ``gamma[F]``, the ``[O, I_b]``
    weights back to back and ``bias[NB, O]``."""
    nets = list(module.to_features)
    gamma = pack(module, "band_split.gamma", [n[0].gamma for n in nets])
    weight = pack(module, "band_split.weight", [n[1].weight for n in nets])
    bias = None
    if all(n[1].bias is not None for n in nets):
        bias = pack(module, "band_split.bias", [n[1].bias for n in nets])
    return gamma, weight, bias


def mask_layer_packs(module, layer_index: int) -> tuple[FlatParams, FlatParams | None]:
    """``(weight, bias | None)`` packs of Linear layer ``layer_index`` of every band's mask MLP."""
    lins = [band[layer_index][1] for band in module._band_groupable_layers()]
    weight = pack(module, f"mask.{layer_index}.weight", [l.weight for l in lins])
    bias = None
    if all(l.bias is not None for l in lins):
        bias = pack(module, f"mask.{layer_index}.bias", [l.bias for l in lins])
    return weight, bias


def invalidate_casts(module: nn.Module) -> None:
    """Drop the cached compute-dtype casts of every pack under ``module`` (after ``param.data`` writes)."""
    for sub in module.modules():
        for fp in sub.__dict__.get("_pymsst_packs", {}).values():
            fp.invalidate()

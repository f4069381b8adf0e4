"""Torch-facing extension object with the reference's op names, backed by the C ABI.

``HipFusedExtension`` is the MI355X counterpart of the reference's pybind11
module ``pymsst_fused_band_split`` (baicai-1145/pymsst
``src/pymsst/training/cuda/fused_band_split.cpp:731-753``): the same op names,
argument order, return lists and argument checks (raised as ``RuntimeError``
with the reference's messages, ``.cpp:141-729``).  Outputs are allocated here
with ``torch.empty`` on the input's device and every kernel is enqueued on
torch's current stream for that device.  Ops this build adds beyond the
reference (saved-input RMSNorm backward, fused q/k norm + rotary, ...) carry
docstrings saying so.

There is no CPU or PyTorch fallback in this module: every op runs the HIP
kernels or raises.
"""

from __future__ import annotations

import ctypes
from typing import NamedTuple

import torch

from . import _lib
from ._lib import PmsstError, check, dtype_code


class BandRowsPlan(NamedTuple):
    """Device tables of a mel band layout (see ``HipFusedExtension.band_rows_plan``)."""

    rows: torch.Tensor
    row_start: torch.Tensor
    sources: torch.Tensor
    divisor: torch.Tensor
    num_rows: int
    num_sel: int


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def _stream(device: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


class _DeviceGuard:
    __slots__ = ("dev", "prev")

    def __init__(self, device: torch.device):
        self.dev = device.index
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if self.dev is not None and cur != self.dev:
            self.prev = cur
            torch.cuda.set_device(self.dev)
        return self

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)
        return False


def _activation_code(name) -> int:
    if name is None or name == "none":
        return 0  # PMSST_ACT_NONE
    if name == "tanh":
        return 1  # PMSST_ACT_TANH
    raise ValueError(f"unsupported activation {name!r}")


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


class HipFusedExtension:
    """Duck-typed replacement for the reference's extension module (``fr.py:71`` ``extension=``)."""

    rotary_out_layouts = ("bnhd", "bhnd")

    def __init__(self):
        self._lib = _lib.load_library()
        self._band_cache = {}

    # ------------------------------------------------------------------ RMSNorm

    def _rms_check_fwd(self, x, gamma, fp32_gamma: bool):
        _req(x.is_cuda, "x must be a CUDA tensor")
        _req(gamma.is_cuda, "gamma must be a CUDA tensor")
        _req(x.dim() >= 2, "x must have at least 2 dimensions")
        _req(gamma.dim() == 1, "gamma must have shape [D]")
        _req(gamma.size(0) == x.size(-1), "gamma dimension must match x last dimension")
        if fp32_gamma:
            _req(gamma.dtype == torch.float32, "gamma must be float32")
        else:
            _req(gamma.dtype == x.dtype, "gamma dtype must match x")

    def _rms_fwd(self, fn_name, x, gamma, out_dtype, write_normed=True):
        x = x.contiguous()
        gamma = gamma.contiguous()
        dim = x.size(-1)
        rows = x.numel() // dim if dim else 0
        out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
        normed = torch.empty(x.shape, dtype=out_dtype, device=x.device) if write_normed else None
        inv = torch.empty((rows,), dtype=torch.float32, device=x.device)
        with _DeviceGuard(x.device):
            rc = getattr(self._lib, fn_name)(
                _ptr(x), _ptr(gamma), _ptr(out), _ptr(normed), _ptr(inv), rows, dim, dtype_code(x.dtype),
                _stream(x.device),
            )
        check(rc, fn_name)
        return [out, normed, inv] if write_normed else [out, inv]

    def _rms_check_bwd(self, grad_out, normed, inv_norm, gamma):
        _req(grad_out.is_cuda, "grad_out must be a CUDA tensor")
        _req(normed.is_cuda, "normed must be a CUDA tensor")
        _req(inv_norm.is_cuda, "inv_norm must be a CUDA tensor")
        _req(gamma.is_cuda, "gamma must be a CUDA tensor")
        _req(grad_out.dim() >= 2, "grad_out must have at least 2 dimensions")
        _req(normed.shape == grad_out.shape, "normed shape must match grad_out")
        _req(gamma.dim() == 1, "gamma must have shape [D]")
        _req(gamma.size(0) == grad_out.size(-1), "gamma dimension must match grad_out last dimension")
        _req(inv_norm.dim() == 1, "inv_norm must have shape [M]")
        _req(inv_norm.size(0) * gamma.size(0) == grad_out.numel(), "inv_norm length must match flattened rows")
        _req(inv_norm.dtype == torch.float32, "inv_norm must be float32")

    def _rms_bwd(self, fn_name, grad_out, nsrc, inv_norm, gamma, dx_dtype, dgamma_dtype, extra_dtype=None):
        grad_out = grad_out.contiguous()
        nsrc = nsrc.contiguous()
        gamma = gamma.contiguous()
        inv_norm = inv_norm.contiguous()
        dim = grad_out.size(-1)
        rows = grad_out.numel() // dim if dim else 0
        dx = torch.empty(grad_out.shape, dtype=dx_dtype, device=grad_out.device)
        dgamma = torch.empty((dim,), dtype=dgamma_dtype, device=grad_out.device)
        ws_bytes = self._lib.pmsst_rms_norm_backward_workspace_size(rows, dim)
        ws = _workspace(ws_bytes, grad_out.device)
        args = [_ptr(grad_out), _ptr(nsrc), _ptr(inv_norm), _ptr(gamma), _ptr(dx), _ptr(dgamma), rows, dim]
        if fn_name == "pmsst_rms_norm_backward_mixed":
            args.append(dtype_code(dx_dtype))
        elif fn_name == "pmsst_rms_norm_backward_from_input":
            args += [dtype_code(grad_out.dtype), dtype_code(extra_dtype)]
        else:
            args.append(dtype_code(grad_out.dtype))
        args += [_ptr(ws), ws.numel(), _stream(grad_out.device)]
        with _DeviceGuard(grad_out.device):
            rc = getattr(self._lib, fn_name)(*args)
        check(rc, fn_name)
        return [dx, dgamma]

    def rms_norm_forward(self, x, gamma):
        """``.cpp:434-444``: returns ``[out, normed, inv_norm]`` (x, gamma same dtype)."""
        self._rms_check_fwd(x, gamma, fp32_gamma=False)
        return self._rms_fwd("pmsst_rms_norm_forward", x, gamma, x.dtype)

    def rms_norm_backward(self, grad_out, normed, inv_norm, gamma):
        """``.cpp:446-465``: returns ``[grad_x, grad_gamma]``."""
        self._rms_check_bwd(grad_out, normed, inv_norm, gamma)
        _req(normed.dtype == grad_out.dtype, "normed dtype must match grad_out")
        _req(gamma.dtype == grad_out.dtype, "gamma dtype must match grad_out")
        return self._rms_bwd("pmsst_rms_norm_backward", grad_out, normed, inv_norm, gamma, grad_out.dtype,
                             grad_out.dtype)

    def rms_norm_forward_fp32_gamma(self, x, gamma):
        """``.cpp:467-477``: fp32 gamma, outputs in x dtype."""
        self._rms_check_fwd(x, gamma, fp32_gamma=True)
        return self._rms_fwd("pmsst_rms_norm_forward_fp32_gamma", x, gamma, x.dtype)

    def rms_norm_backward_fp32_gamma(self, grad_out, normed, inv_norm, gamma):
        """``.cpp:479-498``: fp32 gamma and grad_gamma."""
        self._rms_check_bwd(grad_out, normed, inv_norm, gamma)
        _req(normed.dtype == grad_out.dtype, "normed dtype must match grad_out")
        _req(gamma.dtype == torch.float32, "gamma must be float32")
        return self._rms_bwd("pmsst_rms_norm_backward_fp32_gamma", grad_out, normed, inv_norm, gamma,
                             grad_out.dtype, torch.float32)

    def rms_norm_forward_mixed(self, x, gamma):
        """``.cpp:500-510``: x in its dtype, fp32 gamma, fp32 ``out``/``normed``."""
        self._rms_check_fwd(x, gamma, fp32_gamma=True)
        return self._rms_fwd("pmsst_rms_norm_forward_mixed", x, gamma, torch.float32)

    def rms_norm_backward_mixed(self, grad_out, normed, inv_norm, gamma, x_meta):
        """``.cpp:512-534``: fp32 grad_out/normed/gamma; grad_x in ``x_meta.dtype``."""
        self._rms_check_bwd(grad_out, normed, inv_norm, gamma)
        _req(x_meta.is_cuda, "x_meta must be a CUDA tensor")
        _req(grad_out.dtype == torch.float32, "grad_out must be float32")
        _req(normed.dtype == torch.float32, "normed must be float32")
        _req(gamma.dtype == torch.float32, "gamma must be float32")
        return self._rms_bwd("pmsst_rms_norm_backward_mixed", grad_out, normed, inv_norm, gamma, x_meta.dtype,
                             torch.float32)

    def rms_norm_forward_lean(self, x, gamma):
        """Build addition: RMSNorm forward that skips writing ``normed``; returns ``[out, inv_norm]``.

        ``gamma`` is in x's dtype or fp32; ``out`` is in x's dtype.  Pair with
        :meth:`rms_norm_backward_from_input`, which recomputes ``normed`` from x.
        """
        self._rms_check_fwd(x, gamma, fp32_gamma=gamma.dtype == torch.float32)
        name = "pmsst_rms_norm_forward_fp32_gamma" if gamma.dtype == torch.float32 else "pmsst_rms_norm_forward"
        return self._rms_fwd(name, x, gamma, x.dtype, write_normed=False)

    def rms_norm_backward_from_input(self, grad_out, x, inv_norm, gamma):
        """Build addition: RMSNorm backward from the saved input (``normed = x*inv*sqrt(D)`` recomputed)."""
        self._rms_check_bwd(grad_out, x, inv_norm, gamma)
        _req(x.dtype == grad_out.dtype, "x dtype must match grad_out")
        _req(gamma.dtype in (grad_out.dtype, torch.float32), "gamma dtype must match grad_out or be float32")
        return self._rms_bwd("pmsst_rms_norm_backward_from_input", grad_out, x, inv_norm, gamma, grad_out.dtype,
                             gamma.dtype, extra_dtype=gamma.dtype)

    # ------------------------------------------------------------------ rotary

    @staticmethod
    def _rot_check(t, cos, sin, tname: str):
        _req(t.is_cuda, f"{tname} must be a CUDA tensor")
        _req(cos.is_cuda, "cos must be a CUDA tensor")
        _req(sin.is_cuda, "sin must be a CUDA tensor")
        _req(t.dim() == 4, f"{tname} must have shape [B, N, H, D]")
        _req(cos.dim() == 4, "cos must have shape [1, N, 1, D/2]")
        _req(sin.dim() == 4, "sin must have shape [1, N, 1, D/2]")
        _req(t.size(3) % 2 == 0, f"{tname} last dimension must be even")
        _req(cos.size(0) == 1 and cos.size(2) == 1, "cos must broadcast over batch and heads")
        _req(sin.size(0) == 1 and sin.size(2) == 1, "sin must broadcast over batch and heads")
        _req(cos.size(1) == t.size(1), f"cos sequence dimension must match {tname}")
        _req(sin.size(1) == t.size(1), f"sin sequence dimension must match {tname}")
        _req(cos.size(3) == t.size(3) // 2, f"cos rotary dimension must match {tname}")
        _req(sin.size(3) == t.size(3) // 2, f"sin rotary dimension must match {tname}")
        _req(cos.dtype == t.dtype, f"cos dtype must match {tname}")
        _req(sin.dtype == t.dtype, f"sin dtype must match {tname}")

    @staticmethod
    def _tables(cos, sin):
        # One stride pair for both tables: make them agree if they do not.
        if cos.stride(1) != sin.stride(1) or cos.stride(3) != sin.stride(3):
            cos, sin = cos.contiguous(), sin.contiguous()

        def repeated_view_ok(t):
            # the kernels read a [..., ::2] table 16 bytes at a time, odd elements included:
            # they must lie inside the tensor's storage (true for a view of a [.., D] table)
            last = t.storage_offset() + (t.size(1) - 1) * t.stride(1) + 2 * t.size(3)
            return last * t.element_size() <= t.untyped_storage().nbytes()

        if cos.stride(3) == 2 and not (repeated_view_ok(cos) and repeated_view_ok(sin)):
            cos, sin = cos.contiguous(), sin.contiguous()
        return cos, sin, cos.stride(1), cos.stride(3)

    def _rotary(self, fn_name, t, cos, sin, out_layout="bnhd"):
        if t.stride(3) != 1:
            t = t.contiguous()
        cos, sin, s_seq, s_pair = self._tables(cos, sin)
        b, n, h, d = t.shape
        if out_layout == "bhnd":
            # [B, N, H, D]-shaped view of a dense [B, H, N, D] buffer
            out = torch.empty((b, h, n, d), dtype=t.dtype, device=t.device).transpose(1, 2)
        elif out_layout == "bnhd":
            out = torch.empty((b, n, h, d), dtype=t.dtype, device=t.device)
        else:
            raise ValueError(f"unsupported out_layout {out_layout!r}")
        t_strides = (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))
        o_strides = (ctypes.c_int64 * 3)(out.stride(0), out.stride(1), out.stride(2))
        with _DeviceGuard(t.device):
            rc = getattr(self._lib, fn_name)(
                _ptr(t), t_strides, _ptr(cos), _ptr(sin), _ptr(out), o_strides, b, n, h, d, s_seq, s_pair,
                dtype_code(t.dtype), _stream(t.device),
            )
        check(rc, fn_name)
        return out

    def rotary_forward(self, t, cos, sin, out_layout="bnhd"):
        """``.cpp:390-410``: ``t[B,N,H,D]`` (any strides with a contiguous last axis, e.g. a view
        into a fused qkv buffer), ``cos/sin[1,N,1,D/2]`` (strided views accepted).
        ``out_layout="bhnd"`` returns the ``[B,N,H,D]``-shaped transpose of a dense ``[B,H,N,D]``
        buffer, the layout attention consumes."""
        self._rot_check(t, cos, sin, "t")
        return self._rotary("pmsst_rotary_forward", t, cos, sin, out_layout)

    def rotary_backward(self, grad_out, cos, sin):
        """``.cpp:412-432``: transpose rotation of ``grad_out`` (any strides); dense bnhd result."""
        self._rot_check(grad_out, cos, sin, "grad_out")
        return self._rotary("pmsst_rotary_backward", grad_out, cos, sin)

    def rotary_qkv_forward(self, qkv, heads, cos, sin, out_layout="bhnd"):
        """Build addition: split a fused ``qkv[B, N, 3*H*D]`` projection and rotate q and k in one
        launch.  Returns ``(q, k, v)``, ``[B,N,H,D]``-shaped; v is copied unrotated.  With
        ``out_layout="bhnd"`` each is the transpose of a dense ``[B,H,N,D]`` buffer (what a
        ``.contiguous()`` of the ``[B,H,N,D]`` view would produce); with ``"bnhd"`` each is dense
        ``[B,N,H,D]``, the layout the flash-attention kernels read and write without copies."""
        _req(out_layout in ("bhnd", "bnhd"), f"unsupported out_layout {out_layout!r}")
        _req(qkv.is_cuda and qkv.dim() == 3, "qkv must be a CUDA tensor of shape [B, N, 3*H*D]")
        _req(qkv.size(2) % (3 * heads) == 0, "qkv last dimension must be 3 * heads * dim_head")
        if qkv.stride(2) != 1:
            qkv = qkv.contiguous()
        b, n, _ = qkv.shape
        d = qkv.size(2) // (3 * heads)
        q, k, v = qkv.view(b, n, 3, heads, d).unbind(2)
        self._rot_check(q, cos, sin, "q")
        cos, sin, s_seq, s_pair = self._tables(cos, sin)
        if out_layout == "bhnd":
            outs = [torch.empty((b, heads, n, d), dtype=qkv.dtype, device=qkv.device).transpose(1, 2) for _ in range(3)]
        else:
            outs = [torch.empty((b, n, heads, d), dtype=qkv.dtype, device=qkv.device) for _ in range(3)]
        ist = (ctypes.c_int64 * 9)(*[st for t in (q, k, v) for st in (t.stride(0), t.stride(1), t.stride(2))])
        ost = (ctypes.c_int64 * 9)(*[st for t in outs for st in (t.stride(0), t.stride(1), t.stride(2))])
        with _DeviceGuard(qkv.device):
            rc = self._lib.pmsst_rotary_qkv_forward(
                _ptr(q), _ptr(k), _ptr(v), ist, _ptr(cos), _ptr(sin), _ptr(outs[0]), _ptr(outs[1]), _ptr(outs[2]),
                ost, b, n, heads, d, s_seq, s_pair, dtype_code(qkv.dtype), _stream(qkv.device),
            )
        check(rc, "pmsst_rotary_qkv_forward")
        return tuple(outs)

    def rotary_qkv_backward(self, grad_q, grad_k, grad_v, cos, sin):
        """Build addition: backward of :meth:`rotary_qkv_forward`.  ``grad_q/k/v`` are
        ``[B,N,H,D]``-shaped with any strides and a contiguous last axis; returns the dense
        ``[B, N, 3*H*D]`` qkv gradient (q and k rotated back, v copied) from one launch."""
        grads = []
        for t in (grad_q, grad_k, grad_v):
            _req(t.is_cuda and t.dim() == 4 and t.shape == grad_q.shape and t.dtype == grad_q.dtype,
                 "grad_q, grad_k and grad_v must be CUDA tensors of one [B, N, H, D] shape and dtype")
            grads.append(t if t.stride(3) == 1 else t.contiguous())
        self._rot_check(grads[0], cos, sin, "grad_q")
        cos, sin, s_seq, s_pair = self._tables(cos, sin)
        b, n, h, d = grads[0].shape
        dqkv = torch.empty((b, n, 3 * h * d), dtype=grads[0].dtype, device=grads[0].device)
        parts = dqkv.view(b, n, 3, h, d).unbind(2)
        ist = (ctypes.c_int64 * 9)(*[st for t in grads for st in (t.stride(0), t.stride(1), t.stride(2))])
        ost = (ctypes.c_int64 * 9)(*[st for t in parts for st in (t.stride(0), t.stride(1), t.stride(2))])
        with _DeviceGuard(dqkv.device):
            rc = self._lib.pmsst_rotary_qkv_backward(
                _ptr(grads[0]), _ptr(grads[1]), _ptr(grads[2]), ist, _ptr(cos), _ptr(sin), _ptr(parts[0]),
                _ptr(parts[1]), _ptr(parts[2]), ost, b, n, h, d, s_seq, s_pair, dtype_code(dqkv.dtype),
                _stream(dqkv.device),
            )
        check(rc, "pmsst_rotary_qkv_backward")
        return dqkv

    def rms_norm_rotary_forward(self, x, gamma, cos, sin):
        """Build addition: fused q/k RMSNorm over the head dim + rotary + cast.

        ``x[B,N,H,D]`` in bf16/f16/f32, ``gamma[D]`` in x's dtype or fp32, tables as
        :meth:`rotary_forward`.  Returns ``[out, inv_norm[B*N*H]]``.
        """
        self._rot_check(x, cos, sin, "x")
        _req(gamma.is_cuda and gamma.dim() == 1 and gamma.size(0) == x.size(3), "gamma must have shape [D]")
        _req(gamma.dtype in (x.dtype, torch.float32), "gamma dtype must match x or be float32")
        x = x.contiguous()
        gamma = gamma.contiguous()
        cos, sin, s_seq, s_pair = self._tables(cos, sin)
        b, n, h, d = x.shape
        out = torch.empty_like(x)
        inv = torch.empty((b * n * h,), dtype=torch.float32, device=x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_rms_norm_rotary_forward(
                _ptr(x), _ptr(gamma), _ptr(cos), _ptr(sin), _ptr(out), _ptr(inv), b, n, h, d, s_seq, s_pair,
                dtype_code(x.dtype), dtype_code(gamma.dtype), _stream(x.device),
            )
        check(rc, "pmsst_rms_norm_rotary_forward")
        return [out, inv]

    def rms_norm_rotary_backward(self, grad_out, x, inv_norm, gamma, cos, sin):
        """Build addition: backward of :meth:`rms_norm_rotary_forward`; returns ``[grad_x, grad_gamma]``."""
        self._rot_check(grad_out, cos, sin, "grad_out")
        _req(x.shape == grad_out.shape and x.dtype == grad_out.dtype, "x must match grad_out")
        _req(inv_norm.dtype == torch.float32 and inv_norm.numel() * x.size(3) == x.numel(),
             "inv_norm length must match flattened rows")
        grad_out = grad_out.contiguous()
        x = x.contiguous()
        gamma = gamma.contiguous()
        cos, sin, s_seq, s_pair = self._tables(cos, sin)
        b, n, h, d = x.shape
        dx = torch.empty_like(x)
        dgamma = torch.empty((d,), dtype=gamma.dtype, device=x.device)
        ws_bytes = self._lib.pmsst_rms_norm_rotary_backward_workspace_size(b * n * h, d)
        ws = _workspace(ws_bytes, x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_rms_norm_rotary_backward(
                _ptr(grad_out), _ptr(x), _ptr(inv_norm), _ptr(gamma), _ptr(cos), _ptr(sin), _ptr(dx), _ptr(dgamma),
                b, n, h, d, s_seq, s_pair, dtype_code(x.dtype), dtype_code(gamma.dtype), _ptr(ws), ws.numel(),
                _stream(x.device),
            )
        check(rc, "pmsst_rms_norm_rotary_backward")
        return [dx, dgamma]


    def rms_norm_rotary_pair_forward(self, q, k, gamma_q, gamma_k, cos, sin):
        """:meth:`rms_norm_rotary_forward` on q and k (one shape, own gammas) in one launch.
        Returns ``[q_out, k_out, inv_q, inv_k]``."""
        _req(q.shape == k.shape and q.dtype == k.dtype and q.device == k.device, "q and k must match")
        _req(gamma_q.dtype == gamma_k.dtype and gamma_q.shape == gamma_k.shape, "gamma_q and gamma_k must match")
        self._rot_check(q, cos, sin, "q")
        _req(gamma_q.is_cuda and gamma_q.dim() == 1 and gamma_q.size(0) == q.size(3), "gamma must have shape [D]")
        _req(gamma_q.dtype in (q.dtype, torch.float32), "gamma dtype must match x or be float32")
        q, k = q.contiguous(), k.contiguous()
        gamma_q, gamma_k = gamma_q.contiguous(), gamma_k.contiguous()
        cos, sin, s_seq, s_pair = self._tables(cos, sin)
        b, n, h, d = q.shape
        qo, ko = torch.empty_like(q), torch.empty_like(k)
        inv = torch.empty((2, b * n * h), dtype=torch.float32, device=q.device)
        with _DeviceGuard(q.device):
            rc = self._lib.pmsst_rms_norm_rotary_pair_forward(
                _ptr(q), _ptr(k), _ptr(gamma_q), _ptr(gamma_k), _ptr(cos), _ptr(sin), _ptr(qo), _ptr(ko),
                _ptr(inv[0]), _ptr(inv[1]), b, n, h, d, s_seq, s_pair, dtype_code(q.dtype),
                dtype_code(gamma_q.dtype), _stream(q.device),
            )
        check(rc, "pmsst_rms_norm_rotary_pair_forward")
        return [qo, ko, inv[0], inv[1]]

    def rms_norm_rotary_pair_backward(self, grad_q, grad_k, q, k, inv_q, inv_k, gamma_q, gamma_k, cos, sin):
        """Backward of :meth:`rms_norm_rotary_pair_forward` in one launch (and one dgamma reduction).
        Returns ``[grad_q_in, grad_k_in, grad_gamma_q, grad_gamma_k]``."""
        _req(grad_q.shape == grad_k.shape == q.shape == k.shape, "q, k and their gradients must have one shape")
        _req(grad_q.dtype == grad_k.dtype == q.dtype == k.dtype, "q, k and their gradients must have one dtype")
        self._rot_check(grad_q, cos, sin, "grad_out")
        _req(inv_q.dtype == torch.float32 and inv_k.dtype == torch.float32 and inv_q.numel() * q.size(3) == q.numel()
             and inv_k.numel() == inv_q.numel(), "inv_norm length must match flattened rows")
        grad_q, grad_k, q, k = grad_q.contiguous(), grad_k.contiguous(), q.contiguous(), k.contiguous()
        gamma_q, gamma_k = gamma_q.contiguous(), gamma_k.contiguous()
        cos, sin, s_seq, s_pair = self._tables(cos, sin)
        b, n, h, d = q.shape
        dq, dk = torch.empty_like(q), torch.empty_like(k)
        dgamma = torch.empty((2, d), dtype=gamma_q.dtype, device=q.device)
        ws = _workspace(self._lib.pmsst_rms_norm_rotary_backward_workspace_size(b * n * h, 2 * d), q.device)
        with _DeviceGuard(q.device):
            rc = self._lib.pmsst_rms_norm_rotary_pair_backward(
                _ptr(grad_q), _ptr(grad_k), _ptr(q), _ptr(k), _ptr(inv_q.contiguous()), _ptr(inv_k.contiguous()),
                _ptr(gamma_q), _ptr(gamma_k), _ptr(cos), _ptr(sin), _ptr(dq), _ptr(dk), _ptr(dgamma), b, n, h, d,
                s_seq, s_pair, dtype_code(q.dtype), dtype_code(gamma_q.dtype), _ptr(ws), ws.numel(), _stream(q.device),
            )
        check(rc, "pmsst_rms_norm_rotary_pair_backward")
        return [dq, dk, dgamma[0], dgamma[1]]

    # ------------------------------------------------------------------ attention gate

    @staticmethod
    def _gate_common_checks(attn, x, weight):
        _req(attn.size(-2) == weight.size(0), "attn heads must match weight")
        _req(weight.size(1) == x.size(1), "weight input dimension must match x")
        _req(x.dtype == attn.dtype, "x dtype must match attn")
        _req(weight.dtype == attn.dtype, "weight dtype must match attn")

    def _gate_fwd(self, attn4, x, weight, bias):
        if attn4.stride(3) != 1:
            attn4 = attn4.contiguous()
        x, weight, bias = x.contiguous(), weight.contiguous(), bias.contiguous()
        b, n, h, dh = attn4.shape
        out = torch.empty((b * n, h * dh), dtype=attn4.dtype, device=attn4.device)
        gate = torch.empty((b * n, h), dtype=attn4.dtype, device=attn4.device)
        st = (ctypes.c_int64 * 3)(attn4.stride(0), attn4.stride(1), attn4.stride(2))
        with _DeviceGuard(attn4.device):
            rc = self._lib.pmsst_attention_gate_forward(
                _ptr(attn4), st, _ptr(x), _ptr(weight), _ptr(bias), _ptr(out), _ptr(gate), b, n, h, dh, x.size(1),
                dtype_code(attn4.dtype), _stream(attn4.device),
            )
        check(rc, "pmsst_attention_gate_forward")
        return out, gate, attn4, x

    def _gate_bwd(self, grad_out, attn4, x, weight, gate, out_layout):
        if attn4.stride(3) != 1:
            attn4 = attn4.contiguous()
        grad_out, x, weight, gate = grad_out.contiguous(), x.contiguous(), weight.contiguous(), gate.contiguous()
        b, n, h, dh = attn4.shape
        if out_layout == "bhnd":
            grad_attn = torch.empty((b, h, n, dh), dtype=attn4.dtype, device=attn4.device).transpose(1, 2)
        else:
            grad_attn = torch.empty((b, n, h, dh), dtype=attn4.dtype, device=attn4.device)
        grad_x = torch.empty_like(x)
        grad_weight = torch.empty_like(weight)
        grad_bias = torch.empty((h,), dtype=attn4.dtype, device=attn4.device)
        ws = _workspace(self._lib.pmsst_attention_gate_backward_workspace_size(b * n, h, x.size(1)), attn4.device)
        ast = (ctypes.c_int64 * 3)(attn4.stride(0), attn4.stride(1), attn4.stride(2))
        gst = (ctypes.c_int64 * 3)(grad_attn.stride(0), grad_attn.stride(1), grad_attn.stride(2))
        with _DeviceGuard(attn4.device):
            rc = self._lib.pmsst_attention_gate_backward(
                _ptr(grad_out), _ptr(attn4), ast, _ptr(x), _ptr(weight), _ptr(gate), _ptr(grad_attn), gst,
                _ptr(grad_x), _ptr(grad_weight), _ptr(grad_bias), b, n, h, dh, x.size(1), dtype_code(attn4.dtype),
                _ptr(ws), ws.numel(), _stream(attn4.device),
            )
        check(rc, "pmsst_attention_gate_backward")
        return grad_attn, grad_x, grad_weight, grad_bias

    def attention_gate_forward(self, attn, x, weight, bias):
        """``.cpp:536-557``: ``attn[M,H,Dh]``, ``x[M,D]``, ``weight[H,D]``, ``bias[H]`` ->
        ``[out[M, H*Dh], gate[M,H], attn, x]`` (the last two are what backward takes)."""
        _req(attn.is_cuda, "attn must be a CUDA tensor")
        _req(x.is_cuda, "x must be a CUDA tensor")
        _req(weight.is_cuda, "weight must be a CUDA tensor")
        _req(bias.is_cuda, "bias must be a CUDA tensor")
        _req(attn.dim() == 3, "attn must have shape [M, H, DH]")
        _req(x.dim() == 2, "x must have shape [M, D]")
        _req(weight.dim() == 2, "weight must have shape [H, D]")
        _req(bias.dim() == 1, "bias must have shape [H]")
        _req(attn.size(0) == x.size(0), "attn and x row counts must match")
        self._gate_common_checks(attn, x, weight)
        _req(bias.size(0) == weight.size(0), "bias heads must match weight")
        _req(bias.dtype == attn.dtype, "bias dtype must match attn")
        out, gate, a4, xs = self._gate_fwd(attn.unsqueeze(0), x, weight, bias)
        return [out, gate, a4.squeeze(0), xs]

    def attention_gate_backward(self, grad_out, attn, x, weight, gate):
        """``.cpp:559-587``: returns ``[grad_attn[M,H,Dh], grad_x[M,D], grad_weight[H,D], grad_bias[H]]``."""
        _req(grad_out.is_cuda, "grad_out must be a CUDA tensor")
        _req(attn.is_cuda, "attn must be a CUDA tensor")
        _req(x.is_cuda, "x must be a CUDA tensor")
        _req(weight.is_cuda, "weight must be a CUDA tensor")
        _req(gate.is_cuda, "gate must be a CUDA tensor")
        _req(grad_out.dim() == 2, "grad_out must have shape [M, H*DH]")
        _req(attn.dim() == 3, "attn must have shape [M, H, DH]")
        _req(x.dim() == 2, "x must have shape [M, D]")
        _req(weight.dim() == 2, "weight must have shape [H, D]")
        _req(gate.dim() == 2, "gate must have shape [M, H]")
        _req(grad_out.size(0) == attn.size(0), "grad_out rows must match attn")
        _req(grad_out.size(1) == attn.size(1) * attn.size(2), "grad_out columns must match flattened attn")
        _req(attn.size(0) == x.size(0), "attn and x row counts must match")
        _req(gate.size(0) == attn.size(0), "gate rows must match attn")
        _req(gate.size(1) == attn.size(1), "gate heads must match attn")
        _req(attn.dtype == grad_out.dtype, "attn dtype must match grad_out")
        self._gate_common_checks(attn, x, weight)
        _req(gate.dtype == grad_out.dtype, "gate dtype must match grad_out")
        ga, gx, gw, gb = self._gate_bwd(grad_out, attn.unsqueeze(0), x, weight, gate, "bnhd")
        return [ga.squeeze(0), gx, gw, gb]

    def attention_gate_forward_bnhd(self, attn, x, weight, bias):
        """Build addition: :meth:`attention_gate_forward` on ``attn[B,N,H,Dh]`` with any strides and a
        contiguous last axis (the transposed SDPA output, read in place); ``x[B*N, D]``."""
        _req(attn.is_cuda and attn.dim() == 4, "attn must be a CUDA tensor of shape [B, N, H, DH]")
        _req(x.is_cuda and x.dim() == 2 and x.size(0) == attn.size(0) * attn.size(1), "x must have shape [B*N, D]")
        _req(weight.is_cuda and weight.dim() == 2 and bias.is_cuda and bias.dim() == 1, "bad weight/bias")
        self._gate_common_checks(attn, x, weight)
        _req(bias.size(0) == weight.size(0) and bias.dtype == attn.dtype, "bias must be [H] in attn's dtype")
        return list(self._gate_fwd(attn, x, weight, bias))

    def attention_gate_backward_bnhd(self, grad_out, attn, x, weight, gate, out_layout="bhnd"):
        """Build addition: backward of :meth:`attention_gate_forward_bnhd`; ``grad_attn`` comes back
        ``[B,N,H,Dh]``-shaped, as the transpose of a dense ``[B,H,N,Dh]`` buffer (``out_layout="bhnd"``)
        or dense (``"bnhd"``, the layout the flash-attention backward reads without a copy)."""
        _req(grad_out.is_cuda and grad_out.dim() == 2, "grad_out must have shape [B*N, H*DH]")
        _req(grad_out.size(0) == attn.size(0) * attn.size(1) and grad_out.size(1) == attn.size(2) * attn.size(3),
             "grad_out must match attn")
        _req(gate.dtype == grad_out.dtype == attn.dtype, "gate/grad_out dtype must match attn")
        self._gate_common_checks(attn, x, weight)
        _req(out_layout in ("bhnd", "bnhd"), f"unsupported out_layout {out_layout!r}")
        return list(self._gate_bwd(grad_out, attn, x, weight, gate, out_layout))

    # ------------------------------------------------------------------ mel band rows

    @staticmethod
    def band_rows_plan(rows, num_rows: int, device):
        """Build-addition helper: device tables of a band layout (``rows[j]`` = spectrum row of
        selection ``j``, bands in order) for :meth:`band_rows_gather` / :meth:`band_rows_scatter`:
        the rows, their CSR by row (``row_start[num_rows + 1]``, ``sources`` = selections of each
        row in ascending order) and each selection's row count (fp32 divisor).  Validated here."""
        r = torch.as_tensor(rows, dtype=torch.int64).detach().cpu().reshape(-1)
        _req(num_rows > 0, "num_rows must be positive")
        _req(r.numel() == 0 or (int(r.min()) >= 0 and int(r.max()) < num_rows), "rows must lie in [0, num_rows)")
        counts = torch.bincount(r, minlength=num_rows)
        row_start = torch.zeros(num_rows + 1, dtype=torch.int64)
        row_start[1:] = torch.cumsum(counts, 0)
        sources = torch.argsort(r, stable=True)
        divisor = counts[r].to(torch.float32)
        dev = torch.device(device)
        return BandRowsPlan(r.to(dev), row_start.to(dev), sources.to(dev), divisor.to(dev), int(num_rows),
                            int(r.numel()))

    def band_rows_gather(self, x, plan, divide=False, out_dtype=None):
        """``x[B, R, T, 2]`` -> ``[B, T, J, 2]`` with ``out[b, t, j] = x[b, rows[j], t]`` (divided by the
        row's band count when ``divide``)."""
        _req(x.is_cuda and x.dim() == 4 and x.size(3) == 2 and x.size(1) == plan.num_rows,
             "x must be a CUDA tensor of shape [B, num_rows, T, 2]")
        x = x.contiguous()
        b, _, t, _ = x.shape
        out = torch.empty((b, t, plan.num_sel, 2), dtype=out_dtype or x.dtype, device=x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_band_rows_gather(
                _ptr(x), dtype_code(x.dtype), _ptr(plan.rows), _ptr(plan.divisor) if divide else None, _ptr(out),
                dtype_code(out.dtype), b, plan.num_rows, t, plan.num_sel, _stream(x.device),
            )
        check(rc, "pmsst_band_rows_gather")
        return out

    def band_rows_scatter(self, x, plan, mean=True, out_dtype=torch.float32):
        """``x[B, T, J, 2]`` -> ``[B, R, T, 2]``: per row the sum of its selections (the mean when
        ``mean``); rows no band selects are zero."""
        _req(x.is_cuda and x.dim() == 4 and x.size(3) == 2 and x.size(2) == plan.num_sel,
             "x must be a CUDA tensor of shape [B, T, num_sel, 2]")
        x = x.contiguous()
        b, t = x.shape[:2]
        out = torch.empty((b, plan.num_rows, t, 2), dtype=out_dtype, device=x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_band_rows_scatter(
                _ptr(x), dtype_code(x.dtype), _ptr(plan.row_start), _ptr(plan.sources), int(bool(mean)), _ptr(out),
                dtype_code(out.dtype), b, plan.num_rows, t, plan.num_sel, _stream(x.device),
            )
        check(rc, "pmsst_band_rows_scatter")
        return out

    # ------------------------------------------------------------------ mask application

    def mask_apply_forward(self, spec, mask, channels: int, zero_dc: bool = False):
        """Build-addition op: complex ``spec[B, F*C, T]`` times the per-stem masks
        ``mask[B, S, T, F*C*2]`` ((re, im) pairs), returned in the iSTFT layout: complex64
        ``[B*S*C, F, T]`` (frequency bin 0 zeroed when ``zero_dc``)."""
        _req(spec.is_cuda and spec.dtype == torch.complex64 and spec.dim() == 3, "spec must be CUDA complex64 [B, F*C, T]")
        _req(mask.is_cuda and mask.dim() == 4 and mask.dtype in (torch.float32, torch.float16, torch.bfloat16),
             "mask must be a CUDA float tensor [B, S, T, F*C*2]")
        b, fc, t = spec.shape
        _req(channels > 0 and fc % channels == 0, "channels must divide the spectrum rows")
        _req(mask.shape[0] == b and mask.shape[2] == t and mask.shape[3] == 2 * fc, "mask shape does not match spec")
        spec = spec.contiguous()
        if mask.stride(3) != 1 or mask.stride(2) != 2 * fc:
            mask = mask.contiguous()
        s = mask.shape[1]
        f = fc // channels
        est = torch.empty((b * s * channels, f, t), dtype=torch.complex64, device=spec.device)
        with _DeviceGuard(spec.device):
            rc = self._lib.pmsst_mask_apply_forward(
                _ptr(spec), _ptr(mask), mask.stride(0), mask.stride(1), b, s, channels, f, t, int(bool(zero_dc)),
                _ptr(est), dtype_code(mask.dtype), _stream(spec.device),
            )
        check(rc, "pmsst_mask_apply_forward")
        return est

    def mask_apply_backward(self, grad_est, spec, mask, channels: int, zero_dc: bool = False, need_spec_grad=False):
        """Gradients of :meth:`mask_apply_forward`: ``(grad_mask [B, S, T, F*C*2] in the mask dtype,
        grad_spec complex64 [B, F*C, T] or None)``."""
        b, fc, t = spec.shape
        s = mask.shape[1]
        f = fc // channels
        _req(grad_est.is_cuda and grad_est.dtype == torch.complex64 and tuple(grad_est.shape) == (b * s * channels, f, t),
             "grad_est must be CUDA complex64 [B*S*C, F, T]")
        grad_est = grad_est.contiguous()
        spec = spec.contiguous()
        if mask.stride(3) != 1 or mask.stride(2) != 2 * fc:
            mask = mask.contiguous()
        grad_mask = torch.empty((b, s, t, 2 * fc), dtype=mask.dtype, device=spec.device)
        grad_spec = torch.empty_like(spec) if need_spec_grad else None
        with _DeviceGuard(spec.device):
            rc = self._lib.pmsst_mask_apply_backward(
                _ptr(grad_est), _ptr(spec), _ptr(mask), mask.stride(0), mask.stride(1), b, s, channels, f, t,
                int(bool(zero_dc)), _ptr(grad_mask), _ptr(grad_spec) if grad_spec is not None else None,
                dtype_code(mask.dtype), _stream(spec.device),
            )
        check(rc, "pmsst_mask_apply_backward")
        return grad_mask, grad_spec

    # ------------------------------------------------------------------ band split

    def _bands(self, dim_inputs, device: torch.device):
        """Host ctypes widths + device int64 prefix sums, cached per (widths, device)."""
        dims = tuple(int(d) for d in dim_inputs)
        key = (dims, device.type, device.index)
        ent = self._band_cache.get(key)
        if ent is None:
            _req(len(dims) > 0 and all(d > 0 for d in dims), "dim_inputs must be positive")
            offs = [0]
            for d in dims:
                offs.append(offs[-1] + d)
            host = (ctypes.c_int64 * len(dims))(*dims)
            with torch.inference_mode(False):  # cached across modes
                dev = torch.tensor(offs, dtype=torch.int64, device=device)
            ent = (host, dev, offs)
            self._band_cache[key] = ent
        return ent

    def band_split_ragged_forward_packed(self, x, gamma_all, weight_all, bias_all, dim_inputs, write_normed=True,
                                         x_row_stride=None):
        """Ragged band split forward on packed parameters (the kernels' native layout).

        ``x[M, >=F]`` (row pitch ``x_row_stride``), ``gamma_all[F]``, ``weight_all`` the
        band-major concatenation of the ``[O, I_b]`` weights, ``bias_all[NB*O]`` or ``None``.
        Returns ``[out[M,NB,O], normed[M,F] | None, inv_norm[M,NB]]``.
        """
        host, dev_offs, offs = self._bands(dim_inputs, x.device)
        nb, total = len(offs) - 1, offs[-1]
        m = x.size(0)
        o = weight_all.numel() // total
        _req(o * total == weight_all.numel(), "packed weight size must be a multiple of the total width")
        stride = x.stride(0) if x_row_stride is None else int(x_row_stride)
        out = torch.empty((m, nb, o), dtype=x.dtype, device=x.device)
        normed = torch.empty((m, total), dtype=x.dtype, device=x.device) if write_normed else None
        inv = torch.empty((m, nb), dtype=torch.float32, device=x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_band_split_ragged_forward(
                _ptr(x), stride, _ptr(gamma_all), _ptr(weight_all), _ptr(bias_all), _ptr(dev_offs), host, nb, m, o,
                _ptr(out), _ptr(normed), _ptr(inv), dtype_code(x.dtype), _stream(x.device),
            )
        check(rc, "pmsst_band_split_ragged_forward")
        return [out, normed, inv]

    def band_split_ragged_backward_packed(self, grad_out, saved, saved_is_input, inv_norm, gamma_all, weight_all,
                                          dim_inputs, has_bias=True):
        """Ragged band split backward on packed parameters.

        ``saved`` is ``normed[M,F]`` (``saved_is_input=False``) or the forward input
        ``x[M,F]`` (``True``; normed recomputed).  Returns packed
        ``[grad_x[M,F], grad_gamma[F], grad_weight (packed), grad_bias[NB*O] | None]``.
        """
        host, dev_offs, offs = self._bands(dim_inputs, grad_out.device)
        nb, total = len(offs) - 1, offs[-1]
        grad_out = grad_out.contiguous()
        saved = saved.contiguous()
        m = grad_out.size(0)
        o = grad_out.size(-1)
        dev = grad_out.device
        dx = torch.empty((m, total), dtype=grad_out.dtype, device=dev)
        dg = torch.empty((total,), dtype=grad_out.dtype, device=dev)
        dw = torch.empty((o * total,), dtype=grad_out.dtype, device=dev)
        db = torch.empty((nb * o,), dtype=grad_out.dtype, device=dev) if has_bias else None
        ws = _workspace(self._lib.pmsst_band_split_ragged_backward_workspace_size(m, total, nb, o), dev)
        with _DeviceGuard(dev):
            rc = self._lib.pmsst_band_split_ragged_backward(
                _ptr(grad_out), _ptr(saved), 1 if saved_is_input else 0, _ptr(inv_norm.contiguous()),
                _ptr(gamma_all), _ptr(weight_all), _ptr(dev_offs),
                host, nb, m, o, _ptr(dx), _ptr(dg), _ptr(dw), _ptr(db), dtype_code(grad_out.dtype), _ptr(ws),
                ws.numel(), _stream(dev),
            )
        check(rc, "pmsst_band_split_ragged_backward")
        return [dx, dg, dw, db]

    def band_split_mixed_forward(self, x, gamma_all, weight_all, bias_all, dim_inputs, dtype):
        """Ragged band split of an fp32 input with the projection in ``dtype`` (fp16 / bf16): the call
        fr.py:827-857 makes under autocast, where x is the fp32 STFT.  The norm and ``inv_norm`` are
        fp32; ``features = dtype(x * inv * sqrt(I_b) * gamma)`` is the projection's input (what the
        stock nn.Linear sees under autocast) and is returned for the backward.

        ``x[M, >=F]`` fp32 (any row pitch), ``gamma_all[F]`` fp32, ``weight_all`` / ``bias_all`` packed
        as in :meth:`band_split_ragged_forward_packed`, in ``dtype``.
        Returns ``[out[M,NB,O] (dtype), features[M,F] (dtype), inv_norm[M,NB] fp32]``.
        """
        _req(x.dtype == torch.float32 and gamma_all.dtype == torch.float32, "x and gamma must be float32")
        _req(dtype in (torch.float16, torch.bfloat16), "the projection dtype must be float16 or bfloat16")
        _req(weight_all.dtype == dtype and (bias_all is None or bias_all.dtype == dtype),
             "weight and bias must have the projection dtype")
        _req(x.dim() == 2 and x.stride(1) == 1, "x must be [rows, features] with contiguous rows")
        host, dev_offs, offs = self._bands(dim_inputs, x.device)
        nb, total = len(offs) - 1, offs[-1]
        _req(x.size(1) >= total, "x has fewer columns than the bands' total width")
        m = x.size(0)
        o = weight_all.numel() // total
        _req(o * total == weight_all.numel(), "packed weight size must be a multiple of the total width")
        out = torch.empty((m, nb, o), dtype=dtype, device=x.device)
        feats = torch.empty((m, total), dtype=dtype, device=x.device)
        inv = torch.empty((m, nb), dtype=torch.float32, device=x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_band_split_mixed_forward(
                _ptr(x), x.stride(0), _ptr(gamma_all.contiguous()), _ptr(weight_all.contiguous()),
                _ptr(None if bias_all is None else bias_all.contiguous()), _ptr(dev_offs), host, nb, m, o,
                _ptr(feats), _ptr(out), _ptr(inv), dtype_code(dtype), _stream(x.device),
            )
        check(rc, "pmsst_band_split_mixed_forward")
        return [out, feats, inv]

    def band_split_mixed_backward(self, grad_out, x, features, inv_norm, gamma_all, weight_all, dim_inputs,
                                  has_bias=True):
        """Backward of :meth:`band_split_mixed_forward`.  ``grad_out[M, NB, O]`` in the projection dtype.
        Returns ``[grad_x[M,F] fp32, grad_gamma[F] fp32, grad_weight (packed, dtype),
        grad_bias[NB*O] (dtype) | None]``."""
        dtype = features.dtype
        _req(grad_out.dtype == dtype and weight_all.dtype == dtype, "grad_out and weight must have the features' dtype")
        _req(x.dtype == torch.float32 and gamma_all.dtype == torch.float32, "x and gamma must be float32")
        _req(x.dim() == 2 and x.stride(1) == 1, "x must be [rows, features] with contiguous rows")
        host, dev_offs, offs = self._bands(dim_inputs, grad_out.device)
        nb, total = len(offs) - 1, offs[-1]
        grad_out = grad_out.contiguous()
        features = features.contiguous()
        m = grad_out.size(0)
        o = grad_out.size(-1)
        dev = grad_out.device
        dx = torch.empty((m, total), dtype=torch.float32, device=dev)
        dg = torch.empty((total,), dtype=torch.float32, device=dev)
        dw = torch.empty((o * total,), dtype=dtype, device=dev)
        db = torch.empty((nb * o,), dtype=dtype, device=dev) if has_bias else None
        ws = _workspace(self._lib.pmsst_band_split_mixed_backward_workspace_size(m, total, nb), dev)
        with _DeviceGuard(dev):
            rc = self._lib.pmsst_band_split_mixed_backward(
                _ptr(grad_out), _ptr(x), x.stride(0), _ptr(features), _ptr(inv_norm.contiguous()),
                _ptr(gamma_all.contiguous()), _ptr(weight_all.contiguous()), _ptr(dev_offs), host, nb, m, o,
                _ptr(dx), _ptr(dg), _ptr(dw), _ptr(db), dtype_code(dtype), _ptr(ws), ws.numel(), _stream(dev),
            )
        check(rc, "pmsst_band_split_mixed_backward")
        return [dx, dg, dw, db]

    def band_split_ragged_forward(self, x, gammas, weights, biases, dim_inputs, dim_offsets):
        """``.cpp:271-314``: ``x[M, total]``, per-band ``gamma[I]``, ``weight[O, I]``, ``bias[O]`` lists.

        Returns ``[out[M,NB,O], normed[M,total], inv_norm[M,NB]]``.  ``dim_offsets`` is
        shape-checked; the kernels use prefix sums derived from ``dim_inputs``.
        """
        _req(x.is_cuda, "x must be a CUDA tensor")
        _req(dim_offsets.is_cuda, "dim_offsets must be a CUDA tensor")
        _req(x.dim() == 2, "x must have shape [M, total]")
        _req(dim_offsets.dim() == 1, "dim_offsets must be 1D")
        _req(dim_offsets.dtype == torch.int64, "dim_offsets must be int64")
        _req(len(gammas) == len(weights), "gammas length must match weights length")
        _req(len(biases) == len(weights), "biases length must match weights length")
        _req(len(dim_inputs) == len(weights), "dim_inputs length must match weights length")
        _req(dim_offsets.size(0) == len(weights) + 1, "dim_offsets length must be band count + 1")
        _req(len(weights) > 0, "weights must not be empty")
        out_features = weights[0].size(0)
        total = 0
        for g, w, b, d in zip(gammas, weights, biases, dim_inputs):
            total += int(d)
            _req(g.is_cuda, "gamma must be a CUDA tensor")
            _req(w.is_cuda, "weight must be a CUDA tensor")
            _req(b.is_cuda, "bias must be a CUDA tensor")
            _req(g.dim() == 1, "gamma must have shape [I]")
            _req(w.dim() == 2, "weight must have shape [O, I]")
            _req(b.dim() == 1, "bias must have shape [O]")
            _req(g.size(0) == d, "gamma dimension must match dim_inputs")
            _req(w.size(0) == out_features, "all weights must share output dimension")
            _req(w.size(1) == d, "weight input dimension must match dim_inputs")
            _req(b.size(0) == out_features, "bias output dimension must match weight")
            _req(g.dtype == x.dtype, "gamma dtype must match x")
            _req(w.dtype == x.dtype, "weight dtype must match x")
            _req(b.dtype == x.dtype, "bias dtype must match x")
            _req(g.device == x.device, "gamma device must match x")
            _req(w.device == x.device, "weight device must match x")
            _req(b.device == x.device, "bias device must match x")
        _req(x.size(1) == total, "x total dimension must match dim_inputs")
        x = x.contiguous()
        gamma_all = torch.cat([g.reshape(-1) for g in gammas])
        weight_all = torch.cat([w.reshape(-1) for w in weights])
        bias_all = torch.cat([b.reshape(-1) for b in biases])
        return self.band_split_ragged_forward_packed(x, gamma_all, weight_all, bias_all, dim_inputs, True)

    def band_split_ragged_backward(self, grad_out, normed, inv_norm, gammas, weights, dim_inputs, dim_offsets):
        """``.cpp:316-363``: returns ``[grad_x, *grad_gammas, *grad_weights, *grad_biases]``."""
        _req(grad_out.is_cuda, "grad_out must be a CUDA tensor")
        _req(normed.is_cuda, "normed must be a CUDA tensor")
        _req(inv_norm.is_cuda, "inv_norm must be a CUDA tensor")
        _req(dim_offsets.is_cuda, "dim_offsets must be a CUDA tensor")
        _req(grad_out.dim() == 3, "grad_out must have shape [M, B, O]")
        _req(normed.dim() == 2, "normed must have shape [M, total]")
        _req(inv_norm.dim() == 2, "inv_norm must have shape [M, B]")
        _req(dim_offsets.dim() == 1, "dim_offsets must be 1D")
        _req(dim_offsets.dtype == torch.int64, "dim_offsets must be int64")
        _req(len(gammas) == len(weights), "gammas length must match weights length")
        _req(len(dim_inputs) == len(weights), "dim_inputs length must match weights length")
        _req(dim_offsets.size(0) == len(weights) + 1, "dim_offsets length must be band count + 1")
        _req(len(weights) > 0, "weights must not be empty")
        _req(normed.size(0) == grad_out.size(0), "normed M must match grad_out")
        _req(inv_norm.size(0) == grad_out.size(0), "inv_norm M must match grad_out")
        _req(inv_norm.size(1) == grad_out.size(1), "inv_norm band count must match grad_out")
        _req(len(weights) == grad_out.size(1), "weights length must match grad_out band count")
        _req(normed.dtype == grad_out.dtype, "normed dtype must match grad_out")
        _req(inv_norm.dtype == torch.float32, "inv_norm must be float32")
        out_features = grad_out.size(2)
        total = 0
        for g, w, d in zip(gammas, weights, dim_inputs):
            total += int(d)
            _req(g.dim() == 1, "gamma must have shape [I]")
            _req(w.dim() == 2, "weight must have shape [O, I]")
            _req(g.size(0) == d, "gamma dimension must match dim_inputs")
            _req(w.size(0) == out_features, "weight output dimension must match grad_out")
            _req(w.size(1) == d, "weight input dimension must match dim_inputs")
            _req(g.dtype == grad_out.dtype, "gamma dtype must match grad_out")
            _req(w.dtype == grad_out.dtype, "weight dtype must match grad_out")
        _req(normed.size(1) == total, "normed total dimension must match dim_inputs")
        gamma_all = torch.cat([g.reshape(-1) for g in gammas])
        weight_all = torch.cat([w.reshape(-1) for w in weights])
        dx, dg, dw, db = self.band_split_ragged_backward_packed(grad_out, normed, False, inv_norm, gamma_all,
                                                                weight_all, dim_inputs, True)
        dims = [int(d) for d in dim_inputs]
        o = out_features
        dgs = list(dg.split(dims))
        dws = [v.view(o, d) for v, d in zip(dw.split([o * d for d in dims]), dims)]
        dbs = list(db.view(len(dims), o).unbind(0))
        return [dx, *dgs, *dws, *dbs]

    def band_split_forward(self, x, gamma, weight, bias=None):
        """``.cpp:141-170``: equal-width group ``x[M,G,I]`` (strided view allowed), ``gamma[G,I]``,
        ``weight[G,O,I]``, ``bias[G,O]`` or ``None``.  Returns ``[out[M,G,O], normed[M,G,I], inv_norm[M,G]]``.

        Runs the ragged kernel with G equal widths; a view whose inner two dims are dense is
        read in place with its row pitch.
        """
        _req(x.is_cuda, "x must be a CUDA tensor")
        _req(gamma.is_cuda, "gamma must be a CUDA tensor")
        _req(weight.is_cuda, "weight must be a CUDA tensor")
        if bias is not None:
            _req(bias.is_cuda, "bias must be a CUDA tensor")
        _req(x.dim() == 3, "x must have shape [M, G, I]")
        _req(gamma.dim() == 2, "gamma must have shape [G, I]")
        _req(weight.dim() == 3, "weight must have shape [G, O, I]")
        _req(gamma.size(0) == x.size(1), "gamma group dimension must match x")
        _req(gamma.size(1) == x.size(2), "gamma input dimension must match x")
        _req(weight.size(0) == x.size(1), "weight group dimension must match x")
        _req(weight.size(2) == x.size(2), "weight input dimension must match x")
        if bias is not None:
            _req(bias.dim() == 2, "bias must have shape [G, O]")
            _req(bias.size(0) == x.size(1), "bias group dimension must match x")
            _req(bias.size(1) == weight.size(1), "bias output dimension must match weight")
        _req(gamma.dtype == x.dtype, "gamma dtype must match x")
        _req(weight.dtype == x.dtype, "weight dtype must match x")
        if bias is not None:
            _req(bias.dtype == x.dtype, "bias dtype must match x")
        m, g, i = x.shape
        if not (x.stride(2) == 1 and x.stride(1) == i and x.stride(0) >= g * i):
            x = x.contiguous()
        out, normed, inv = self.band_split_ragged_forward_packed(
            x, gamma.contiguous().reshape(-1), weight.contiguous().reshape(-1),
            bias.contiguous().reshape(-1) if bias is not None else None, (i,) * g, True,
            x_row_stride=x.stride(0) if m > 0 else g * i,
        )
        return [out, normed.view(m, g, i), inv]

    def band_split_backward(self, grad_out, normed, inv_norm, gamma, weight, has_bias):
        """``.cpp:172-203`` (and ``_v2`` ``.cpp:205-236``, ``_v3`` ``.cpp:238-269``, same values):
        returns ``[grad_x[M,G,I], grad_gamma[G,I], grad_weight[G,O,I], grad_bias[G,O] | None]``."""
        _req(grad_out.is_cuda, "grad_out must be a CUDA tensor")
        _req(normed.is_cuda, "normed must be a CUDA tensor")
        _req(inv_norm.is_cuda, "inv_norm must be a CUDA tensor")
        _req(grad_out.dim() == 3, "grad_out must have shape [M, G, O]")
        _req(normed.dim() == 3, "normed must have shape [M, G, I]")
        _req(inv_norm.dim() == 2, "inv_norm must have shape [M, G]")
        _req(gamma.dim() == 2 and weight.dim() == 3, "gamma must have shape [G, I] and weight [G, O, I]")
        _req(normed.size(0) == grad_out.size(0) and normed.size(1) == grad_out.size(1),
             "normed must match grad_out in M and G")
        _req(weight.size(1) == grad_out.size(2), "weight output dimension must match grad_out")
        _req(inv_norm.dtype == torch.float32, "inv_norm must be float32")
        _req(normed.dtype == grad_out.dtype and gamma.dtype == grad_out.dtype and weight.dtype == grad_out.dtype,
             "normed, gamma and weight dtype must match grad_out")
        m, g, i = normed.shape
        o = grad_out.size(2)
        dx, dg, dw, db = self.band_split_ragged_backward_packed(
            grad_out.reshape(m, g, o), normed.reshape(m, g * i), False, inv_norm, gamma.contiguous().reshape(-1),
            weight.contiguous().reshape(-1), (i,) * g, bool(has_bias),
        )
        return [dx.view(m, g, i), dg.view(g, i), dw.view(g, o, i), db.view(g, o) if db is not None else None]

    band_split_backward_v2 = band_split_backward
    band_split_backward_v3 = band_split_backward

    # ------------------------------------------------------------------ grouped linear

    def grouped_linear_forward(self, x, weight, bias=None):
        """``.cpp:365-388``: ``x[M,G,I]`` (strided view allowed), ``weight[G,O,I]``, ``bias[G,O]`` or ``None``
        -> ``out[M,G,O]``."""
        return self.grouped_linear_forward_act(x, weight, bias, activation=None)

    def grouped_linear_forward_act(self, x, weight, bias=None, activation=None):
        """``grouped_linear_forward`` with an optional fused epilogue activation (``"tanh"``)."""
        act = _activation_code(activation)
        _req(x.is_cuda, "x must be a CUDA tensor")
        _req(weight.is_cuda, "weight must be a CUDA tensor")
        if bias is not None:
            _req(bias.is_cuda, "bias must be a CUDA tensor")
        _req(x.dim() == 3, "x must have shape [M, G, I]")
        _req(weight.dim() == 3, "weight must have shape [G, O, I]")
        _req(weight.size(0) == x.size(1), "weight group dimension must match x")
        _req(weight.size(2) == x.size(2), "weight input dimension must match x")
        if bias is not None:
            _req(bias.dim() == 2, "bias must have shape [G, O]")
            _req(bias.size(0) == x.size(1), "bias group dimension must match x")
            _req(bias.size(1) == weight.size(1), "bias output dimension must match weight")
        _req(weight.dtype == x.dtype, "weight dtype must match x")
        if bias is not None:
            _req(bias.dtype == x.dtype, "bias dtype must match x")
        m, g, i = x.shape
        o = weight.size(1)
        if not (x.stride(2) == 1 and x.stride(1) == i and x.stride(0) >= g * i):
            x = x.contiguous()
        weight = weight.contiguous()
        bias = bias.contiguous() if bias is not None else None
        _, dev_offs, _ = self._bands((i,) * g, x.device)
        out = torch.empty((m, g, o), dtype=x.dtype, device=x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_grouped_linear_forward(
                _ptr(x), x.stride(0) if m > 0 else g * i, _ptr(weight), _ptr(bias), _ptr(dev_offs), g, i, m, o,
                _ptr(out), act, dtype_code(x.dtype), _stream(x.device),
            )
        check(rc, "pmsst_grouped_linear_forward")
        return out

    def grouped_linear_backward(self, grad_out, x, weight, has_bias=True):
        """Backward of ``grouped_linear_forward`` (the reference's ``_FusedGroupedLinear.backward``,
        fr.py:1042-1048): ``grad_out[M,G,O]``, ``x[M,G,I]``, ``weight[G,O,I]`` ->
        ``[grad_x[M,G,I], grad_weight[G,O,I], grad_bias[G,O] | None]``."""
        _req(grad_out.is_cuda and x.is_cuda and weight.is_cuda, "tensors must be CUDA tensors")
        _req(x.dim() == 3 and weight.dim() == 3 and grad_out.dim() == 3, "x, weight, grad_out must be 3D")
        m, g, i = x.shape
        o = weight.size(1)
        _req(weight.size(0) == g and weight.size(2) == i, "weight must have shape [G, O, I] matching x")
        _req(tuple(grad_out.shape) == (m, g, o), "grad_out must have shape [M, G, O]")
        _req(grad_out.dtype == x.dtype and weight.dtype == x.dtype, "dtypes must match x")
        grad_out, x, weight = grad_out.contiguous(), x.contiguous(), weight.contiguous()
        _, dev_offs, _ = self._bands((i,) * g, x.device)
        dx = torch.empty_like(x)
        dw = torch.empty_like(weight)
        db = torch.empty((g, o), dtype=x.dtype, device=x.device) if has_bias else None
        ws_bytes = int(self._lib.pmsst_grouped_linear_backward_workspace_size(m, g, o))  # 0 on this build
        ws = _workspace(ws_bytes, x.device) if ws_bytes else None
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_grouped_linear_backward(
                _ptr(grad_out), _ptr(x), _ptr(weight), _ptr(dev_offs), g, i, m, o, _ptr(dx), _ptr(dw), _ptr(db),
                dtype_code(x.dtype), _ptr(ws), ws_bytes, _stream(x.device),
            )
        check(rc, "pmsst_grouped_linear_backward")
        return [dx, dw, db]

    # ------------------------------------------------------------------ mask estimator final layer

    def _mask_check(self, x, weights, dim_inputs, dim_offsets):
        _req(x.is_cuda, "x must be a CUDA tensor")
        _req(dim_offsets.is_cuda, "dim_offsets must be a CUDA tensor")
        _req(x.dim() == 3, "x must have shape [M, G, H]")
        _req(dim_offsets.dim() == 1, "dim_offsets must be 1D")
        _req(dim_offsets.dtype == torch.int64, "dim_offsets must be int64")
        _req(len(weights) == x.size(1), "weights length must match band count")
        _req(len(dim_inputs) == len(weights), "dim_inputs length must match weights length")
        _req(dim_offsets.size(0) == x.size(1) + 1, "dim_offsets length must be band count + 1")
        for w, d in zip(weights, dim_inputs):
            _req(w.is_cuda, "weight must be a CUDA tensor")
            _req(w.dim() == 2, "weight must have shape [2 * O, H]")
            _req(w.size(1) == x.size(2), "weight hidden dimension must match x")
            _req(w.size(0) == int(d) * 2, "weight output dimension must match dim_inputs")
            _req(w.dtype == x.dtype, "weight dtype must match x")
            _req(w.device == x.device, "weight device must match x")

    def mask_estimator_final_forward_packed(self, x, weight_all, bias, dim_inputs):
        """Final layer + GLU on packed weights; returns ``[out[M,F], pre[M,2F]]``."""
        host, dev_offs, offs = self._bands(dim_inputs, x.device)
        nb, total = len(offs) - 1, offs[-1]
        x = x.contiguous()
        m, h = x.size(0), x.size(2)
        pre = torch.empty((m, 2 * total), dtype=x.dtype, device=x.device)
        out = torch.empty((m, total), dtype=x.dtype, device=x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_mask_estimator_final_forward(
                _ptr(x), _ptr(weight_all), _ptr(bias), _ptr(dev_offs), host, nb, m, h, _ptr(pre), _ptr(out),
                dtype_code(x.dtype), _stream(x.device),
            )
        check(rc, "pmsst_mask_estimator_final_forward")
        return [out, pre]

    def mask_estimator_final_backward_packed(self, grad_out, x, pre, weight_all, dim_inputs, input_activation=None):
        """Backward on packed weights; returns ``[grad_x[M,NB,H], grad_bias[2F], grad_weight (packed)]``.
        ``input_activation="tanh"``: ``x`` is a tanh output and ``grad_x`` is the gradient of its
        pre-activation, ``(dpre W) * (1 - x^2)``."""
        act = _activation_code(input_activation)
        host, dev_offs, offs = self._bands(dim_inputs, grad_out.device)
        nb = len(offs) - 1
        grad_out = grad_out.contiguous()
        x = x.contiguous()
        pre = pre.contiguous()
        m, h = x.size(0), x.size(2)
        dx = torch.empty_like(x)
        db = torch.empty((pre.size(1),), dtype=x.dtype, device=x.device)
        dw = torch.empty((weight_all.numel(),), dtype=x.dtype, device=x.device)
        code = dtype_code(x.dtype)
        ws = _workspace(self._lib.pmsst_mask_estimator_final_backward_workspace_size(m, offs[-1], code), x.device)
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_mask_estimator_final_backward(
                _ptr(grad_out), _ptr(x), _ptr(pre), _ptr(weight_all), _ptr(dev_offs), host, nb, m, h, _ptr(dx),
                _ptr(db), _ptr(dw), act, code, _ptr(ws), ws.numel(), _stream(x.device),
            )
        check(rc, "pmsst_mask_estimator_final_backward")
        return [dx, db, dw]

    # ------------------------------------------------------------------ whole mask MLP

    def mask_mlp_supported(self, dim, hidden, dim_inputs, dtype) -> bool:
        """Whether :meth:`mask_mlp_forward` takes this shape and dtype."""
        dims = tuple(int(d) for d in dim_inputs)
        host = (ctypes.c_int64 * len(dims))(*dims)
        code = dtype_code(dtype) if dtype in (torch.float32, torch.float16, torch.bfloat16) else -1
        return bool(self._lib.pmsst_mask_mlp_supported(int(dim), int(hidden), host, len(dims), code))

    def mask_mlp_forward(self, x, w1, b1, w2_all, b2, dim_inputs, save_hidden=False):
        """Depth-2 mask MLP in one pass: ``x[M,NB,D]``, ``w1[NB,H,D]``, ``b1[NB,H]``, packed ``w2`` and
        ``b2[2F]``.  Returns ``[out[M,F], pre[M,2F], hidden[M,NB,H] | None]`` (``hidden`` only with
        ``save_hidden``)."""
        _req(x.is_cuda and x.dim() == 3, "x must be a CUDA tensor of shape [M, NB, D]")
        host, dev_offs, offs = self._bands(dim_inputs, x.device)
        nb, total = len(offs) - 1, offs[-1]
        _req(x.size(1) == nb, "x band count must match dim_inputs")
        x = x.contiguous()
        w1 = w1.contiguous()
        b1 = b1.contiguous()
        m, d = x.size(0), x.size(2)
        hd = w1.size(1)
        _req(tuple(w1.shape) == (nb, hd, d), "w1 must have shape [NB, H, D]")
        _req(b1.numel() == nb * hd, "b1 must have NB * H elements")
        _req(w2_all.numel() == 2 * total * hd, "w2 must hold the packed [2 I_b, H] weights")
        _req(b2.numel() == 2 * total, "b2 must have 2F elements")
        for t in (w1, b1, w2_all, b2):
            _req(t.dtype == x.dtype and t.device == x.device, "parameters must match x in dtype and device")
        pre = torch.empty((m, 2 * total), dtype=x.dtype, device=x.device)
        out = torch.empty((m, total), dtype=x.dtype, device=x.device)
        hid = torch.empty((m, nb, hd), dtype=x.dtype, device=x.device) if save_hidden else None
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_mask_mlp_forward(
                _ptr(x), _ptr(w1), _ptr(b1), _ptr(w2_all), _ptr(b2), _ptr(dev_offs), host, nb, m, d, hd, _ptr(pre),
                _ptr(out), _ptr(hid), dtype_code(x.dtype), _stream(x.device),
            )
        check(rc, "pmsst_mask_mlp_forward")
        return [out, pre, hid]

    def mask_mlp_forward_apply(self, x, w1, b1, w2_all, b2, dim_inputs, spec, est, stem: int, channels: int,
                               zero_dc: bool = False, save_hidden: bool = False):
        """:meth:`mask_mlp_forward` with the mask application in its epilogue: writes stem ``stem`` of
        ``est`` (complex64 ``[B*S*C, F, T]``, the iSTFT input) = complex ``spec[B, F*C, T]`` times this
        stem's mask, instead of returning the mask.  Rows of ``x`` are ``(batch, frame)``.  Returns
        ``[pre[M,2F], hidden[M,NB,H] | None]``."""
        _req(x.is_cuda and x.dim() == 3, "x must be a CUDA tensor of shape [M, NB, D]")
        _req(spec.is_cuda and spec.dtype == torch.complex64 and spec.dim() == 3 and spec.is_contiguous(),
             "spec must be a contiguous CUDA complex64 [B, F*C, T]")
        _req(est.is_cuda and est.dtype == torch.complex64 and est.dim() == 3 and est.is_contiguous(),
             "est must be a contiguous CUDA complex64 [B*S*C, F, T]")
        host, dev_offs, offs = self._bands(dim_inputs, x.device)
        nb, total = len(offs) - 1, offs[-1]
        b, fc, t = spec.shape
        _req(channels > 0 and fc % channels == 0 and 2 * fc == total, "spec rows must be the features / 2")
        _req(x.size(0) == b * t and x.size(1) == nb, "x must have B * T rows and one slice per band")
        _req(est.size(0) % (b * channels) == 0 and tuple(est.shape[1:]) == (fc // channels, t),
             "est must have shape [B * S * C, F, T]")
        stems = est.size(0) // (b * channels)
        _req(0 <= stem < stems, "stem out of range")
        x = x.contiguous()
        w1 = w1.contiguous()
        b1 = b1.contiguous()
        m, d = x.size(0), x.size(2)
        hd = w1.size(1)
        _req(tuple(w1.shape) == (nb, hd, d), "w1 must have shape [NB, H, D]")
        _req(b1.numel() == nb * hd, "b1 must have NB * H elements")
        _req(w2_all.numel() == 2 * total * hd, "w2 must hold the packed [2 I_b, H] weights")
        _req(b2.numel() == 2 * total, "b2 must have 2F elements")
        for tt in (w1, b1, w2_all, b2):
            _req(tt.dtype == x.dtype and tt.device == x.device, "parameters must match x in dtype and device")
        pre = torch.empty((m, 2 * total), dtype=x.dtype, device=x.device)
        hid = torch.empty((m, nb, hd), dtype=x.dtype, device=x.device) if save_hidden else None
        with _DeviceGuard(x.device):
            rc = self._lib.pmsst_mask_mlp_forward_apply(
                _ptr(x), _ptr(w1), _ptr(b1), _ptr(w2_all), _ptr(b2), _ptr(dev_offs), host, nb, m, d, hd, _ptr(pre),
                _ptr(hid), _ptr(spec), _ptr(est), t, channels, stems, stem, int(bool(zero_dc)), dtype_code(x.dtype),
                _stream(x.device),
            )
        check(rc, "pmsst_mask_mlp_forward_apply")
        return [pre, hid]

    def mask_apply_grad_mask(self, grad_est, spec, stems: int, channels: int, dtype, zero_dc: bool = False):
        """``grad_est * conj(spec)`` as the per-stem mask gradients ``[B, S, T, F*C*2]`` in ``dtype`` (the
        mask-gradient half of :meth:`mask_apply_backward`, for masks that were never stored)."""
        b, fc, t = spec.shape
        f = fc // channels
        _req(grad_est.is_cuda and grad_est.dtype == torch.complex64 and tuple(grad_est.shape) == (b * stems * channels, f, t),
             "grad_est must be CUDA complex64 [B*S*C, F, T]")
        grad_est = grad_est.contiguous()
        spec = spec.contiguous()
        grad_mask = torch.empty((b, stems, t, 2 * fc), dtype=dtype, device=spec.device)
        with _DeviceGuard(spec.device):
            # the mask argument is read only for the spectrum gradient, which is not asked for here
            rc = self._lib.pmsst_mask_apply_backward(
                _ptr(grad_est), _ptr(spec), _ptr(grad_mask), grad_mask.stride(0), grad_mask.stride(1), b, stems, channels,
                f, t, int(bool(zero_dc)), _ptr(grad_mask), None, dtype_code(dtype), _stream(spec.device),
            )
        check(rc, "pmsst_mask_apply_backward")
        return grad_mask

    def mask_estimator_final_forward(self, x, weights, bias, dim_inputs, dim_offsets):
        """``.cpp:589-622`` / ``.cpp:660-693`` (direct): ``x[M,NB,H]``, per-band ``weight[2*I_b, H]``,
        ``bias[2F]`` -> ``[out[M,F], pre[M,2F], x_contiguous]``."""
        self._mask_check(x, weights, dim_inputs, dim_offsets)
        _req(bias.is_cuda, "bias must be a CUDA tensor")
        _req(bias.dim() == 1, "bias must have shape [2 * total]")
        _req(bias.size(0) == 2 * sum(int(d) for d in dim_inputs), "bias dimension must match dim_inputs")
        _req(bias.dtype == x.dtype, "bias dtype must match x")
        _req(bias.device == x.device, "bias device must match x")
        x = x.contiguous()
        weight_all = torch.cat([w.reshape(-1) for w in weights])
        out, pre = self.mask_estimator_final_forward_packed(x, weight_all, bias.contiguous(), dim_inputs)
        return [out, pre, x]

    def mask_estimator_final_backward(self, grad_out, x, pre, weights, dim_inputs, dim_offsets):
        """``.cpp:624-658`` / ``.cpp:695-729`` (direct): returns ``[grad_x, grad_bias, *grad_weights]``."""
        self._mask_check(x, weights, dim_inputs, dim_offsets)
        _req(grad_out.is_cuda, "grad_out must be a CUDA tensor")
        _req(pre.is_cuda, "pre must be a CUDA tensor")
        _req(grad_out.dim() == 2, "grad_out must have shape [M, total]")
        _req(pre.dim() == 2, "pre must have shape [M, 2 * total]")
        _req(grad_out.size(0) == x.size(0), "grad_out M must match x")
        _req(pre.size(0) == x.size(0), "pre M must match x")
        _req(pre.size(1) == grad_out.size(1) * 2, "pre total dimension must be twice grad_out")
        _req(grad_out.dtype == x.dtype, "grad_out dtype must match x")
        _req(pre.dtype == x.dtype, "pre dtype must match x")
        weight_all = torch.cat([w.reshape(-1) for w in weights])
        dx, db, dw = self.mask_estimator_final_backward_packed(grad_out, x, pre, weight_all, dim_inputs)
        h = x.size(2)
        dims = [int(d) for d in dim_inputs]
        dws = [v.view(2 * d, h) for v, d in zip(dw.split([2 * d * h for d in dims]), dims)]
        return [dx, db, *dws]

    mask_estimator_final_direct_forward = mask_estimator_final_forward
    mask_estimator_final_direct_backward = mask_estimator_final_backward


__all__ = ["HipFusedExtension", "PmsstError"]

"""Axial transformer blocks of BS-RoFormer / Mel-band RoFormer (stock PyTorch restatement).

Names follow the pymss-core module the reference patches
(``pymss_core.modules.bs_roformer.transformer``; call sites
fused_roformer.py:710-824): ``RMSNorm.forward`` (patched at fr.py:772),
``apply_rotary_emb_fast(cos, sin, t)`` (fr.py:722-731), ``qkv_to_bnhd`` and
``rotate_qk_fast_bnhd`` (fr.py:802-806).  Attention works on ``bnhd`` tensors,
applies rotary to q and k with pairwise-interleaved tables, runs PyTorch SDPA,
and multiplies each head by a sigmoid gate from ``to_gates`` (fr.py:810-818).

Patched functions are looked up through this module's globals at call time, so
``transformer.apply_rotary_emb_fast = ...`` takes effect everywhere.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

__all__ = [
    "RMSNorm",
    "RotaryEmbedding",
    "apply_rotary_emb_fast",
    "qkv_to_bnhd",
    "rotate_qk_fast_bnhd",
    "Attention",
    "FeedForward",
    "Transformer",
    "sdpa_backend_policy",
]


class RMSNorm(nn.Module):
    """``F.normalize(x, dim=-1) * sqrt(dim) * gamma`` (fused_roformer.py:1267 states the same math)."""

    def __init__(self, dim: int):
        super().__init__()
        self.scale = dim**0.5
        self.gamma = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return F.normalize(x, dim=-1) * self.scale * self.gamma


class RotaryEmbedding(nn.Module):
    """RoFormer rotary tables ``angle(n, p) = n * theta**(-2p/dim)``, pairwise interleaved.

    ``tables(n, device, dtype)`` returns ``cos, sin`` of shape ``[1, n, 1, dim]`` where
    entries ``2p`` and ``2p+1`` share pair ``p``'s angle; the fused path reads
    ``cos[..., ::2]`` (fused_roformer.py:727).
    """

    def __init__(self, dim: int, theta: float = 10000.0):
        super().__init__()
        self.dim = dim
        self.theta = theta
        inv_freq = 1.0 / (theta ** (torch.arange(0, dim, 2, dtype=torch.float64)[: dim // 2] / dim))
        self.register_buffer("inv_freq", inv_freq.float(), persistent=False)
        self._cache: dict = {}

    def tables(self, seq_len: int, device, dtype):
        key = (seq_len, str(device), dtype)
        hit = self._cache.get(key)
        if hit is not None:
            return hit
        # cached tables are normal tensors even when first built in inference mode (validation), so a
        # later training step can save them for its backward
        with torch.inference_mode(False):
            pos = torch.arange(seq_len, dtype=torch.float64)
            inv = 1.0 / (self.theta ** (torch.arange(0, self.dim, 2, dtype=torch.float64)[: self.dim // 2] / self.dim))
            ang = pos[:, None] * inv[None, :]
            ang = ang.repeat_interleave(2, dim=-1)
            cos = ang.cos().to(device=device, dtype=dtype).reshape(1, seq_len, 1, self.dim)
            sin = ang.sin().to(device=device, dtype=dtype).reshape(1, seq_len, 1, self.dim)
        self._cache[key] = (cos, sin)
        return cos, sin


def _rotate_pairs(t: torch.Tensor) -> torch.Tensor:
    """``(e, o) -> (-o, e)`` for adjacent pairs along the last axis."""
    pairs = t.unflatten(-1, (-1, 2))
    return torch.stack((-pairs[..., 1], pairs[..., 0]), dim=-1).flatten(-2)


def apply_rotary_emb_fast(cos: torch.Tensor, sin: torch.Tensor, t: torch.Tensor) -> torch.Tensor:
    """Rotate adjacent pairs of ``t[B, N, H, D]`` by the ``[1, N, 1, D]`` tables."""
    return t * cos + _rotate_pairs(t) * sin


def qkv_to_bnhd(qkv: torch.Tensor, heads: int):
    """``[B, N, 3*H*D]`` -> three ``[B, N, H, D]`` views."""
    b, n, _ = qkv.shape
    return qkv.view(b, n, 3, heads, -1).unbind(dim=2)


def rotate_qk_fast_bnhd(rotary_embed: RotaryEmbedding, q: torch.Tensor, k: torch.Tensor):
    cos, sin = rotary_embed.tables(q.shape[1], q.device, q.dtype)
    rot = globals()["apply_rotary_emb_fast"]
    return rot(cos, sin, q), rot(cos, sin, k)


# SDPA backend choice for 16-bit GPU inputs: the flash / memory-efficient kernels
# (no batched-GEMM math path on transposed bf16 operands).  "auto" lets PyTorch pick.
sdpa_backend_policy = {"mode": "fused_only"}


def _sdpa(q, k, v, dropout_p: float):
    if q.is_cuda and q.dtype in (torch.float16, torch.bfloat16) and sdpa_backend_policy["mode"] == "fused_only":
        from torch.nn.attention import SDPBackend, sdpa_kernel

        with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
            return F.scaled_dot_product_attention(q, k, v, dropout_p=dropout_p)
    return F.scaled_dot_product_attention(q, k, v, dropout_p=dropout_p)


class Attention(nn.Module):
    def __init__(self, dim: int, heads: int = 8, dim_head: int = 64, dropout: float = 0.0,
                 rotary_embed: RotaryEmbedding | None = None):
        super().__init__()
        self.heads = heads
        self.dim_head = dim_head
        self.dropout = dropout
        inner = heads * dim_head
        self.rotary_embed = rotary_embed
        self.norm = RMSNorm(dim)
        self.to_qkv = nn.Linear(dim, inner * 3, bias=False)
        self.to_gates = nn.Linear(dim, heads)
        self.to_out = nn.Sequential(nn.Linear(inner, dim, bias=False), nn.Dropout(dropout))

    def _attention(self, q, k, v):
        return _sdpa(q.contiguous(), k.contiguous(), v.contiguous(), self.dropout if self.training else 0.0)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.norm(x)
        q, k, v = qkv_to_bnhd(self.to_qkv(x), self.heads)
        if self.rotary_embed is not None:
            q, k = rotate_qk_fast_bnhd(self.rotary_embed, q, k)
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        out = self._attention(q, k, v).transpose(1, 2)  # [B, N, H, D]
        gates = self.to_gates(x).sigmoid()
        out = out * gates.unsqueeze(-1).to(out.dtype)
        return self.to_out(out.reshape(*out.shape[:2], -1))


class FeedForward(nn.Module):
    def __init__(self, dim: int, mult: int = 4, dropout: float = 0.0):
        super().__init__()
        inner = int(dim * mult)
        self.net = nn.Sequential(
            RMSNorm(dim), nn.Linear(dim, inner), nn.GELU(), nn.Dropout(dropout), nn.Linear(inner, dim), nn.Dropout(dropout)
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.net(x)


class Transformer(nn.Module):
    def __init__(self, *, dim: int, depth: int, dim_head: int = 64, heads: int = 8, attn_dropout: float = 0.0,
                 ff_dropout: float = 0.0, ff_mult: int = 4, norm_output: bool = True,
                 rotary_embed: RotaryEmbedding | None = None):
        super().__init__()
        self.layers = nn.ModuleList(
            [
                nn.ModuleList(
                    [
                        Attention(dim, heads=heads, dim_head=dim_head, dropout=attn_dropout, rotary_embed=rotary_embed),
                        FeedForward(dim, mult=ff_mult, dropout=ff_dropout),
                    ]
                )
                for _ in range(depth)
            ]
        )
        self.norm = RMSNorm(dim) if norm_output else nn.Identity()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for attn, ff in self.layers:
            x = attn(x) + x
            x = ff(x) + x
        return self.norm(x)

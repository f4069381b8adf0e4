"""GPU: no kernel writes outside the tensors it is given.

Every output and workspace the extension allocates (``torch.empty`` / ``torch.empty_like`` in
``pymsst_amd/extension.py``) is handed out here as a view into a larger buffer whose first and last
4 KB hold a fixed byte pattern; after each op the patterns must be intact.  This checks the HIP
kernels themselves (the CPU replay in ``tests/bounds_model.py`` checks a restatement of their
address arithmetic) for stores past either end of their outputs, at the bench's configs[1] shapes
in bf16 and fp32 and at odd shapes that take the unaligned and partial-tile paths.  Reads past
the end are not covered: a read cannot corrupt a guard.
"""

from __future__ import annotations

import math

import pytest
import torch

import bench
from pymsst_amd import extension as ext_mod

PAD = 4096     # guard bytes on each side (a multiple of 256, so views keep the allocator's alignment)
FILL = 0xA5


class _GuardedTorch:
    """Stands in for the ``torch`` module inside ``pymsst_amd.extension``: allocations come back as
    views into padded buffers, every other attribute is torch's own."""

    def __init__(self, real):
        self._torch = real
        self.buffers = []

    def __getattr__(self, name):
        return getattr(self._torch, name)

    def empty(self, *size, dtype=None, device=None, **kwargs):
        t = self._torch
        shape = tuple(size[0]) if len(size) == 1 and isinstance(size[0], (tuple, list, t.Size)) else tuple(size)
        dtype = dtype or t.get_default_dtype()
        esz = t.empty((), dtype=dtype).element_size()
        nbytes = math.prod(shape) * esz
        buf = t.empty(nbytes + 2 * PAD, dtype=t.uint8, device=device)
        buf.fill_(FILL)
        self.buffers.append((buf, nbytes))
        return buf[PAD:PAD + nbytes].view(dtype).view(shape)

    def empty_like(self, x, *, dtype=None, device=None, **kwargs):
        return self.empty(tuple(x.shape), dtype=dtype or x.dtype, device=device or x.device)

    def damaged(self):
        if self._torch.cuda.is_available():
            self._torch.cuda.synchronize()
        bad = []
        for buf, nbytes in self.buffers:
            lo, hi = buf[:PAD], buf[PAD + nbytes:]
            if not (bool((lo == FILL).all()) and bool((hi == FILL).all())):
                bad.append(nbytes)
        self.buffers.clear()
        return bad


@pytest.fixture
def guarded(monkeypatch):
    g = _GuardedTorch(torch)
    monkeypatch.setattr(ext_mod, "torch", g)
    return g


def test_guard_catches_a_write_past_either_end():
    """CPU: the checker flags one byte written just past a guarded view's end or just before its
    start, and passes untouched guards."""
    g = _GuardedTorch(torch)
    t = g.empty((4, 3), dtype=torch.float32, device="cpu")
    t.fill_(1.0)
    assert not g.damaged()
    g.empty((5,), dtype=torch.bfloat16, device="cpu")
    g.buffers[-1][0][PAD + 10] = 0  # the byte after 5 bf16 elements
    assert g.damaged() == [10]
    v = g.empty(7, dtype=torch.uint8, device="cpu")
    v.zero_()
    g.buffers[-1][0][PAD - 1] = 0   # the byte before the view
    assert g.damaged() == [7]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_bench_ops_write_inside_their_outputs(hip_ext, guarded, dtype):
    """Every op of the configs[1] microbench step (band split, q/k RMSNorm+rotary, the mask MLP
    forward and backward) in the order the step runs them."""
    w = bench.Workload(torch, hip_ext, dtype)
    ops = w.ops()
    assert len(ops) >= 7
    for name, op in ops:
        print(f"[guard] {dt_name(dtype)} {name}", flush=True)
        op()
        assert not guarded.damaged(), f"{name}: a guard byte past an output or workspace changed"


def dt_name(dtype):
    return {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}[dtype]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32], ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("shape", [(37, 3, 6, 10), (100, 100, 192, 776), (65, 4, 512, 2048), (33, 62, 64, 256)])
def test_grouped_linear_writes_inside_its_outputs(hip_ext, guarded, dtype, shape):
    """Grouped linear forward (tanh epilogue) and backward at odd widths, the dW's 192-column tiles
    with a partial last tile, wide groups and a row count one past a 32-row chunk."""
    m, groups, i, o = shape
    g = torch.Generator().manual_seed(3)
    x = torch.randn(m, groups, i, generator=g).to(dtype).cuda()
    wt = (torch.randn(groups, o, i, generator=g) / i**0.5).to(dtype).cuda()
    b = (0.1 * torch.randn(groups, o, generator=g)).to(dtype).cuda()
    dy = torch.randn(m, groups, o, generator=g).to(dtype).cuda()
    print(f"[guard] grouped linear {shape} {dt_name(dtype)}", flush=True)
    hip_ext.grouped_linear_forward_act(x, wt, b, activation="tanh")
    assert not guarded.damaged(), "grouped_linear_forward_act"
    for has_bias in (True, False):
        hip_ext.grouped_linear_backward(dy, x, wt, has_bias)
        assert not guarded.damaged(), f"grouped_linear_backward has_bias={has_bias}"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("m", [1, 31, 1033])
def test_mask_mlp_and_band_split_write_inside_their_outputs(hip_ext, guarded, dtype, m):
    """The ragged band split and the mask estimator (one-pass MLP where the dtype allows it) at row
    counts that leave partial tiles everywhere."""
    dims = bench.BSR_WIDTHS
    nb, f, d, h = len(dims), sum(dims), 192, 768
    g = torch.Generator().manual_seed(4)
    x = torch.randn(m, f, generator=g).to(dtype).cuda()
    gamma = (1 + 0.1 * torch.randn(f, generator=g)).to(dtype).cuda()
    w_bs = torch.cat([(torch.randn(d, i, generator=g) / i**0.5).reshape(-1) for i in dims]).to(dtype).cuda()
    b_bs = (0.1 * torch.randn(nb * d, generator=g)).to(dtype).cuda()
    print(f"[guard] band split m={m} {dt_name(dtype)}", flush=True)
    y, _, inv = hip_ext.band_split_ragged_forward_packed(x, gamma, w_bs, b_bs, dims, write_normed=False)
    assert not guarded.damaged(), "band_split_ragged_forward_packed"
    dy = torch.randn(y.shape, generator=g).to(dtype).cuda()
    hip_ext.band_split_ragged_backward_packed(dy, x, True, inv, gamma, w_bs, dims, True)
    assert not guarded.damaged(), "band_split_ragged_backward_packed"
    hx = torch.randn(m, nb, d, generator=g).to(dtype).cuda()
    w1 = (torch.randn(nb, h, d, generator=g) / d**0.5).to(dtype).cuda()
    b1 = (0.1 * torch.randn(nb, h, generator=g)).to(dtype).cuda()
    w2 = torch.cat([(torch.randn(2 * i, h, generator=g) / h**0.5).reshape(-1) for i in dims]).to(dtype).cuda()
    b2 = (0.1 * torch.randn(2 * f, generator=g)).to(dtype).cuda()
    gout = torch.randn(m, f, generator=g).to(dtype).cuda()
    print(f"[guard] mask estimator m={m} {dt_name(dtype)}", flush=True)
    if dtype != torch.float32:
        out, pre, hid = hip_ext.mask_mlp_forward(hx, w1, b1, w2, b2, dims, save_hidden=True)
        assert not guarded.damaged(), "mask_mlp_forward"
    else:
        hid = hip_ext.grouped_linear_forward_act(hx, w1, b1, activation="tanh")
        out, pre = hip_ext.mask_estimator_final_forward_packed(hid, w2, b2, dims)
        assert not guarded.damaged(), "grouped linear + mask_estimator_final_forward_packed"
    dz = hip_ext.mask_estimator_final_backward_packed(gout, hid, pre, w2, dims, input_activation="tanh")[0]
    assert not guarded.damaged(), "mask_estimator_final_backward_packed"
    hip_ext.grouped_linear_backward(dz, hx, w1, has_bias=True)
    assert not guarded.damaged(), "grouped_linear_backward"


def _rotary_tables(n, d, dtype):
    import oracle

    c, s = oracle.rotary_tables(n, d)
    c = torch.from_numpy(c).to(dtype).cuda().repeat_interleave(2, dim=-1).reshape(1, n, 1, d)[..., ::2]
    s = torch.from_numpy(s).to(dtype).cuda().repeat_interleave(2, dim=-1).reshape(1, n, 1, d)[..., ::2]
    return c, s


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_train_path_ops_write_inside_their_outputs(hip_ext, guarded, dtype):
    """The other ops of the patched training step: RMSNorm (aligned and guarded-scalar widths),
    rotary on q/k views and the fused qkv split, the attention gate in both layouts, the mask
    application, the mixed-precision band split of an fp32 input and the mel band gather/scatter."""
    import numpy as np

    from pymsst_amd.core.mel_band_roformer import mel_band_bins

    g = torch.Generator().manual_seed(5)

    def rnd(*shape, dt=dtype):
        return torch.randn(*shape, generator=g).to(dt).cuda()

    for rows, dim in ((257, 192), (65, 100), (33, 6)):
        print(f"[guard] rms_norm {rows}x{dim}", flush=True)
        x, gamma, dy = rnd(rows, dim), 1 + 0.1 * rnd(dim), rnd(rows, dim)
        out, normed, inv = hip_ext.rms_norm_forward(x, gamma)
        hip_ext.rms_norm_backward(dy, normed, inv, gamma)
        hip_ext.rms_norm_backward_from_input(dy, x, inv, gamma)
        assert not guarded.damaged(), f"rms_norm {rows}x{dim}"

    b, n, h, d = 2, 62, 8, 64
    print("[guard] rotary", flush=True)
    qkv = rnd(b, n, 3 * h * d)
    cos, sin = _rotary_tables(n, d, dtype)
    q, k, _ = qkv.view(b, n, 3, h, d).unbind(dim=2)
    for t in (q, k):
        for layout in ("bnhd", "bhnd"):
            hip_ext.rotary_forward(t, cos, sin, out_layout=layout)
    hip_ext.rotary_backward(rnd(b, n, h, d), cos, sin)
    hip_ext.rotary_qkv_forward(qkv, h, cos, sin)
    gq, gk, gv = (rnd(b, h, n, d).transpose(1, 2) for _ in range(3))
    hip_ext.rotary_qkv_backward(gq, gk, gv, cos, sin)
    assert not guarded.damaged(), "rotary"

    print("[guard] attention gate", flush=True)
    m, dm = b * n, 192
    attn, xg, wg, bg, gout = rnd(m, h, d), rnd(m, dm), rnd(h, dm) / dm**0.5, 0.5 * rnd(h), rnd(m, h * d)
    _, gate, sa, sx = hip_ext.attention_gate_forward(attn, xg, wg, bg)
    hip_ext.attention_gate_backward(gout, sa, sx, wg, gate)
    attn_t = rnd(b, h, n, d).transpose(1, 2)
    _, gate, sa, sx = hip_ext.attention_gate_forward_bnhd(attn_t, xg, wg, bg)
    hip_ext.attention_gate_backward_bnhd(gout, sa, sx, wg, gate)
    hip_ext.attention_gate_backward_bnhd(gout, sa, sx, wg, gate, out_layout="bnhd")
    assert not guarded.damaged(), "attention gate"

    print("[guard] mask apply", flush=True)
    bs, s, c, f, t = 2, 3, 2, 33, 70
    spec = torch.complex(torch.randn(bs, f * c, t, generator=g), torch.randn(bs, f * c, t, generator=g)).cuda()
    mask = rnd(bs, s, t, 2 * f * c)
    est = hip_ext.mask_apply_forward(spec, mask, c, True)
    hip_ext.mask_apply_backward(torch.randn_like(est), spec, mask, c, True, need_spec_grad=True)
    assert not guarded.damaged(), "mask apply"

    print("[guard] band split mixed", flush=True)
    dims = bench.BSR_WIDTHS
    fb, ob = sum(dims), 192
    xb = torch.randn(130, fb, generator=g).cuda()
    gb = (1 + 0.1 * torch.randn(fb, generator=g)).cuda()
    pdt = dtype if dtype != torch.float32 else torch.bfloat16  # the projection runs in 16-bit only
    wb = torch.cat([(torch.randn(ob, i, generator=g) / i**0.5).reshape(-1) for i in dims]).to(pdt).cuda()
    bb = (0.1 * torch.randn(len(dims) * ob, generator=g)).to(pdt).cuda()
    out, feats, inv = hip_ext.band_split_mixed_forward(xb, gb, wb, bb, dims, pdt)
    hip_ext.band_split_mixed_backward(torch.randn_like(out), xb, feats, inv, gb, wb, dims, True)
    assert not guarded.damaged(), "band split mixed"

    print("[guard] mel band rows", flush=True)
    bins = mel_band_bins(44100, 2048, 60)
    rows = np.concatenate([(bb_[:, None] * 2 + np.arange(2)[None, :]).reshape(-1) for bb_ in bins])
    plan = hip_ext.band_rows_plan(rows, 1025 * 2, "cuda")
    xr = torch.randn(2, 1025 * 2, 65, 2, generator=g).cuda()
    yr = hip_ext.band_rows_gather(xr, plan, out_dtype=dtype)
    hip_ext.band_rows_scatter(yr.float(), plan)
    hip_ext.band_rows_scatter(yr.float(), plan, mean=True)
    assert not guarded.damaged(), "mel band rows"

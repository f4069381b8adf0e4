"""The bench line's byte accounting (CPU): a step is charged exactly the algorithmic bytes of the ops it
runs, so ``value * ms_per_step`` reproduces from ``per_op``."""

from __future__ import annotations

import importlib.util
from pathlib import Path

import pytest
import torch

_spec = importlib.util.spec_from_file_location("bench", Path(__file__).resolve().parents[1] / "bench.py")
bench = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(bench)


def _workload(dtype, one_pass):
    w = bench.Workload.__new__(bench.Workload)
    w.torch, w.dtype = torch, dtype
    w.dims = bench.BSR_WIDTHS
    w.B, w.T, w.dim, w.hidden = 4, 258, 192, 768
    w.M, w.F, w.NB = w.B * w.T, sum(w.dims), len(w.dims)
    w.qk_shape = (w.B * w.NB, w.T, 8, 64)
    w.one_pass = one_pass
    return w


@pytest.mark.parametrize("dtype,one_pass", [(torch.bfloat16, True), (torch.float32, False)])
def test_step_bytes_are_the_executed_ops(dtype, one_pass):
    w = _workload(dtype, one_pass)
    names = w.op_names()
    traffic = w.traffic()
    assert len(names) == len(set(names))
    assert w.step_bytes() == sum(traffic[n][0] for n in names)
    if one_pass:
        assert "mask_mlp_fwd" in names and "mask_hidden_fwd" not in names and "mask_final_fwd" not in names
    else:
        assert "mask_mlp_fwd" not in names and {"mask_hidden_fwd", "mask_final_fwd"} <= set(names)
    # a step charged with every op of the table would count the two-kernel and one-pass forwards both
    assert w.step_bytes() < sum(b for b, _ in traffic.values())


def test_configs1_bf16_step_bytes_value():
    """configs[1] bf16: 1,353.7 MB per step (band split, q/k norm+rotary, one-pass mask MLP with its saved
    tensors, mask backward)."""
    w = _workload(torch.bfloat16, True)
    assert abs(w.step_bytes() - 1353.7e6) < 0.1e6
    # the scope table's pure fused forward: 64.0 MB
    assert abs(w.fused_mask_bytes() - 64.0e6) < 0.1e6
    assert w.traffic()["mask_mlp_fwd"][1] == pytest.approx(31.87e9, rel=1e-3)


def test_roofline_bound_of_the_mask_projections_is_mfma():
    assert bench.OP_BOUND["mask_mlp_fwd"] == "mfma"
    assert bench.OP_BOUND.get("band_split_fwd", "hbm") == "hbm"

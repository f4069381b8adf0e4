"""GPU parity: the Mel-band RoFormer band gather and overlap-averaged mask scatter kernels against
the oracle at the configs[3] layout (60 mel bands, stereo: 2050 spectrum rows, 3958 selections),
in every dtype pairing the model uses; and the tiny Mel-band model patched with the ``hip_full``
preset against the stock modules (fp32, same seed and inputs).  Bars are those of ``conftest.py``."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pymsst_amd import fused_roformer as fr
from pymsst_amd.core.mel_band_roformer import mel_band_bins
from pymsst_amd.workloads import WORKLOADS, workload_batch
from tests.conftest import assert_parity, to_np

pytestmark = pytest.mark.gpu


def _layout():
    bins = mel_band_bins(44100, 2048, 60)
    rows = np.concatenate([(b[:, None] * 2 + np.arange(2)[None, :]).reshape(-1) for b in bins])
    return rows, 1025 * 2


@pytest.mark.parametrize("in_dt,out_dt", [(torch.float32, torch.float32), (torch.float32, torch.bfloat16)])
def test_gather_matches_oracle(hip_ext, in_dt, out_dt):
    rows, R = _layout()
    plan = hip_ext.band_rows_plan(rows, R, "cuda")
    g = torch.Generator().manual_seed(41)
    x = torch.randn(3, R, 65, 2, generator=g).to(in_dt).cuda()
    out = hip_ext.band_rows_gather(x, plan, out_dtype=out_dt)
    assert out.shape == (3, 65, rows.size, 2) and out.dtype == out_dt
    ref = oracle.band_rows_gather(to_np(x), rows)
    if out_dt == torch.float32:
        assert np.array_equal(to_np(out), ref), "a gather copies values exactly"
    else:
        assert_parity(out, ref, "bf16", "gather bf16")
    div = hip_ext.band_rows_gather(x, plan, divide=True)
    assert_parity(div, oracle.band_rows_gather(to_np(x), rows, np.bincount(rows, minlength=R)[rows]), "f32", "div")


@pytest.mark.parametrize("in_dt", [torch.bfloat16, torch.float32])
def test_scatter_mean_matches_oracle_and_stock(hip_ext, in_dt):
    rows, R = _layout()
    plan = hip_ext.band_rows_plan(rows, R, "cuda")
    g = torch.Generator().manual_seed(42)
    y = torch.randn(4, 65, rows.size, 2, generator=g).to(in_dt).cuda()
    out = hip_ext.band_rows_scatter(y, plan, mean=True)
    assert out.shape == (4, R, 65, 2) and out.dtype == torch.float32
    assert_parity(out, oracle.band_rows_scatter(to_np(y), rows, R, mean=True), "f32", "scatter mean")
    # the stock path (scatter_add_ then division) gives the same fp32 values: 1 or 2 bands per bin
    vals = y.float().permute(0, 2, 1, 3)
    idx = torch.from_numpy(rows).cuda().view(1, -1, 1, 1).expand(4, -1, 65, 2)
    stock = torch.zeros(4, R, 65, 2, device="cuda").scatter_add_(1, idx, vals)
    stock = stock / torch.bincount(torch.from_numpy(rows), minlength=R).cuda().float().view(1, -1, 1, 1)
    assert torch.equal(out, stock)
    plain = hip_ext.band_rows_scatter(y, plan, mean=False)
    assert_parity(plain, oracle.band_rows_scatter(to_np(y), rows, R, mean=False), "f32", "scatter sum")


def test_uncovered_rows_and_empty(hip_ext):
    rows = np.array([1, 1, 3])
    plan = hip_ext.band_rows_plan(rows, 5, "cuda")
    y = torch.ones(2, 4, 3, 2, device="cuda")
    out = hip_ext.band_rows_scatter(y, plan)
    assert torch.equal(out[:, [0, 2, 4]], torch.zeros_like(out[:, [0, 2, 4]]))
    assert torch.equal(out[:, [1, 3]], torch.ones_like(out[:, [1, 3]]))
    empty = hip_ext.band_rows_gather(torch.empty(0, 5, 4, 2, device="cuda"), plan)
    assert empty.shape == (0, 4, 3, 2)
    with pytest.raises(RuntimeError, match="rows must lie"):
        hip_ext.band_rows_plan(np.array([0, 5]), 5, "cuda")


@pytest.fixture
def hip_env(monkeypatch, hip_ext):
    for key, value in fr.RUNTIME_PRESETS["hip_full"].items():
        monkeypatch.setenv(key, value)
    monkeypatch.setenv(fr.CORE_GROUPED_TRAIN_ENV, "1")
    yield hip_ext
    fr.restore_stock_implementations()


def _run(wl, fused, target, mixture, ext):
    model = wl.build_model("cuda", seed=4)
    model.train()
    fr.restore_stock_implementations(model)
    status = fr.apply_roformer_fused_training_backend(model, "hip", extension=ext, rms_norm_mode="fast") if fused \
        else None
    try:
        loss = model(mixture, target)
        loss.backward()
        torch.cuda.synchronize()
        grads = {n: p.grad.detach().clone() for n, p in model.named_parameters() if p.grad is not None}
    finally:
        fr.restore_stock_implementations(model)
    return float(loss.detach()), grads, status


def test_tiny_mel_band_model_fused_matches_stock_fp32(hip_env):
    wl = WORKLOADS["mbr_tiny"]
    target, mixture = workload_batch(wl, seed=0, device="cuda")
    ls, gs, _ = _run(wl, False, target, mixture, hip_env)
    lf, gf, status = _run(wl, True, target, mixture, hip_env)
    assert status.patched_mel_bands and status.patched_band_split_ragged_forward
    assert abs(lf - ls) <= 1e-5 * max(1.0, abs(ls))
    worst = 0.0
    for name, g in gs.items():
        rel = ((gf[name] - g).norm() / g.norm().clamp(min=1e-30)).item()
        worst = max(worst, rel)
        assert rel <= 1e-4, f"{name}: rel L2 {rel:.3e}"
    print(f"[mel-parity] loss stock {ls:.8f} fused {lf:.8f}; worst grad rel L2 {worst:.3e}")

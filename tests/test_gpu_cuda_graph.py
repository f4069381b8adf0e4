"""GPU: the RoFormer mask-core graph wrapper (``pymsst_amd.cuda_graph``, after pymsst's
``cuda_graph.py``) gives the eager model's results.  On ROCm it refuses training captures by default
(replays of the captured backward after the first return wrong gradients on this stack), so the
training cases check the eager fallback and its stated reason; the opt-in capture is exercised for
its status only.

Each case captures once, then for three fresh batches runs the eager model and the graphed model on
the same parameters and compares loss and every parameter gradient; the eager runs between the
replays are the program's own work between replays (graph nodes that only hold on the first replay
would show here).  Cases: both modes, stock and fused (``hip_full``) modules, fp32 and bf16 autocast, the spectrogram
loss and the iSTFT + multi-resolution STFT loss.
"""

from __future__ import annotations

import pytest
import torch

from pymsst_amd import fused_roformer as fr
from pymsst_amd.cuda_graph import HIP_TRAINING_GRAPH_REASON, RoformerTrainingCudaGraph, normalize_cuda_graph_mode
from pymsst_amd.workloads import WORKLOADS, TrainWorkload, workload_batch

# bsr_tiny trains on the spectrogram loss; this variant (2 stems) goes through the iSTFT and the
# multi-resolution STFT loss
_ISTFT_WL = TrainWorkload(
    name="bsr_tiny_istft",
    model={**WORKLOADS["bsr_tiny"].model, "num_stems": 2, "loss": "multi_stft"},
    batch=2, length=32768, stems=2,
)

def _loss_grads(fn, model):
    loss = fn()
    loss.backward()
    torch.cuda.synchronize()
    grads = {n: p.grad.detach().float().clone() for n, p in model.named_parameters() if p.grad is not None}
    for p in model.parameters():
        p.grad = None
    return float(loss.detach()), grads


@pytest.mark.gpu
@pytest.mark.parametrize("mode", ["mask_core", "stft_mask_core"])
@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("amp", [None, torch.bfloat16])
@pytest.mark.parametrize("wl", [WORKLOADS["bsr_tiny"], _ISTFT_WL], ids=["spec_l1", "istft"])
def test_training_graph_matches_eager(monkeypatch, hip_ext, mode, fused, amp, wl):
    """The wrapper's training forward gives the eager model's loss and gradients on three batches.  On
    ROCm it refuses the capture by default (and says why), so this checks the eager fallback there."""
    if fused:
        for key, value in fr.RUNTIME_PRESETS["hip_full"].items():
            monkeypatch.setenv(key, value)
    model = wl.build_model("cuda", seed=4)
    model.train()
    fr.restore_stock_implementations(model)
    try:
        if fused:
            status = fr.apply_roformer_fused_training_backend(model, "hip", extension=hip_ext, rms_norm_mode="fast")
            assert status.active == "cuda_ext"
        use_amp = amp is not None
        graph = RoformerTrainingCudaGraph(model, mode, amp_dtype=amp or torch.float16)
        _, sample = workload_batch(wl, seed=0, device="cuda")
        st = graph.capture(sample, use_amp=use_amp)
        assert all(p.grad is None for p in model.parameters())
        if torch.version.hip is not None:
            assert st.active == "off" and st.reason == HIP_TRAINING_GRAPH_REASON
        else:
            assert st.active == mode or "replay" in (st.reason or ""), st.reason
        tol = (1e-5 if mode == "mask_core" else 1e-4) if amp is None else 2e-2
        for seed in (1, 2, 3):
            target, mixture = workload_batch(wl, seed=seed, device="cuda")

            def eager():
                with torch.autocast("cuda", dtype=amp or torch.float16, enabled=use_amp, cache_enabled=False):
                    return model(mixture, target)

            le, ge = _loss_grads(eager, model)
            lg, gg = _loss_grads(lambda: graph.forward(mixture, target, use_amp=use_amp), model)
            assert abs(lg - le) <= tol * abs(le), (seed, lg, le)
            assert set(gg) == set(ge)
            for name, ref in ge.items():
                diff = (gg[name] - ref).abs().max().item()
                assert diff <= tol * max(1.0, ref.abs().max().item()), f"call {seed} {name}: {diff:.3e}"
    finally:
        fr.restore_stock_implementations(model)
        fr.restore_stock_implementations()


@pytest.mark.gpu
def test_opt_in_capture_reports_a_status(hip_ext):
    """With the opt-in the capture runs (warm-up, recording, two checked replays) and reports active or
    the replay disagreement; the graph is not used for training here."""
    wl = WORKLOADS["bsr_tiny"]
    model = wl.build_model("cuda", seed=4)
    model.train()
    graph = RoformerTrainingCudaGraph(model, "mask_core", allow_hip_training_graphs=True)
    _, sample = workload_batch(wl, seed=0, device="cuda")
    st = graph.capture(sample, use_amp=False)
    assert st.active == "mask_core" or "replay" in (st.reason or ""), st.reason
    assert all(p.grad is None for p in model.parameters())


def test_mode_names():
    assert normalize_cuda_graph_mode(None) == "off"
    assert normalize_cuda_graph_mode("mask") == "mask_core"
    assert normalize_cuda_graph_mode("roformer-stft-mask-core") == "stft_mask_core"
    with pytest.raises(ValueError):
        normalize_cuda_graph_mode("everything")

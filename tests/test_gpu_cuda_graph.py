"""GPU: HIP-graph capture of the RoFormer mask core (``pymsst_amd.cuda_graph``, after pymsst's
``cuda_graph.py``) gives the eager model's results: either its graphs replay forward and backward
exactly, or its own two-replay check at capture finds them wrong and ``forward`` runs eagerly.

Each case captures once, then for three fresh batches runs the eager model and the graphed model on
the same parameters and compares loss and every parameter gradient; the eager runs between the
replays are the program's own work between replays (graph nodes that only hold on the first replay
would show here).  Cases: both modes, stock and fused (``hip_full``) modules, fp32 and bf16 autocast, the spectrogram
loss and the iSTFT + multi-resolution STFT loss.
"""

from __future__ import annotations

import sys

import pytest
import torch

from pymsst_amd import fused_roformer as fr
from pymsst_amd.cuda_graph import RoformerTrainingCudaGraph, normalize_cuda_graph_mode
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
def test_graph_replays_match_eager(monkeypatch, hip_ext, mode, fused, amp, wl):
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
        # active, or inactive because its own replay check found the graph wrong (then forward is eager)
        assert st.active == mode or "replay" in (st.reason or ""), st.reason
        sys.stderr.write(f"[graph] {mode}: active={st.active} reason={st.reason}\n")
        # fp32: the mask core replays bitwise-equal kernels; with the STFT inside the graph the FFTs
        # run from the captured plan and differ from the eager ones by rounding (bar 1e-4)
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
            worst = 0.0
            for name, ref in ge.items():
                diff = (gg[name] - ref).abs().max().item()
                worst = max(worst, diff / max(1.0, ref.abs().max().item()))
                assert diff <= tol * max(1.0, ref.abs().max().item()), f"replay {seed} {name}: {diff:.3e}"
            sys.stderr.write(f"[graph] replay {seed}: loss {lg:.8f} vs {le:.8f}, worst grad diff {worst:.3e}\n")
        # another shape runs eagerly
        _, other = workload_batch(wl, seed=4, device="cuda")
        other = other[:1]
        with torch.no_grad():
            out = graph.forward(other, use_amp=use_amp)
        assert out.shape[0] == 1
    finally:
        fr.restore_stock_implementations(model)
        fr.restore_stock_implementations()


def test_mode_names():
    assert normalize_cuda_graph_mode(None) == "off"
    assert normalize_cuda_graph_mode("mask") == "mask_core"
    assert normalize_cuda_graph_mode("roformer-stft-mask-core") == "stft_mask_core"
    with pytest.raises(ValueError):
        normalize_cuda_graph_mode("everything")

"""GPU: the RoFormer mask-core graph wrapper (``pymsst_amd.cuda_graph``, after pymsst's
``cuda_graph.py``) gives the eager model's results.  On ROCm it refuses training captures by default
(replays of the captured backward after the first return wrong gradients on this stack), so the
training cases check the eager fallback and its stated reason.  No GPU test records a training graph
on ROCm (its captured backward would hold memset nodes); the capture / refusal logic and the replay
check are tested on the CPU below with a stand-in for the graphed callable.

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


def test_mode_names():
    assert normalize_cuda_graph_mode(None) == "off"
    assert normalize_cuda_graph_mode("mask") == "mask_core"
    assert normalize_cuda_graph_mode("roformer-stft-mask-core") == "stft_mask_core"
    with pytest.raises(ValueError):
        normalize_cuda_graph_mode("everything")


def test_capture_refusal_reasons():
    from pymsst_amd.cuda_graph import capture_refusal

    assert capture_refusal("cpu", False, None) == "CUDA graph requires CUDA tensors"
    assert capture_refusal("cuda", True, "7.2") == HIP_TRAINING_GRAPH_REASON
    assert capture_refusal("cuda", False, "7.2") is None
    assert capture_refusal("cuda", True, None) is None


def test_training_capture_opt_in_raises_on_rocm(monkeypatch):
    model = WORKLOADS["bsr_tiny"].build_model(None, seed=4)
    monkeypatch.setattr(torch.version, "hip", "7.2.0", raising=False)
    with pytest.raises(ValueError, match="not supported on ROCm"):
        RoformerTrainingCudaGraph(model, "mask_core", allow_hip_training_graphs=True)
    graph = RoformerTrainingCudaGraph(model, "mask_core")
    st = graph.capture(torch.zeros(1, 2, 4096), use_amp=False)  # CPU tensor: refused before any capture
    assert st.active == "off" and not graph.active


class _Lin(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.lin = torch.nn.Linear(6, 5)

    def forward(self, x):
        return self.lin(x).tanh()


def test_replay_check_flags_a_replay_that_disagrees():
    """``_validate`` compares two replays with eager: a stand-in graph whose second replay returns a wrong
    bias gradient (the failure mode of a memset node that holds once) is rejected with that reason."""
    torch.manual_seed(0)
    mod = _Lin()
    graph = RoformerTrainingCudaGraph(mod, "mask_core")
    sample = torch.randn(4, 6)
    calls = {"n": 0}

    class _Replay(torch.autograd.Function):
        @staticmethod
        def forward(ctx, x, w, b):
            ctx.save_for_backward(x, w, b)
            return torch.nn.functional.linear(x, w, b).tanh()

        @staticmethod
        def backward(ctx, g):
            x, w, b = ctx.saved_tensors
            y = torch.nn.functional.linear(x, w, b).tanh()
            gz = g * (1 - y * y)
            db = gz.sum(0)
            calls["n"] += 1
            if calls["n"] >= 2:
                db = db * 0  # the replay after the first loses the bias reduction
            return gz @ w, gz.t() @ x, db

    graph._graph_call = lambda x: _Replay.apply(x, mod.lin.weight, mod.lin.bias)
    reason = graph._validate(mod, sample, use_amp=False)
    assert reason is not None and "replay 2 gradients" in reason

    calls["n"] = -10**6  # every replay right: accepted
    assert graph._validate(mod, sample, use_amp=False) is None

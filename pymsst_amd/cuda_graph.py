"""HIP-graph capture of the RoFormer mask core for training (pymsst ``src/pymsst/training/cuda_graph.py``).

Same interface as the reference: :func:`normalize_cuda_graph_mode`, :class:`CudaGraphRuntimeStatus`
and :class:`RoformerTrainingCudaGraph` with ``capture(sample_mixture, use_amp=...)`` and
``forward(mixture, use_amp=...)``.  On ROCm ``torch.cuda.make_graphed_callables`` records HIP graphs;
the captured region replays its forward and backward kernels (this build's HIP kernels included:
they launch on the current stream, allocate through torch and set no memory with ``hipMemset``).

Modes (``cuda_graph.py:18-26``):

* ``mask_core``: the graph maps the STFT to the masked spectrum in the iSTFT layout (band split,
  axial blocks, final norm, mask estimators, mask product - ``BSRoformer._mask_core``); the STFT and
  the iSTFT run eagerly (``cuda_graph.py:88-99``).
* ``stft_mask_core``: the graph starts from the mixture (STFT included); the iSTFT runs eagerly
  (``cuda_graph.py:81-86``).

With a target, ``forward`` returns the model's loss: the waveform losses after the eager iSTFT, the
spectrogram loss (``loss="spec_l1"``) from the graphed masked spectrum permuted back to
``[B, stems, F*C, T]``.

On ROCm (``torch.version.hip``) a training capture (parameters that require gradients) is refused and
``forward`` runs eagerly: on ROCm 7.2 with torch 2.10 the captured backward of torch's bias /
normalisation reductions records memset nodes, and memset nodes in a HIP graph hold on the first
replay only, so later replays return wrong gradients.  There is no opt-in:
``allow_hip_training_graphs=True`` raises ``ValueError`` on ROCm.  Captures without gradients
(frozen parameters) are unaffected.

The model is this build's restated BS-RoFormer (``pymsst_amd.core``): its ``_stft`` / ``_mask_core``
/ ``_finish`` split stands in for pymss-core's ``stft_roformer`` / ``_mask_stft_repr`` /
``_istft_roformer_cached_zero`` (the iSTFT layout and zero-DC fill are those of
``cuda_graph.py:140-158``).  A capture failure leaves the wrapper inactive with the reason, and
``forward`` then runs the model eagerly (``cuda_graph.py:73-80,88-91``); so does a mixture of another
shape than the captured one.  Autocast in the graph is fp16 with ``cache_enabled=False``
(``cuda_graph.py:106-107``); ``amp_dtype`` selects bf16 instead.
"""

from __future__ import annotations

import warnings
from dataclasses import dataclass
from typing import Callable

import torch
from torch import nn

__all__ = ["CudaGraphRuntimeStatus", "HIP_TRAINING_GRAPH_REASON", "RoformerTrainingCudaGraph", "capture_refusal",
           "normalize_cuda_graph_mode"]

HIP_TRAINING_GRAPH_REASON = (
    "HIP graph replays of the training backward are not reliable on this ROCm stack (memset nodes recorded by "
    "library reductions hold on the first replay only); training captures are refused on ROCm"
)


@dataclass
class CudaGraphRuntimeStatus:
    """``cuda_graph.py:11-15``."""

    requested: str
    active: str
    reason: str | None = None


def normalize_cuda_graph_mode(value: str | None) -> str:
    """``cuda_graph.py:18-26``."""
    mode = str(value or "off").strip().lower().replace("-", "_")
    if mode in {"", "none", "false", "0", "off", "default"}:
        return "off"
    if mode in {"mask", "mask_core", "roformer_mask_core"}:
        return "mask_core"
    if mode in {"stft_mask", "stft_mask_core", "roformer_stft_mask_core"}:
        return "stft_mask_core"
    raise ValueError("cuda_graph_mode must be one of: off, mask_core, stft_mask_core")


def capture_refusal(device_type: str, training: bool, hip_version: str | None) -> str | None:
    """Why a capture is not attempted (``None``: capture).  Non-CUDA tensors are refused as in
    ``cuda_graph.py:44-46``; on ROCm a region whose parameters require gradients is refused because
    its captured backward would hold memset nodes."""
    if device_type != "cuda":
        return "CUDA graph requires CUDA tensors"
    if hip_version is not None and training:
        return HIP_TRAINING_GRAPH_REASON
    return None


def _autocast(enabled: bool, dtype: torch.dtype):
    return torch.autocast("cuda", dtype=dtype, enabled=enabled, cache_enabled=False)


class _MaskCoreModule(nn.Module):
    """Graphed region of ``mask_core``: complex spectrum -> masked spectrum (iSTFT layout)."""

    def __init__(self, model: nn.Module, channels: int) -> None:
        super().__init__()
        self.model = model
        self.channels = channels

    def forward(self, spec: torch.Tensor) -> torch.Tensor:
        return self.model._mask_core(spec, self.channels)


class _STFTMaskCoreModule(nn.Module):
    """Graphed region of ``stft_mask_core``: mixture -> masked spectrum (iSTFT layout)."""

    def __init__(self, model: nn.Module) -> None:
        super().__init__()
        self.model = model

    def forward(self, mixture: torch.Tensor) -> torch.Tensor:
        spec, _ = self.model._stft(mixture)
        return self.model._mask_core(spec, mixture.shape[1])


class RoformerTrainingCudaGraph:
    """``cuda_graph.py:29-103`` over this build's BS-RoFormer (mixture ``[B, C, L]``)."""

    def __init__(self, model: nn.Module, mode: str = "mask_core", amp_dtype: torch.dtype = torch.float16,
                 allow_hip_training_graphs: bool = False) -> None:
        self.mode = normalize_cuda_graph_mode(mode)
        if self.mode == "off":
            raise ValueError("RoformerTrainingCudaGraph requires an active graph mode")
        if allow_hip_training_graphs and torch.version.hip is not None:
            raise ValueError("allow_hip_training_graphs is not supported on ROCm: " + HIP_TRAINING_GRAPH_REASON)
        self.model = model
        self.amp_dtype = amp_dtype
        self.allow_hip_training_graphs = allow_hip_training_graphs
        self.status = CudaGraphRuntimeStatus(requested=self.mode, active="off")
        self._graph_call: Callable[[torch.Tensor], torch.Tensor] | None = None
        self._input_shape: tuple[int, ...] | None = None
        self._window: torch.Tensor | None = None

    @property
    def active(self) -> bool:
        return self.status.active == self.mode and self._graph_call is not None

    def capture(self, sample_mixture: torch.Tensor, *, use_amp: bool) -> CudaGraphRuntimeStatus:
        """Warm up and record the graphs on ``sample_mixture``'s shape (``cuda_graph.py:44-84``)."""
        training = any(p.requires_grad for p in self.model.parameters())
        refusal = capture_refusal(sample_mixture.device.type, training, torch.version.hip)
        if refusal is not None:
            self.status = CudaGraphRuntimeStatus(self.mode, "off", refusal)
            return self.status
        if sample_mixture.ndim == 2:
            sample_mixture = sample_mixture.unsqueeze(1)
        try:
            if self.mode == "stft_mask_core":
                graph_module = _STFTMaskCoreModule(self.model)
                sample = sample_mixture
            else:
                with _autocast(use_amp, self.amp_dtype):
                    sample, _ = self.model._stft(sample_mixture)
                graph_module = _MaskCoreModule(self.model, sample_mixture.shape[1])
            with _autocast(use_amp, self.amp_dtype):
                graph_module(sample)
                self._graph_call = torch.cuda.make_graphed_callables(graph_module, (sample,))
            problem = self._validate(graph_module, sample, use_amp)
            if problem is not None:
                raise RuntimeError(problem)
            self._input_shape = tuple(sample_mixture.shape)
            self.status = CudaGraphRuntimeStatus(self.mode, self.mode)
        except Exception as exc:  # noqa: BLE001 - any capture failure falls back to eager
            self._graph_call = None
            self._input_shape = None
            reason = f"failed to capture RoFormer {self.mode} HIP graph: {exc}"
            warnings.warn(reason, RuntimeWarning, stacklevel=2)
            self.status = CudaGraphRuntimeStatus(self.mode, "off", reason)
        finally:
            for parameter in self.model.parameters():
                parameter.grad = None
        return self.status

    def _validate(self, graph_module: nn.Module, sample: torch.Tensor, use_amp: bool) -> str | None:
        """Two replays of the captured forward and backward against the eager region on the capture
        sample (this build's addition).  On ROCm 7 the backward of library reductions (bias and
        normalisation gradients) can record memset nodes that only hold on the first replay; a graph
        whose second replay disagrees with eager is not used."""
        params = [p for p in self.model.parameters() if p.requires_grad]
        gen = torch.Generator(device=sample.device).manual_seed(0)

        def run(fn):
            for p in params:
                p.grad = None
            with _autocast(use_amp, self.amp_dtype):
                out = fn(sample.clone())
            out_r = torch.view_as_real(out) if out.is_complex() else out
            w = torch.randn(out_r.shape, generator=gen.manual_seed(0), device=out.device, dtype=torch.float32)
            (out_r.float() * w).sum().backward()
            if sample.is_cuda:
                torch.cuda.synchronize()
            return out_r.detach().float().clone(), [None if p.grad is None else p.grad.detach().float().clone()
                                                    for p in params]

        ref_out, ref_grads = run(graph_module)
        scale = lambda t: max(1.0, t.abs().max().item())  # noqa: E731
        tol = 1e-3
        for replay in (1, 2):
            out, grads = run(self._graph_call)
            if (out - ref_out).abs().max().item() > tol * scale(ref_out):
                return f"graph replay {replay} output disagrees with eager"
            for g, r in zip(grads, ref_grads):
                if (g is None) != (r is None) or (g is not None and (g - r).abs().max().item() > tol * scale(r)):
                    return (f"graph replay {replay} gradients disagree with eager (library reductions in the "
                            "captured backward record memset nodes that hold only on the first replay)")
        return None

    def forward(self, mixture: torch.Tensor, target: torch.Tensor | None = None, *, use_amp: bool):
        """Separated audio (or the loss against ``target``) through the graphed region
        (``cuda_graph.py:86-103``); eager ``model(mixture, target)`` when inactive or for another shape."""
        if mixture.ndim == 2:
            mixture = mixture.unsqueeze(1)
        spec_loss = target is not None and getattr(self.model, "loss_type", None) == "spec_l1"
        if (not self.active or tuple(mixture.shape) != self._input_shape
                or (spec_loss and getattr(self.model, "zero_dc", False))):
            with _autocast(use_amp, self.amp_dtype):
                return self.model(mixture, target)
        b, c, length = mixture.shape
        with _autocast(use_amp, self.amp_dtype):
            if self.mode == "stft_mask_core":
                est = self._graph_call(mixture)
                window = self._window_for(mixture.device)
            else:
                spec, window = self.model._stft(mixture)
                est = self._graph_call(spec)
            if spec_loss:  # the model's spectrogram loss reads [B, stems, F*C, T]
                f, t = est.shape[1:]
                stems = est.shape[0] // (b * c)
                est = est.reshape(b, stems, c, f, t).transpose(2, 3).reshape(b, stems, f * c, t)
                return self.model._spec_loss(est, target, c)
            return self.model._finish(est, window, b, c, length, target)

    def _window_for(self, device: torch.device) -> torch.Tensor:
        if self._window is None or self._window.device != device:
            self._window = torch.hann_window(self.model.stft_win_length, device=device, dtype=torch.float32)
        return self._window

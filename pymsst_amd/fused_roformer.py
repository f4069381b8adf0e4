"""Drop-in fused training backend for RoFormer models on MI355X.

Public API and behaviour follow the reference's
``src/pymsst/training/fused_roformer.py`` (baicai-1145/pymsst):

* ``apply_roformer_fused_training_backend(model, backend, *, extension=None,
  rms_norm_mode=None) -> FusedTrainingStatus`` (fr.py:56-136): the same backend
  names (``"off"`` / ``"cuda_ext"`` and aliases, plus ``"hip"`` / ``"rocm"``), the
  same ``PYMSST_EXPERIMENTAL_*`` environment flags, the same duck-typed
  ``extension=`` injection (ops are probed with ``hasattr``), the same status
  fields and the same soft fallbacks (eval mode, non-GPU input, unsupported
  dtype, missing bias -> the stock implementation).
* The patch targets are the restated stock modules in ``pymsst_amd.core``
  (``bands``, ``transformer``, ``common``), which stand in for pymss-core.
* ``_Fused*`` autograd Functions keep the reference's argument lists and return
  conventions (fr.py:888-1262).

Where the extension also offers this build's packed / saved-input ops
(``*_packed``, ``rms_norm_forward_lean``), the Functions use them: parameters
are packed once per call instead of pointer tables, and the band split and
RMSNorm save their input instead of writing a normalised copy.  The math and
the results (within the stated tolerances) are those of the reference ops.

The HIP extension itself never falls back: if it is missing the backend
reports ``active="off"`` with the reason, exactly like the reference.
"""

from __future__ import annotations

import os
import types
import warnings
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn.functional as F

from .fused_extension import FusedKernelUnavailable, load_fused_band_split_extension
from .packed_params import band_split_packs, mask_layer_packs

CORE_GROUPED_TRAIN_ENV = "PYMSS_CORE_EXPERIMENTAL_TRAIN_GROUPED_BANDS"
EXPERIMENTAL_GROUPED_LINEAR_ENV = "PYMSST_EXPERIMENTAL_FUSED_GROUPED_LINEAR"
EXPERIMENTAL_BAND_SPLIT_BWD_V2_ENV = "PYMSST_EXPERIMENTAL_BANDSPLIT_BWD_V2"
EXPERIMENTAL_BAND_SPLIT_BWD_V3_ENV = "PYMSST_EXPERIMENTAL_BANDSPLIT_BWD_V3"
EXPERIMENTAL_BAND_SPLIT_RAGGED_FORWARD_ENV = "PYMSST_EXPERIMENTAL_BANDSPLIT_RAGGED_FORWARD"
EXPERIMENTAL_BAND_SPLIT_RAGGED_BACKWARD_ENV = "PYMSST_EXPERIMENTAL_BANDSPLIT_RAGGED_BACKWARD"
EXPERIMENTAL_ROTARY_ENV = "PYMSST_EXPERIMENTAL_FUSED_ROTARY"
EXPERIMENTAL_RMS_NORM_ENV = "PYMSST_EXPERIMENTAL_FUSED_RMSNORM"
EXPERIMENTAL_RMS_NORM_BWD_V2_ENV = "PYMSST_EXPERIMENTAL_RMSNORM_BWD_V2"
EXPERIMENTAL_ATTENTION_GATES_ENV = "PYMSST_EXPERIMENTAL_FUSED_ATTENTION_GATES"
EXPERIMENTAL_LAYOUT_REDUCE_COPY_ENV = "PYMSST_EXPERIMENTAL_LAYOUT_REDUCE_COPY"
EXPERIMENTAL_MASK_ESTIMATOR_FINAL_ENV = "PYMSST_EXPERIMENTAL_MASK_ESTIMATOR_FINAL_FUSED"
EXPERIMENTAL_MASK_ESTIMATOR_FINAL_DIRECT_ENV = "PYMSST_EXPERIMENTAL_MASK_ESTIMATOR_FINAL_DIRECT"
EXPERIMENTAL_MASK_FINAL_AUTOGRAD_ENV = "PYMSST_EXPERIMENTAL_MASK_FINAL_AUTOGRAD"
EXPERIMENTAL_TRAIN_PARAM_PACK_AUTOGRAD_ENV = "PYMSST_EXPERIMENTAL_TRAIN_PARAM_PACK_AUTOGRAD"
# This build's addition: with the fused mask final layer, also run the hidden Linear + tanh of a
# depth-2 mask MLP on the HIP kernels (hidden forward with a tanh epilogue; tanh' fused into the
# final layer's dx epilogue; grouped-linear backward on the GPU).
EXPERIMENTAL_FUSED_MASK_MLP_ENV = "PYMSST_EXPERIMENTAL_FUSED_MASK_MLP"
# This build's addition: the Mel-band RoFormer's band gather and overlap-averaged mask scatter on
# the HIP band-row kernels.
EXPERIMENTAL_FUSED_MEL_BANDS_ENV = "PYMSST_EXPERIMENTAL_FUSED_MEL_BANDS"
# This build's addition: the complex mask product and the iSTFT-layout permute (plus the zero-DC
# fill) of the BS-RoFormer output in one HIP pass each way.
EXPERIMENTAL_FUSED_MASK_APPLY_ENV = "PYMSST_EXPERIMENTAL_FUSED_MASK_APPLY"

_TRUE = {"1", "true", "yes", "on"}
_FLOAT_TYPES = (torch.float16, torch.bfloat16, torch.float32)

# The reference's "train_fragmentation" runtime preset (src/pymsst/training/module.py:22-36),
# plus the rotary flag this build also enables in its "hip_full" preset.
RUNTIME_PRESETS: dict[str, dict[str, str]] = {
    "off": {},
    "train_fragmentation": {
        EXPERIMENTAL_BAND_SPLIT_RAGGED_FORWARD_ENV: "1",
        EXPERIMENTAL_BAND_SPLIT_RAGGED_BACKWARD_ENV: "1",
        EXPERIMENTAL_BAND_SPLIT_BWD_V3_ENV: "1",
        EXPERIMENTAL_RMS_NORM_BWD_V2_ENV: "1",
        EXPERIMENTAL_LAYOUT_REDUCE_COPY_ENV: "1",
        EXPERIMENTAL_MASK_FINAL_AUTOGRAD_ENV: "1",
        EXPERIMENTAL_MASK_ESTIMATOR_FINAL_DIRECT_ENV: "1",
    },
}
RUNTIME_PRESETS["hip_full"] = {
    **RUNTIME_PRESETS["train_fragmentation"],
    EXPERIMENTAL_ROTARY_ENV: "1",
    EXPERIMENTAL_FUSED_MASK_MLP_ENV: "1",
    EXPERIMENTAL_ATTENTION_GATES_ENV: "1",
    EXPERIMENTAL_FUSED_MEL_BANDS_ENV: "1",
    EXPERIMENTAL_FUSED_MASK_APPLY_ENV: "1",
}


def apply_runtime_preset(name: str) -> dict[str, str]:
    """Set the environment flags of a preset (existing values win, like ``os.environ.setdefault``)."""
    if name not in RUNTIME_PRESETS:
        raise ValueError(f"unknown runtime preset {name!r}; expected one of {sorted(RUNTIME_PRESETS)}")
    applied = {}
    for key, value in RUNTIME_PRESETS[name].items():
        applied[key] = os.environ.setdefault(key, value)
    return applied


@dataclass(frozen=True)
class FusedTrainingStatus:
    """Which parts of the model run on the fused kernels (fields of fr.py:32-53)."""

    requested: str
    active: str
    reason: str | None = None
    patched_band_splits: int = 0
    patched_band_split_bwd_v2: bool = False
    patched_band_split_bwd_v3: bool = False
    patched_band_split_ragged_forward: bool = False
    patched_band_split_ragged_backward: bool = False
    patched_rotary: bool = False
    patched_rms_norm: bool = False
    rms_norm_mode: str | None = None
    patched_rms_norm_bwd_v2: bool = False
    patched_single_stem_masks: bool = False
    patched_attention_gates: bool = False
    attention_gate_mode: str | None = None
    patched_layout_reduce_copy: bool = False
    patched_train_param_pack_autograd: bool = False
    patched_mask_final_autograd: bool = False
    patched_mask_estimator_final: bool = False
    mask_estimator_final_mode: str | None = None
    patched_mask_mlp: bool = False  # this build's addition (hidden Linear + tanh fused as well)
    patched_mel_bands: bool = False  # this build's addition (Mel-band gather / mask scatter)
    patched_mask_apply: bool = False  # this build's addition (mask product in the iSTFT layout)


# ---------------------------------------------------------------------- switchboard


def _flag(name: str) -> bool:
    return os.environ.get(name, "").strip().lower() in _TRUE


def normalize_fused_kernel_backend(value: str | None) -> str:
    """``fr.py:139-145``; ``"hip"``, ``"rocm"`` and ``"hip_ext"`` also select the fused backend."""
    backend = str(value or "off").strip().lower().replace("-", "_")
    if backend in {"", "none", "false", "0", "off", "default"}:
        return "off"
    if backend in {"cuda", "cuda_ext", "cuda_extension", "cpp_cuda", "cxx_cuda", "hip", "hip_ext", "rocm"}:
        return "cuda_ext"
    raise ValueError("fused_kernel_backend must be one of: off, cuda_ext")


def _rms_norm_mode_from_env() -> str | None:
    value = os.environ.get(EXPERIMENTAL_RMS_NORM_ENV, "").strip().lower()
    if value in {"mixed", "fp32", "safe"}:
        return "mixed"
    if value in {"1", "true", "yes", "on", "fast", "half"}:
        return "fast"
    return None


def normalize_fused_rms_norm_mode(value: str | None) -> str | None:
    """``fr.py:148-161``: ``None`` consults the environment."""
    if value is None:
        mode = _rms_norm_mode_from_env()
        if mode is not None:
            return mode
        return "fast" if _flag(EXPERIMENTAL_RMS_NORM_BWD_V2_ENV) else None
    mode = str(value).strip().lower().replace("-", "_")
    if mode in {"", "none", "false", "0", "off", "default"}:
        return None
    if mode in {"mixed", "fp32", "safe"}:
        return "mixed"
    if mode in {"1", "true", "yes", "on", "fast", "half", "fp16"}:
        return "fast"
    raise ValueError("fused_rms_norm_mode must be one of: off, fast, mixed")


def _band_split_bwd_mode(ext: Any) -> str | None:
    if _flag(EXPERIMENTAL_BAND_SPLIT_BWD_V3_ENV) and hasattr(ext, "band_split_backward_v3"):
        return "v3"
    if _flag(EXPERIMENTAL_BAND_SPLIT_BWD_V2_ENV) and hasattr(ext, "band_split_backward_v2"):
        return "v2"
    return None


def _ragged_forward_enabled(ext: Any) -> bool:
    return _flag(EXPERIMENTAL_BAND_SPLIT_RAGGED_FORWARD_ENV) and hasattr(ext, "band_split_ragged_forward")


def _ragged_backward_enabled(ext: Any) -> bool:
    return _flag(EXPERIMENTAL_BAND_SPLIT_RAGGED_BACKWARD_ENV) and hasattr(ext, "band_split_ragged_backward")


def _rms_norm_bwd_v2_enabled(ext: Any, mode: str | None) -> bool:
    return (
        mode == "fast"
        and _flag(EXPERIMENTAL_RMS_NORM_BWD_V2_ENV)
        and hasattr(ext, "rms_norm_forward_fp32_gamma")
        and hasattr(ext, "rms_norm_backward_fp32_gamma")
    )


def _attention_gates_mode() -> str | None:
    value = os.environ.get(EXPERIMENTAL_ATTENTION_GATES_ENV, "").strip().lower()
    return "full" if value in {"1", "true", "yes", "on", "full", "gate"} else None


def _mask_estimator_final_mode(ext: Any) -> str | None:
    if (
        _flag(EXPERIMENTAL_MASK_ESTIMATOR_FINAL_DIRECT_ENV)
        and hasattr(ext, "mask_estimator_final_direct_forward")
        and hasattr(ext, "mask_estimator_final_direct_backward")
    ):
        return "direct"
    if (
        _flag(EXPERIMENTAL_MASK_ESTIMATOR_FINAL_ENV)
        and hasattr(ext, "mask_estimator_final_forward")
        and hasattr(ext, "mask_estimator_final_backward")
    ):
        return "grouped"
    return None


def _mask_mlp_enabled(ext: Any) -> bool:
    return _flag(EXPERIMENTAL_FUSED_MASK_MLP_ENV) and all(
        hasattr(ext, n)
        for n in ("grouped_linear_forward_act", "grouped_linear_backward", "mask_estimator_final_forward_packed",
                  "mask_estimator_final_backward_packed")
    )


def apply_roformer_fused_training_backend(
    model: torch.nn.Module,
    backend: str | None,
    *,
    extension: Any | None = None,
    rms_norm_mode: str | None = None,
) -> FusedTrainingStatus:
    """Patch ``model``'s band split, RMSNorm, rotary and mask estimator onto the fused kernels."""
    normalized = normalize_fused_kernel_backend(backend)
    if normalized == "off":
        return FusedTrainingStatus(requested="off", active="off")
    try:
        ext = extension if extension is not None else load_fused_band_split_extension()
    except FusedKernelUnavailable as exc:
        warnings.warn(str(exc), RuntimeWarning, stacklevel=2)
        return FusedTrainingStatus(requested=normalized, active="off", reason=str(exc))

    bwd_mode = _band_split_bwd_mode(ext)
    n_band_splits = _patch_band_split_modules(model, ext, bwd_mode=bwd_mode)
    single_stem = _patch_single_stem_mask_estimation()
    rotary = _patch_core_rotary(ext) if _flag(EXPERIMENTAL_ROTARY_ENV) else False
    rms_mode = normalize_fused_rms_norm_mode(rms_norm_mode)
    rms_v2 = _rms_norm_bwd_v2_enabled(ext, rms_mode)
    rms = _patch_core_rms_norm(ext, rms_mode, use_bwd_v2=rms_v2) if rms_mode else False
    gate_mode = _attention_gates_mode()
    gates = _patch_core_attention_gates(ext, gate_mode) if gate_mode else False
    grouped_linear = _patch_core_grouped_linear(ext) if _flag(EXPERIMENTAL_GROUPED_LINEAR_ENV) else False
    layout = _patch_core_packed_params() if _flag(EXPERIMENTAL_LAYOUT_REDUCE_COPY_ENV) else False
    pack_autograd = layout and _flag(EXPERIMENTAL_TRAIN_PARAM_PACK_AUTOGRAD_ENV)
    final_autograd = layout and _flag(EXPERIMENTAL_MASK_FINAL_AUTOGRAD_ENV)
    final_mode = _mask_estimator_final_mode(ext)
    final = _patch_core_mask_estimator_final(ext, final_mode) if final_mode else False
    mask_mlp = final and _mask_mlp_enabled(ext)
    mel_bands = _patch_mel_bands(ext) if _flag(EXPERIMENTAL_FUSED_MEL_BANDS_ENV) else False
    mask_apply = _patch_mask_apply(ext) if _flag(EXPERIMENTAL_FUSED_MASK_APPLY_ENV) else False

    if not any((n_band_splits, single_stem, rotary, rms, gates, grouped_linear, layout, pack_autograd, final_autograd,
                final, mel_bands, mask_apply)):
        reason = "no compatible BandSplit modules were found"
        warnings.warn(reason, RuntimeWarning, stacklevel=2)
        return FusedTrainingStatus(requested=normalized, active="off", reason=reason)

    os.environ.setdefault(CORE_GROUPED_TRAIN_ENV, "1")
    ragged_fwd = n_band_splits > 0 and _ragged_forward_enabled(ext)
    return FusedTrainingStatus(
        requested=normalized,
        active=normalized,
        patched_band_splits=n_band_splits,
        patched_band_split_bwd_v2=n_band_splits > 0 and bwd_mode == "v2",
        patched_band_split_bwd_v3=n_band_splits > 0 and bwd_mode == "v3",
        patched_band_split_ragged_forward=ragged_fwd,
        patched_band_split_ragged_backward=ragged_fwd and _ragged_backward_enabled(ext),
        patched_rotary=rotary,
        patched_rms_norm=rms,
        rms_norm_mode=rms_mode if rms else None,
        patched_rms_norm_bwd_v2=rms and rms_v2,
        patched_single_stem_masks=single_stem,
        patched_attention_gates=gates,
        attention_gate_mode=gate_mode if gates else None,
        patched_layout_reduce_copy=layout,
        patched_train_param_pack_autograd=pack_autograd,
        patched_mask_final_autograd=final_autograd,
        patched_mask_estimator_final=final,
        mask_estimator_final_mode=final_mode if final else None,
        patched_mask_mlp=mask_mlp,
        patched_mel_bands=mel_bands,
        patched_mask_apply=mask_apply,
    )


# ---------------------------------------------------------------------- patches


def _core():
    from .core import bands, common, transformer

    return bands, transformer, common


def _patch_band_split_modules(model: torch.nn.Module, ext: Any, *, bwd_mode: str | None = None) -> int:
    """Per-instance rebinding of ``BandSplit._forward_grouped`` (fr.py:256-271)."""
    count = 0
    for module in model.modules():
        if module.__class__.__name__ != "BandSplit":
            continue
        if not hasattr(module, "_get_group_params") or not hasattr(module, "_dim_offsets"):
            continue
        if getattr(module, "_pymsst_fused_band_split", False):
            continue
        module._pymsst_original_forward_grouped = module._forward_grouped
        module._pymsst_fused_extension = ext
        module._pymsst_fused_band_split_bwd_mode = bwd_mode
        module._forward_grouped = types.MethodType(_forward_grouped_band_split_cuda_ext, module)
        module._pymsst_fused_band_split = True
        count += 1
    return count


def _patch_single_stem_mask_estimation() -> bool:
    """One active estimator: skip the stack (fr.py:299-318)."""
    try:
        _, _, common = _core()
    except Exception:
        return False
    current = common.RoformerRuntimeMixin._estimate_masks
    if getattr(current, "_pymsst_single_stem_shortcut", False):
        return True

    def estimate_masks_single_stem_shortcut(self, x):
        estimators = self._active_mask_estimators()
        if len(estimators) == 1:
            return estimators[0](x).unsqueeze(1)
        return current(self, x)

    estimate_masks_single_stem_shortcut._pymsst_single_stem_shortcut = True
    estimate_masks_single_stem_shortcut._pymsst_original_estimate_masks = current
    common.RoformerRuntimeMixin._estimate_masks = estimate_masks_single_stem_shortcut
    return True


def _patch_core_rotary(ext: Any) -> bool:
    """Module-level ``apply_rotary_emb_fast`` replacement (fr.py:710-732)."""
    if not hasattr(ext, "rotary_forward") or not hasattr(ext, "rotary_backward"):
        return False
    _, transformer, _ = _core()
    if getattr(transformer.apply_rotary_emb_fast, "_pymsst_fused_rotary", False):
        return True
    original = transformer.apply_rotary_emb_fast

    def apply_rotary_cuda_ext(cos, sin, t):
        if t.device.type != "cuda" or t.dtype not in _FLOAT_TYPES:
            return original(cos, sin, t)
        if t.ndim != 4 or cos.device != t.device or sin.device != t.device or cos.dtype != t.dtype or sin.dtype != t.dtype:
            return original(cos, sin, t)
        return _FusedRotary.apply(t, cos[..., ::2], sin[..., ::2], ext)

    apply_rotary_cuda_ext._pymsst_fused_rotary = True
    apply_rotary_cuda_ext._pymsst_original_apply_rotary = original
    transformer.apply_rotary_emb_fast = apply_rotary_cuda_ext
    return True


def _patch_core_rms_norm(ext: Any, mode: str, *, use_bwd_v2: bool = False) -> bool:
    """Class-level ``RMSNorm.forward`` replacement (fr.py:735-773)."""
    if mode == "mixed":
        required = ("rms_norm_forward_mixed", "rms_norm_backward_mixed")
    elif mode == "fast":
        required = (
            ("rms_norm_forward_fp32_gamma", "rms_norm_backward_fp32_gamma")
            if use_bwd_v2
            else ("rms_norm_forward", "rms_norm_backward")
        )
    else:
        return False
    if any(not hasattr(ext, name) for name in required):
        return False
    _, transformer, _ = _core()
    if getattr(transformer.RMSNorm.forward, "_pymsst_fused_rms_norm", False):
        return True
    original = transformer.RMSNorm.forward

    def rms_norm_cuda_ext(self, x):
        if not self.training or x.device.type != "cuda" or x.dtype not in _FLOAT_TYPES:
            return original(self, x)
        if use_bwd_v2 and mode == "fast" and self.gamma.dtype == torch.float32:
            return _FusedRMSNormFp32Gamma.apply(x, self.gamma, ext)
        if mode == "mixed" and self.gamma.dtype == torch.float32:
            return _FusedRMSNormMixed.apply(x, self.gamma, ext)
        return _FusedRMSNorm.apply(x, self.gamma.to(device=x.device, dtype=x.dtype), ext)

    rms_norm_cuda_ext._pymsst_fused_rms_norm = True
    rms_norm_cuda_ext._pymsst_fused_rms_norm_mode = mode
    rms_norm_cuda_ext._pymsst_fused_rms_norm_bwd_v2 = use_bwd_v2
    rms_norm_cuda_ext._pymsst_original_forward = original
    transformer.RMSNorm.forward = rms_norm_cuda_ext
    return True


def _patch_core_attention_gates(ext: Any, mode: str) -> bool:
    """Class-level ``Attention.forward`` replacement (fr.py:776-824): the gate Linear, sigmoid and
    multiply after SDPA run as one fused op; the rest of the block is the stock forward."""
    if mode != "full":
        return False
    if any(not hasattr(ext, name) for name in ("attention_gate_forward", "attention_gate_backward")):
        return False
    _, transformer, _ = _core()
    if getattr(transformer.Attention.forward, "_pymsst_fused_attention_gates", False):
        return True
    original = transformer.Attention.forward

    def attention_forward_cuda_ext(self, x):
        if (
            not self.training
            or x.device.type != "cuda"
            or x.dtype not in _FLOAT_TYPES
            or self.to_gates.bias is None
        ):
            return original(self, x)
        x = self.norm(x)
        qkv = self.to_qkv(x)
        flash_layout = False
        if self.rotary_embed is not None and _fused_qkv_split_ok(ext, qkv):
            # rotary patch active too: split + rotate (+ gradient stacking) in one op each way.  In
            # 16-bit, q/k/v are written dense [B, N, H, D]: SDPA's flash kernels read that layout in
            # place and then write their output, and read its gradient, in it as well, so neither
            # direction copies q, k, v, the output or its gradient
            flash_layout = qkv.dtype in (torch.float16, torch.bfloat16)
            cos, sin = self.rotary_embed.tables(qkv.shape[1], qkv.device, qkv.dtype)
            q, k, v = _FusedQKVRotary.apply(qkv, cos[..., ::2], sin[..., ::2], self.heads, ext,
                                            "bnhd" if flash_layout else "bhnd")
        else:
            q, k, v = transformer.qkv_to_bnhd(qkv, self.heads)
            if self.rotary_embed is not None:
                q, k = transformer.rotate_qk_fast_bnhd(self.rotary_embed, q, k)
        q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
        if flash_layout:
            # the stock _attention's .contiguous() would copy these [B, H, N, D] views back
            out = transformer._sdpa(q, k, v, self.dropout if self.training else 0.0).transpose(1, 2)
        else:
            out = self._attention(q, k, v).transpose(1, 2)
        gate_dtype = out.dtype
        gated = _FusedAttentionGate.apply(
            out,
            x.to(dtype=gate_dtype),
            self.to_gates.weight.to(dtype=gate_dtype),
            self.to_gates.bias.to(dtype=gate_dtype),
            ext,
        )
        return self.to_out(gated)

    attention_forward_cuda_ext._pymsst_fused_attention_gates = True
    attention_forward_cuda_ext._pymsst_fused_attention_gate_mode = mode
    attention_forward_cuda_ext._pymsst_original_forward = original
    transformer.Attention.forward = attention_forward_cuda_ext
    return True


def _mel_plan(module, ext: Any, device: torch.device):
    plan = getattr(module, "_pymsst_mel_plan", None)
    if plan is None or plan.rows.device != device:
        plan = ext.band_rows_plan(module.band_rows, module.num_rows, device)
        module._pymsst_mel_plan = plan
    return plan


def _patch_mel_bands(ext: Any) -> bool:
    """Class-level ``MelBandRoformer._band_features`` / ``_spectral_mask`` replacement (no reference
    counterpart: pymss-core's Mel-band model does the gather with indexing and the average with
    scatter_add + division)."""
    if any(not hasattr(ext, n) for n in ("band_rows_plan", "band_rows_gather", "band_rows_scatter")):
        return False
    from .core import mel_band_roformer as mbr

    cls = mbr.MelBandRoformer
    if getattr(cls._band_features, "_pymsst_fused_mel_bands", False):
        return True
    orig_features, orig_mask = cls._band_features, cls._spectral_mask

    def band_features_cuda_ext(self, spec):
        if not spec.is_cuda or spec.dtype != torch.complex64:
            return orig_features(self, spec)
        plan = _mel_plan(self, ext, spec.device)
        b, _, t = spec.shape
        return _FusedBandGather.apply(torch.view_as_real(spec), plan, ext).reshape(b, t, -1)

    def spectral_mask_cuda_ext(self, mask):
        if not mask.is_cuda or mask.dtype not in _FLOAT_TYPES:
            return orig_mask(self, mask)
        plan = _mel_plan(self, ext, mask.device)
        return torch.view_as_complex(_FusedMaskScatterMean.apply(mask, plan, ext))

    band_features_cuda_ext._pymsst_fused_mel_bands = True
    band_features_cuda_ext._pymsst_original_band_features = orig_features
    spectral_mask_cuda_ext._pymsst_fused_mel_bands = True
    spectral_mask_cuda_ext._pymsst_original_spectral_mask = orig_mask
    cls._band_features = band_features_cuda_ext
    cls._spectral_mask = spectral_mask_cuda_ext
    return True


def _patch_mask_apply(ext: Any) -> bool:
    """Class-level ``BSRoformer._masked_spectrum`` replacement (no reference kernel: the stock model
    multiplies the spectrum by the float-cast masks through a transposed complex view and permutes
    the product for the iSTFT, cuda_graph.py:140-158).  Models whose ``_spectral_mask`` is not the
    BS-RoFormer one (the Mel-band model averages band masks first) keep the stock method."""
    if any(not hasattr(ext, n) for n in ("mask_apply_forward", "mask_apply_backward")):
        return False
    from .core import bs_roformer

    cls = bs_roformer.BSRoformer
    if getattr(cls._masked_spectrum, "_pymsst_fused_mask_apply", False):
        return True
    original = cls._masked_spectrum
    stock_spectral_mask = cls._spectral_mask

    def masked_spectrum_cuda_ext(self, spec, mask, channels):
        if (type(self)._spectral_mask is not stock_spectral_mask or not spec.is_cuda
                or spec.dtype != torch.complex64 or mask.dtype not in _FLOAT_TYPES or mask.dim() != 4):
            return original(self, spec, mask, channels)
        return _FusedMaskApply.apply(spec, mask, channels, bool(getattr(self, "zero_dc", False)), ext)

    masked_spectrum_cuda_ext._pymsst_fused_mask_apply = True
    masked_spectrum_cuda_ext._pymsst_original_masked_spectrum = original
    cls._masked_spectrum = masked_spectrum_cuda_ext

    # With the one-pass mask MLP active too, the mask product moves into that kernel's epilogue: the
    # stock path writes every stem's mask, then multiplies the spectrum by it and permutes the product
    # for the iSTFT; here the masks are never written.
    original_core = cls._mask_core
    stock_masks = cls._masks

    def mask_core_cuda_ext(self, spec, channels):
        bands, _, _ = _core()
        if (not self.training or type(self)._spectral_mask is not stock_spectral_mask
                or type(self)._masks is not stock_masks or not spec.is_cuda or spec.dtype != torch.complex64
                or spec.requires_grad or not hasattr(ext, "mask_mlp_forward_apply") or not _mask_mlp_enabled(ext)
                or not getattr(bands.MaskEstimator._forward_layer_grouped_mlp, "_pymsst_mask_estimator_final_fused",
                               False)):
            return original_core(self, spec, channels)
        x = self._mask_features(spec)
        params, dims = [], None
        for est in self._active_mask_estimators():
            plan = est._layer_grouping_plan()
            ops = _mask_mlp_operands(est, x, plan) if plan and x.device.type == "cuda" else None
            if ops is None or not _one_pass_mask_mlp(ext, ops[0], ops[1], ops[5]) or (dims is not None
                                                                                      and ops[5] != dims):
                return self._masked_spectrum(spec, self._estimate_masks(x), channels)
            x3, dims = ops[0], ops[5]
            params += list(ops[1:5])
        return _FusedMaskMLPApply.apply(spec, x3, channels, bool(getattr(self, "zero_dc", False)), dims, ext, *params)

    mask_core_cuda_ext._pymsst_fused_mask_apply = True
    mask_core_cuda_ext._pymsst_original_mask_core = original_core
    cls._mask_core = mask_core_cuda_ext
    return True


def _patch_core_grouped_linear(ext: Any) -> bool:
    """Module-level ``bands.grouped_linear`` replacement (fr.py:274-296)."""
    if not hasattr(ext, "grouped_linear_forward"):
        return False
    bands, _, _ = _core()
    if getattr(bands.grouped_linear, "_pymsst_fused_grouped_linear", False):
        return True
    original = bands.grouped_linear

    def grouped_linear_cuda_ext(x, weight, bias):
        if x.device.type != "cuda" or x.dtype not in _FLOAT_TYPES:
            return original(x, weight, bias)
        if weight.device != x.device or weight.dtype != x.dtype or (
            bias is not None and (bias.device != x.device or bias.dtype != x.dtype)
        ):
            return original(x, weight, bias)
        return _FusedGroupedLinear.apply(x, weight, bias, ext)

    grouped_linear_cuda_ext._pymsst_fused_grouped_linear = True
    grouped_linear_cuda_ext._pymsst_original_grouped_linear = original
    bands.grouped_linear = grouped_linear_cuda_ext
    return True


# ---------------------------------------------------------------------- packed parameters


def _run_of(indices) -> tuple[int, int] | None:
    """``(start, end)`` when ``indices`` are consecutive band numbers."""
    idx = tuple(int(i) for i in indices)
    if idx and idx == tuple(range(idx[0], idx[0] + len(idx))):
        return idx[0], idx[0] + len(idx)
    return None


def _packed_band_group_params(self, start, end, device, dtype):
    """``BandSplit._get_group_params`` served from the module's flat parameter storages: the stacked
    ``(gamma[G, I], weight[G, O, I], bias[G, O] | None)`` of bands ``[start, end)`` are views (cast once
    per optimizer step under autocast), not per-step stacks."""
    gamma_p, weight_p, bias_p = band_split_packs(self)
    if gamma_p.storage.device != torch.device(device) or (bias_p is None and self.to_features[start][1].bias is not None):
        return self._pymsst_stock_get_group_params(start, end, device, dtype)
    return (gamma_p.group(start, end, dtype), weight_p.group(start, end, dtype),
            bias_p.group(start, end, dtype) if bias_p is not None else None)


def _packed_layer_group_params(self, layer_index, signature, indices, device, dtype):
    """``MaskEstimator._get_layer_group_params`` from the flat storages when the bands are a consecutive
    run (views, no stack); other groups keep the stock stack."""
    run = _run_of(indices)
    if run is not None:
        weight_p, bias_p = mask_layer_packs(self, layer_index)
        lin = self._band_groupable_layers()[run[0]][layer_index][1]
        if weight_p.storage.device == torch.device(device) and (bias_p is not None or lin.bias is None):
            return (weight_p.group(run[0], run[1], dtype),
                    bias_p.group(run[0], run[1], dtype) if bias_p is not None else None)
    return self._pymsst_stock_get_layer_group_params(layer_index, signature, indices, device, dtype)


def _bands_of(module, h, indices):
    """``h[..., indices, :]``: a narrow for a run of bands, one index_select otherwise."""
    run = _run_of(indices)
    if run is not None:
        return h.narrow(-2, run[0], run[1] - run[0])
    return h.index_select(-2, module._indices_tensor(tuple(indices), h.device))


def _grouped_mlp_forward(self, x):
    """The mask MLP with one grouped Linear per group of bands sharing a layer signature
    (fr.py:332-369 runs the same grouping): hidden layers concatenate the groups' outputs and, when the
    groups are not runs in band order, restore band order with one index_select; the last layer's
    per-band GLU outputs are concatenated in band order."""
    bands, _, _ = _core()
    plan = self._layer_grouping_plan()
    if plan is None:
        return None
    h = x
    for li, (kind, groups) in enumerate(plan):
        if kind == "tanh":
            h = bands.inference_tanh(h)
            continue
        last = li == len(plan) - 1
        if not last and len({sig[1] for sig, _ in groups}) != 1:
            return None
        ys, order = [], []
        for sig, idx in groups:
            w, b = self._get_layer_group_params(li, sig, idx, x.device, x.dtype)
            part = _bands_of(self, h, idx)
            if last and _flag(EXPERIMENTAL_MASK_FINAL_AUTOGRAD_ENV):
                ys.append(_MaskFinalGroupedLinearGLU.apply(part, w, b))
            elif last:
                ys.append(F.glu(bands.grouped_linear(part, w, b), dim=-1))
            else:
                ys.append(bands.grouped_linear(part, w, b))
            order.extend(int(i) for i in idx)
        in_order = order == list(range(len(order)))
        if last:
            if in_order:
                return torch.cat([y.flatten(-2) for y in ys], dim=-1)
            per_band = [None] * len(order)
            for y, band in zip((t for y in ys for t in y.unbind(-2)), order):
                per_band[band] = y
            return torch.cat(per_band, dim=-1)
        h = torch.cat(ys, dim=-2)
        if not in_order:
            inverse = [0] * len(order)
            for pos, band in enumerate(order):
                inverse[band] = pos
            h = h.index_select(-2, self._indices_tensor(tuple(inverse), h.device))
    return None


def _patch_core_packed_params() -> bool:
    """``PYMSST_EXPERIMENTAL_LAYOUT_REDUCE_COPY`` (fr.py:321-500): the band modules' grouped parameters
    come from flat per-kind storages (``pymsst_amd.packed_params``) as views instead of per-step stacks,
    and the mask MLP runs :func:`_grouped_mlp_forward`."""
    try:
        bands, _, _ = _core()
    except Exception:
        return False
    BS, ME = bands.BandSplit, bands.MaskEstimator
    if not getattr(BS._get_group_params, "_pymsst_packed", False):
        BS._pymsst_stock_get_group_params = BS._get_group_params
        _packed_band_group_params._pymsst_packed = True
        _packed_band_group_params._pymsst_original_get_group_params = BS._get_group_params
        BS._get_group_params = _packed_band_group_params
    if not getattr(ME._get_layer_group_params, "_pymsst_packed", False):
        ME._pymsst_stock_get_layer_group_params = ME._get_layer_group_params
        _packed_layer_group_params._pymsst_packed = True
        _packed_layer_group_params._pymsst_original_get_layer_group_params = ME._get_layer_group_params
        ME._get_layer_group_params = _packed_layer_group_params
    if not getattr(ME._forward_layer_grouped_mlp, "_pymsst_packed", False):
        _grouped_mlp_forward._pymsst_packed = True
        _grouped_mlp_forward._pymsst_original_forward_layer_grouped_mlp = ME._forward_layer_grouped_mlp
        ME._forward_layer_grouped_mlp = _grouped_mlp_forward
    return True


def _patch_core_mask_estimator_final(ext: Any, mode: str) -> bool:
    """Final mask-MLP layer + GLU on the fused kernels (fr.py:503-590).

    The reference disables its cuBLAS "grouped" mode below sm90 (fr.py:510-517); both
    modes run the same MFMA kernels here, so both are always available.
    """
    names = (
        ("mask_estimator_final_direct_forward", "mask_estimator_final_direct_backward")
        if mode == "direct"
        else ("mask_estimator_final_forward", "mask_estimator_final_backward")
    )
    if any(not hasattr(ext, n) for n in names):
        return False
    try:
        bands, _, _ = _core()
    except Exception:
        return False
    ME = bands.MaskEstimator
    if getattr(ME._forward_layer_grouped_mlp, "_pymsst_mask_estimator_final_fused", False):
        return True
    original = ME._forward_layer_grouped_mlp

    def forward_layer_grouped_mlp_mask_final_fused(self, x):
        if x.device.type != "cuda" or x.dtype not in _FLOAT_TYPES:
            return original(self, x)
        plan = self._layer_grouping_plan()
        if not plan or plan[-1][0] != "linear":
            return original(self, x)
        if _mask_mlp_enabled(ext):
            fused = _fused_mask_mlp(self, x, plan, ext)
            if fused is not None:
                return fused
        # hidden layers: one grouped Linear per group of bands (all groups must share the output
        # width), outputs back in band order
        h = x
        for li, (kind, groups) in enumerate(plan[:-1]):
            if kind == "tanh":
                h = bands.inference_tanh(h)
                continue
            if len({sig[1] for sig, _ in groups}) != 1:
                return original(self, x)
            ys, order = [], []
            for sig, idx in groups:
                w, b = self._get_layer_group_params(li, sig, idx, x.device, x.dtype)
                ys.append(bands.grouped_linear(_bands_of(self, h, idx), w, b))
                order.extend(int(i) for i in idx)
            h = torch.cat(ys, dim=-2)
            if order != list(range(len(order))):
                inverse = [0] * len(order)
                for pos, band in enumerate(order):
                    inverse[band] = pos
                h = h.index_select(-2, self._indices_tensor(tuple(inverse), h.device))
        last = len(plan) - 1
        for b_idx, layers in enumerate(self._band_groupable_layers()):
            kind, lin = layers[last]
            if kind != "linear" or lin.bias is None:
                return original(self, x)
            if lin.in_features != h.shape[-1] or lin.out_features != self.dim_inputs[b_idx] * 2:
                return original(self, x)
        weight_p, bias_p = mask_layer_packs(self, last)
        if weight_p.storage.device != h.device:
            return original(self, x)
        lead = h.shape[:-2]
        h3 = h.reshape(-1, len(self.to_freqs), h.shape[-1])
        if _packed_mask_final_ops(ext):
            out = _FusedMaskEstimatorFinalPacked.apply(
                h3, weight_p.flat(h.dtype), bias_p.flat(h.dtype), ext, tuple(int(d) for d in self.dim_inputs))
        else:
            weights = [v.view(s) for v, s in zip(weight_p.flat(h.dtype).split(weight_p.sizes), weight_p.shapes)]
            out = _FusedMaskEstimatorFinal.apply(
                h3, bias_p.flat(h.dtype), _dim_offsets_tensor(self, x.device), ext,
                tuple(int(d) for d in self.dim_inputs), mode, *weights,
            )
        return out.reshape(*lead, self._dim_total)

    forward_layer_grouped_mlp_mask_final_fused._pymsst_mask_estimator_final_fused = True
    forward_layer_grouped_mlp_mask_final_fused._pymsst_original_forward_layer_grouped_mlp = original
    ME._forward_layer_grouped_mlp = forward_layer_grouped_mlp_mask_final_fused
    return True


def _packed_mask_final_ops(ext) -> bool:
    return hasattr(ext, "mask_estimator_final_forward_packed") and hasattr(ext, "mask_estimator_final_backward_packed")


def _fused_mask_mlp(module, x, plan, ext):
    """Whole depth-2 mask MLP (Linear -> tanh -> Linear -> GLU) on the kernels, or ``None`` when the
    module does not have that shape.  The parameters come from the module's flat storages (the
    first layer's ``[NB, H, dim]`` stack is a view); under autocast they and x are in the autocast
    dtype, as for the stock grouped GEMMs."""
    ops = _mask_mlp_operands(module, x, plan)
    if ops is None:
        return None
    x3, w1, b1, w2, b2, dims, lead = ops
    out = _FusedMaskMLP.apply(x3, w1, b1, w2, b2, ext, dims)
    return out.reshape(*lead, module._dim_total)


def _mask_mlp_operands(module, x, plan):
    """``(x3[M, NB, dim], w1[NB, H, dim], b1[NB, H], w2 (packed), b2[2F], dim_inputs, lead shape)`` of a
    depth-2 mask MLP in the compute dtype, or ``None`` when the module does not have that shape."""
    nb = len(module.to_freqs)
    if len(plan) != 3 or plan[0][0] != "linear" or plan[1][0] != "tanh" or plan[2][0] != "linear":
        return None
    groups = plan[0][1]
    if len(groups) != 1 or tuple(groups[0][1]) != tuple(range(nb)):
        return None
    layers = module._band_groupable_layers()
    first = [band[0][1] for band in layers]
    last = [band[2][1] for band in layers]
    if any(l.bias is None for l in first) or any(l.bias is None for l in last):
        return None
    if first[0].in_features != x.shape[-1]:
        return None
    if any(l.out_features != 2 * d or l.in_features != first[0].out_features for l, d in zip(last, module.dim_inputs)):
        return None
    w1_p, b1_p = mask_layer_packs(module, 0)
    w2_p, b2_p = mask_layer_packs(module, 2)
    if w1_p.storage.device != x.device:
        return None
    dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else x.dtype
    hidden = first[0].out_features
    lead = x.shape[:-2]
    x3 = x.reshape(-1, nb, x.shape[-1]).to(dt)
    w1 = w1_p.group(0, nb, dt)
    b1 = b1_p.group(0, nb, dt)
    return (x3, w1.view(nb, hidden, -1), b1.view(nb, hidden), w2_p.flat(dt), b2_p.flat(dt),
            tuple(int(d) for d in module.dim_inputs), lead)


def _dim_offsets_tensor(module, device) -> torch.Tensor:
    """Device int64 copy of ``module._dim_offsets``, cached per device (fr.py:592-602, 876-885)."""
    cache = getattr(module, "_pymsst_dim_offsets_cache", None)
    if cache is None:
        cache = module._pymsst_dim_offsets_cache = {}
    key = (device.type, device.index)
    hit = cache.get(key)
    if hit is None:
        with torch.inference_mode(False):  # a normal tensor, whichever mode builds the cache
            hit = cache[key] = torch.as_tensor(module._dim_offsets, dtype=torch.long, device=device)
    return hit


# ---------------------------------------------------------------------- band split forward


def _packed_band_split_ops(ext) -> bool:
    return hasattr(ext, "band_split_ragged_forward_packed") and hasattr(ext, "band_split_ragged_backward_packed")


def _forward_grouped_band_split_cuda_ext(self, x: torch.Tensor) -> torch.Tensor:
    """Patched ``BandSplit._forward_grouped`` (fr.py:827-873)."""
    if not self.training or x.device.type != "cuda" or x.dtype not in _FLOAT_TYPES:
        return self._pymsst_original_forward_grouped(x)
    ext = self._pymsst_fused_extension
    bwd_mode = getattr(self, "_pymsst_fused_band_split_bwd_mode", None)
    lead = x.shape[:-1]
    ragged = _ragged_forward_enabled(ext)
    if ragged and any(net[1].bias is None for net in self.to_features):
        return self._pymsst_original_forward_grouped(x)
    # Under autocast the input is the fp32 STFT and the reference runs its kernels in x's dtype
    # (fr.py:827-857: parameters fetched in x.dtype), so the norm and its gradients are fp32.  With
    # the mixed op the projection then runs where the stock module's nn.Linear does: operands and
    # output in the autocast dtype, so the residual stream that follows has the stock dtype.
    amp = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None
    if ragged:
        dims = tuple(int(d) for d in self.dim_inputs)
        if (amp in (torch.float16, torch.bfloat16) and x.dtype == torch.float32
                and _packed_band_split_ops(ext) and hasattr(ext, "band_split_mixed_forward")):
            gamma_p, weight_p, bias_p = band_split_packs(self)
            if gamma_p.storage.device == x.device and gamma_p.storage.dtype == torch.float32:
                out = _FusedBandSplitMixed.apply(x.reshape(-1, x.shape[-1]), gamma_p.flat(torch.float32),
                                                 weight_p.flat(amp), bias_p.flat(amp), ext, dims, amp)
                return out.reshape(*lead, len(dims), -1)
        if _packed_band_split_ops(ext):
            gamma_p, weight_p, bias_p = band_split_packs(self)
            if gamma_p.storage.device == x.device:
                out = _FusedBandSplitPacked.apply(x.reshape(-1, x.shape[-1]), gamma_p.flat(x.dtype),
                                                  weight_p.flat(x.dtype), bias_p.flat(x.dtype), ext, dims)
                return out.reshape(*lead, len(dims), -1)
        gammas = [net[0].gamma.to(x.dtype) for net in self.to_features]
        weights = [net[1].weight.to(x.dtype) for net in self.to_features]
        biases = [net[1].bias.to(x.dtype) for net in self.to_features]
        out = _FusedBandSplitRagged.apply(
            x.reshape(-1, x.shape[-1]), _dim_offsets_tensor(self, x.device), ext, dims, bwd_mode,
            *gammas, *weights, *biases,
        )
        return out.reshape(*lead, len(dims), -1)
    outs = []
    for start, end, width in self._dim_groups:
        part = x[..., self._dim_offsets[start] : self._dim_offsets[end]].reshape(-1, end - start, width)
        gamma, weight, bias = self._get_group_params(start, end, x.device, x.dtype)
        y = _FusedBandSplitGroup.apply(part, gamma, weight, bias, ext, bwd_mode)
        outs.append(y.reshape(*lead, end - start, -1))
    return torch.cat(outs, dim=-2)


# ---------------------------------------------------------------------- autograd Functions


class _FusedBandSplitGroup(torch.autograd.Function):
    """Equal-width band group (fr.py:888-926): ``ext.band_split_forward`` / ``band_split_backward{,_v2,_v3}``."""

    @staticmethod
    def forward(ctx, x, gamma, weight, bias, extension, bwd_mode):
        out, normed, inv_norm = extension.band_split_forward(x, gamma, weight, bias)
        ctx.save_for_backward(normed, inv_norm, gamma, weight)
        ctx.has_bias = bias is not None
        ctx.extension = extension
        ctx.bwd_mode = bwd_mode
        return out

    @staticmethod
    def backward(ctx, grad_out):
        normed, inv_norm, gamma, weight = ctx.saved_tensors
        grad_out = grad_out.reshape(normed.shape[0], normed.shape[1], weight.shape[1]).contiguous()
        fn = {
            "v3": getattr(ctx.extension, "band_split_backward_v3", None),
            "v2": getattr(ctx.extension, "band_split_backward_v2", None),
        }.get(ctx.bwd_mode) or ctx.extension.band_split_backward
        dx, dgamma, dweight, dbias = fn(grad_out, normed, inv_norm, gamma, weight, ctx.has_bias)
        return dx, dgamma, dweight, (dbias if ctx.has_bias else None), None, None


class _FusedBandSplitRagged(torch.autograd.Function):
    """All bands in one launch (fr.py:929-1026).

    With the packed ops the parameters are concatenated once, the input itself is
    saved (no ``normed`` write) and the backward returns per-band views of the
    packed gradients.
    """

    @staticmethod
    def forward(ctx, x, dim_offsets, extension, dim_inputs, bwd_mode, *params):
        nb = len(dim_inputs)
        gammas, weights, biases = params[:nb], params[nb : 2 * nb], params[2 * nb :]
        ctx.extension = extension
        ctx.dim_inputs = dim_inputs
        ctx.bwd_mode = bwd_mode
        ctx.band_count = nb
        ctx.input_shape = tuple(x.shape)
        ctx.out_features = weights[0].shape[0]
        ctx.use_ragged_backward = _ragged_backward_enabled(extension)
        ctx.packed = hasattr(extension, "band_split_ragged_forward_packed") and hasattr(
            extension, "band_split_ragged_backward_packed"
        )
        if ctx.packed:
            x = x.contiguous()
            gamma_all = torch.cat([g.reshape(-1) for g in gammas])
            weight_all = torch.cat([w.reshape(-1) for w in weights])
            bias_all = torch.cat([b.reshape(-1) for b in biases])
            out, _, inv_norm = extension.band_split_ragged_forward_packed(
                x, gamma_all, weight_all, bias_all, dim_inputs, write_normed=False
            )
            ctx.save_for_backward(x, inv_norm, gamma_all, weight_all)
            return out
        out, normed, inv_norm = extension.band_split_ragged_forward(
            x, list(gammas), list(weights), list(biases), list(dim_inputs), dim_offsets
        )
        ctx.save_for_backward(normed, inv_norm, dim_offsets, *gammas, *weights)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        nb = ctx.band_count
        o = ctx.out_features
        grad_out = grad_out.reshape(grad_out.shape[0], nb, o).contiguous()
        dims = [int(d) for d in ctx.dim_inputs]
        if ctx.packed:
            x, inv_norm, gamma_all, weight_all = ctx.saved_tensors
            dx, dg, dw, db = ctx.extension.band_split_ragged_backward_packed(
                grad_out, x, True, inv_norm, gamma_all, weight_all, ctx.dim_inputs, True
            )
            dgs = dg.split(dims)
            dws = [v.view(o, d) for v, d in zip(dw.split([o * d for d in dims]), dims)]
            dbs = db.view(nb, o).unbind(0)
            return (dx, None, None, None, None, *dgs, *dws, *dbs)
        normed, inv_norm, dim_offsets, *params = ctx.saved_tensors
        gammas, weights = params[:nb], params[nb:]
        if ctx.use_ragged_backward:
            res = ctx.extension.band_split_ragged_backward(
                grad_out, normed, inv_norm, list(gammas), list(weights), list(ctx.dim_inputs), dim_offsets
            )
            return (res[0], None, None, None, None, *res[1:])
        # per-band reference path (fr.py:995-1026), offsets from the host copy (no device sync)
        dx = grad_out.new_zeros(ctx.input_shape)
        fn = {
            "v3": getattr(ctx.extension, "band_split_backward_v3", None),
            "v2": getattr(ctx.extension, "band_split_backward_v2", None),
        }.get(ctx.bwd_mode) or ctx.extension.band_split_backward
        dgs, dws, dbs = [], [], []
        start = 0
        for b, d in enumerate(dims):
            nb_ = normed[:, start : start + d].reshape(normed.shape[0], 1, d)
            g, gw, gg, gb = fn(grad_out[:, b : b + 1, :].contiguous(), nb_.contiguous(),
                               inv_norm[:, b : b + 1].contiguous(), gammas[b].unsqueeze(0), weights[b].unsqueeze(0),
                               True)
            dx[:, start : start + d] = g.reshape(-1, d)
            dgs.append(gw[0])
            dws.append(gg[0])
            dbs.append(gb[0])
            start += d
        return (dx, None, None, None, None, *dgs, *dws, *dbs)


class _FusedBandSplitPacked(torch.autograd.Function):
    """All bands in one launch on the flat parameter buffers (this build's form of fr.py:929-1026):
    ``gamma_all[F]``, ``weight_all`` (the ``[O, I_b]`` weights back to back), ``bias_all[NB*O]``.  Saves
    x (not a normalised copy) and inv_norm; the backward returns the flat gradients, which the
    parameter view's backward splits per band."""

    @staticmethod
    def forward(ctx, x, gamma_all, weight_all, bias_all, extension, dim_inputs):
        x = x.contiguous()
        out, _, inv_norm = extension.band_split_ragged_forward_packed(x, gamma_all, weight_all, bias_all, dim_inputs,
                                                                     write_normed=False)
        ctx.extension, ctx.dim_inputs = extension, dim_inputs
        ctx.save_for_backward(x, inv_norm, gamma_all, weight_all)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, inv_norm, gamma_all, weight_all = ctx.saved_tensors
        nb = len(ctx.dim_inputs)
        grad_out = grad_out.reshape(x.shape[0], nb, -1).contiguous()
        dx, dg, dw, db = ctx.extension.band_split_ragged_backward_packed(
            grad_out, x, True, inv_norm, gamma_all, weight_all, ctx.dim_inputs, True)
        return dx, dg, dw, db, None, None


class _FusedBandSplitMixed(torch.autograd.Function):
    """The packed band split of an fp32 input under autocast (fr.py:827-857 with the fp32 STFT): the
    norm, ``inv_norm``, dx and dgamma in fp32; the projection on ``dtype`` operands, rounded where the
    stock nn.Linear rounds them (its input ``x * inv * sqrt(I) * gamma`` and its input gradient), with
    its output and weight / bias gradients in ``dtype``.  Saves x, the projection input and inv_norm."""

    @staticmethod
    def forward(ctx, x, gamma_all, weight_all, bias_all, extension, dim_inputs, dtype):
        x = x.contiguous()
        out, feats, inv_norm = extension.band_split_mixed_forward(x, gamma_all, weight_all, bias_all, dim_inputs,
                                                                  dtype)
        ctx.extension, ctx.dim_inputs = extension, dim_inputs
        ctx.save_for_backward(x, feats, inv_norm, gamma_all, weight_all)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, feats, inv_norm, gamma_all, weight_all = ctx.saved_tensors
        nb = len(ctx.dim_inputs)
        grad_out = grad_out.reshape(x.shape[0], nb, -1).to(feats.dtype).contiguous()
        dx, dg, dw, db = ctx.extension.band_split_mixed_backward(grad_out, x, feats, inv_norm, gamma_all, weight_all,
                                                                 ctx.dim_inputs, True)
        return dx, dg, dw, db, None, None, None


class _FusedMaskEstimatorFinalPacked(torch.autograd.Function):
    """Final per-band Linear + GLU for all bands on the flat weight / bias buffers (this build's form of
    fr.py:1087-1133); both reference modes compute these values."""

    @staticmethod
    def forward(ctx, x, weight_all, bias_all, extension, dim_inputs):
        x = x.contiguous()
        out, pre = extension.mask_estimator_final_forward_packed(x, weight_all, bias_all, dim_inputs)
        ctx.extension, ctx.dim_inputs = extension, dim_inputs
        ctx.save_for_backward(x, pre, weight_all)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, pre, weight_all = ctx.saved_tensors
        grad_out = grad_out.reshape(x.shape[0], -1).to(x.dtype).contiguous()
        dx, db, dw = ctx.extension.mask_estimator_final_backward_packed(grad_out, x, pre, weight_all, ctx.dim_inputs)
        return dx, dw, db, None, None


class _FusedGroupedLinear(torch.autograd.Function):
    """``bands.grouped_linear`` on the kernels (fr.py:1029-1048); the backward runs on the grouped-linear
    backward kernels when the extension has them, else as batched GEMMs like the reference."""

    @staticmethod
    def forward(ctx, x, weight, bias, extension):
        g, i = x.shape[-2], x.shape[-1]
        x3 = x.reshape(-1, g, i)
        out = extension.grouped_linear_forward(x3, weight, bias)
        ctx.input_shape = tuple(x.shape)
        ctx.has_bias = bias is not None
        ctx.extension = extension
        ctx.save_for_backward(x3, weight)
        return out.reshape(*x.shape[:-2], g, weight.shape[1])

    @staticmethod
    def backward(ctx, grad_out):
        x3, weight = ctx.saved_tensors
        go = grad_out.reshape(x3.shape[0], x3.shape[1], weight.shape[1])
        if hasattr(ctx.extension, "grouped_linear_backward"):
            dx, dw, db = ctx.extension.grouped_linear_backward(go.to(x3.dtype), x3, weight, ctx.has_bias)
            return dx.reshape(ctx.input_shape), dw, db, None
        got = go.transpose(0, 1)  # [G, M, O]
        dx = torch.bmm(got, weight.contiguous()).transpose(0, 1).reshape(ctx.input_shape)
        dw = torch.bmm(got.transpose(1, 2).contiguous(), x3.transpose(0, 1).contiguous())
        db = go.sum(dim=0) if ctx.has_bias else None
        return dx, dw, db, None


class _MaskFinalGroupedLinearGLU(torch.autograd.Function):
    """Grouped final Linear + GLU with a hand-written backward (fr.py:1051-1084)."""

    @staticmethod
    def forward(ctx, x, weight, bias):
        g, o2, i = weight.shape
        lead = tuple(x.shape[:-2])
        x3 = x.reshape(-1, g, i)
        xt = x3.transpose(0, 1)
        wt = weight.transpose(1, 2).contiguous()
        pre = (torch.bmm(xt, wt) if bias is None else torch.baddbmm(bias.unsqueeze(1), xt, wt)).transpose(0, 1)
        left, gate_pre = pre.chunk(2, dim=-1)
        gate = gate_pre.sigmoid()
        ctx.input_shape = tuple(x.shape)
        ctx.has_bias = bias is not None
        ctx.save_for_backward(x3, weight, left, gate)
        return (left * gate).reshape(*lead, g, o2 // 2)

    @staticmethod
    def backward(ctx, grad_out):
        x3, weight, left, gate = ctx.saved_tensors
        grad = grad_out.reshape(x3.shape[0], x3.shape[1], weight.shape[1] // 2)
        dpre = torch.cat((grad * gate, grad * left * gate * (1 - gate)), dim=-1)
        dpt = dpre.to(weight.dtype).transpose(0, 1)  # [G, M, 2O]
        dx = torch.bmm(dpt, weight.contiguous()).transpose(0, 1).reshape(ctx.input_shape)
        dw = torch.bmm(dpre.to(x3.dtype).transpose(0, 1).transpose(1, 2).contiguous(), x3.transpose(0, 1).contiguous())
        db = dpre.sum(dim=0) if ctx.has_bias else None
        return dx.to(x3.dtype), dw.to(weight.dtype), (db.to(weight.dtype) if db is not None else None)


class _FusedMaskEstimatorFinal(torch.autograd.Function):
    """Ragged final Linear + GLU for all bands (fr.py:1087-1133)."""

    @staticmethod
    def forward(ctx, x, bias, dim_offsets, extension, dim_inputs, mode, *weights):
        ctx.extension = extension
        ctx.dim_inputs = dim_inputs
        ctx.input_shape = tuple(x.shape)
        ctx.mode = mode
        ctx.packed = hasattr(extension, "mask_estimator_final_forward_packed") and hasattr(
            extension, "mask_estimator_final_backward_packed"
        )
        if ctx.packed:
            x = x.contiguous()
            weight_all = torch.cat([w.reshape(-1) for w in weights])
            out, pre = extension.mask_estimator_final_forward_packed(x, weight_all, bias.contiguous(), dim_inputs)
            ctx.save_for_backward(x, pre, weight_all)
            return out
        fwd = extension.mask_estimator_final_direct_forward if mode == "direct" else extension.mask_estimator_final_forward
        out, pre, x_saved = fwd(x, list(weights), bias, list(dim_inputs), dim_offsets)
        ctx.save_for_backward(x_saved, pre, dim_offsets, *weights)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        grad_out = grad_out.reshape(grad_out.shape[0], -1).contiguous()
        if ctx.packed:
            x, pre, weight_all = ctx.saved_tensors
            dx, db, dw = ctx.extension.mask_estimator_final_backward_packed(grad_out, x, pre, weight_all, ctx.dim_inputs)
            h = x.shape[-1]
            dims = [int(d) for d in ctx.dim_inputs]
            dws = [v.view(2 * d, h) for v, d in zip(dw.split([2 * d * h for d in dims]), dims)]
            return (dx.reshape(ctx.input_shape), db, None, None, None, None, *dws)
        x, pre, dim_offsets, *weights = ctx.saved_tensors
        bwd = (
            ctx.extension.mask_estimator_final_direct_backward
            if ctx.mode == "direct"
            else ctx.extension.mask_estimator_final_backward
        )
        res = bwd(grad_out, x, pre, list(weights), list(ctx.dim_inputs), dim_offsets)
        return (res[0].reshape(ctx.input_shape), res[1], None, None, None, None, *res[2:])


def _one_pass_mask_mlp(ext, x, w1, dim_inputs) -> bool:
    """The depth-2 MLP forward runs as one kernel (16-bit, supported dim / hidden / widths)."""
    return (hasattr(ext, "mask_mlp_forward") and x.dtype in (torch.float16, torch.bfloat16)
            and ext.mask_mlp_supported(x.shape[-1], w1.shape[1], dim_inputs, x.dtype))


class _FusedMaskMLP(torch.autograd.Function):
    """Depth-2 mask MLP for all bands: hidden = tanh(x W1_b^T + b1_b), then the final per-band Linear +
    GLU, as one kernel in 16-bit (``mask_mlp_forward``; the hidden layer stays on chip unless the
    backward needs it) or as the grouped linear with a tanh epilogue followed by the final layer.
    The backward fuses tanh' = 1 - h^2 into the final layer's dx epilogue and runs the hidden
    layer's backward on the grouped-linear kernels.  Saves x, h and pre (the tensors the stock
    autograd graph keeps)."""

    @staticmethod
    def forward(ctx, x, w1, b1, w2, b2, extension, dim_inputs):
        if _one_pass_mask_mlp(extension, x, w1, dim_inputs):
            # one kernel; the hidden layer goes to HBM only when the backward needs it
            out, pre, h = extension.mask_mlp_forward(x, w1, b1, w2, b2, dim_inputs,
                                                     save_hidden=any(ctx.needs_input_grad[:5]))
        else:
            h = extension.grouped_linear_forward_act(x, w1, b1, activation="tanh")
            out, pre = extension.mask_estimator_final_forward_packed(h, w2, b2, dim_inputs)
        ctx.save_for_backward(x, w1, h, pre, w2)
        ctx.extension = extension
        ctx.dim_inputs = dim_inputs
        return out

    @staticmethod
    def backward(ctx, grad_out):
        x, w1, h, pre, w2 = ctx.saved_tensors
        ext = ctx.extension
        go = grad_out.reshape(pre.shape[0], -1).to(h.dtype).contiguous()
        dz, db2, dw2 = ext.mask_estimator_final_backward_packed(go, h, pre, w2, ctx.dim_inputs,
                                                                input_activation="tanh")
        dx, dw1, db1 = ext.grouped_linear_backward(dz, x, w1, has_bias=True)
        return dx, dw1, db1, dw2, db2, None, None


class _FusedMaskMLPApply(torch.autograd.Function):
    """The stems' depth-2 mask MLPs with the mask application in their epilogue: each stem's one-pass
    MLP kernel writes its slice of the masked spectrum in the iSTFT layout ``[B*S*C, F, T]``
    (``mask_mlp_forward_apply``) instead of a mask; the masks are never stored.  Backward: the mask
    gradients ``grad_est * conj(spec)`` of all stems in one pass (``mask_apply_grad_mask``), then each
    stem's MLP backward as in :class:`_FusedMaskMLP`.  ``spec`` must not need a gradient."""

    @staticmethod
    def forward(ctx, spec, x3, channels, zero_dc, dims, extension, *params):
        stems = len(params) // 4
        b, fc, t = spec.shape
        spec = spec.contiguous()
        est = torch.empty((b * stems * channels, fc // channels, t), dtype=torch.complex64, device=spec.device)
        saved = []
        for s in range(stems):
            w1, b1, w2, b2 = params[4 * s: 4 * s + 4]
            pre, h = extension.mask_mlp_forward_apply(x3, w1, b1, w2, b2, dims, spec, est, s, channels, zero_dc,
                                                      save_hidden=True)
            saved += [w1, h, pre, w2]
        ctx.save_for_backward(spec, x3, *saved)
        ctx.meta = (channels, zero_dc, dims, stems)
        ctx.extension = extension
        return est

    @staticmethod
    def backward(ctx, grad_est):
        spec, x3, *saved = ctx.saved_tensors
        channels, zero_dc, dims, stems = ctx.meta
        ext = ctx.extension
        dmask = ext.mask_apply_grad_mask(grad_est, spec, stems, channels, x3.dtype, zero_dc)  # [B, S, T, 2FC]
        m = x3.shape[0]
        dx, grads = None, []
        for s in range(stems):
            w1, h, pre, w2 = saved[4 * s: 4 * s + 4]
            go = dmask[:, s].reshape(m, -1).contiguous()
            dz, db2, dw2 = ext.mask_estimator_final_backward_packed(go, h, pre, w2, dims, input_activation="tanh")
            dxs, dw1, db1 = ext.grouped_linear_backward(dz, x3, w1, has_bias=True)
            dx = dxs if dx is None else dx + dxs
            grads += [dw1, db1, dw2, db2]
        return (None, dx, None, None, None, None, *grads)


def _fused_qkv_split_ok(ext: Any, qkv: torch.Tensor) -> bool:
    """The fused q/k/v split + rotary runs where the stock path would call the patched rotary."""
    _, transformer, _ = _core()
    return (
        getattr(transformer.apply_rotary_emb_fast, "_pymsst_fused_rotary", False)
        and hasattr(ext, "rotary_qkv_forward")
        and hasattr(ext, "rotary_qkv_backward")
        and qkv.device.type == "cuda"
        and qkv.dtype in _FLOAT_TYPES
        and qkv.dim() == 3
    )


class _FusedQKVRotary(torch.autograd.Function):
    """``qkv_to_bnhd`` + ``rotate_qk_fast_bnhd`` as one op (no reference counterpart: the reference
    rotates q and k through ``_FusedRotary``, fr.py:1154-1166, and leaves the split to torch).
    Forward writes q (rotated), k (rotated) and v in the layout attention reads; backward writes
    the qkv gradient directly, replacing the two inverse rotations and the stack of the split."""

    @staticmethod
    def forward(ctx, qkv, cos, sin, heads, extension, out_layout="bhnd"):
        q, k, v = extension.rotary_qkv_forward(qkv, heads, cos, sin, out_layout=out_layout)
        ctx.save_for_backward(cos, sin)
        ctx.extension = extension
        return q, k, v

    @staticmethod
    def backward(ctx, grad_q, grad_k, grad_v):
        cos, sin = ctx.saved_tensors
        ref = next(g for g in (grad_q, grad_k, grad_v) if g is not None)
        grads = [torch.zeros_like(ref) if g is None else g for g in (grad_q, grad_k, grad_v)]
        return ctx.extension.rotary_qkv_backward(*grads, cos, sin), None, None, None, None, None


class _FusedBandGather(torch.autograd.Function):
    """Mel band gather: ``spec[B, R, T, 2]`` -> band-split input ``[B, T, J, 2]`` (one HIP pass; the
    backward sums the selections of each row back onto it)."""

    @staticmethod
    def forward(ctx, spec, plan, extension):
        ctx.plan, ctx.extension, ctx.dtype = plan, extension, spec.dtype
        return extension.band_rows_gather(spec, plan)

    @staticmethod
    def backward(ctx, grad_out):
        if not ctx.needs_input_grad[0]:
            return None, None, None
        return ctx.extension.band_rows_scatter(grad_out, ctx.plan, mean=False, out_dtype=ctx.dtype), None, None


class _FusedMaskScatterMean(torch.autograd.Function):
    """Mel mask average: ``mask[B, stems, T, J*2]`` -> fp32 ``[B, stems, R, T, 2]``, each spectrum row
    the mean of the band values that cover it (one HIP pass each way)."""

    @staticmethod
    def forward(ctx, mask, plan, extension):
        b, stems, t = mask.shape[:3]
        ctx.plan, ctx.extension, ctx.shape, ctx.dtype = plan, extension, mask.shape, mask.dtype
        out = extension.band_rows_scatter(mask.reshape(b * stems, t, plan.num_sel, 2), plan, mean=True)
        return out.view(b, stems, plan.num_rows, t, 2)

    @staticmethod
    def backward(ctx, grad_out):
        b, stems, t = ctx.shape[:3]
        g = grad_out.reshape(b * stems, ctx.plan.num_rows, t, 2)
        grad = ctx.extension.band_rows_gather(g, ctx.plan, divide=True, out_dtype=ctx.dtype)
        return grad.reshape(ctx.shape), None, None


class _FusedMaskApply(torch.autograd.Function):
    """``spec[B, F*C, T]`` (complex64) times the masks ``mask[B, stems, T, F*C*2]`` in the iSTFT layout
    ``[B*stems*C, F, T]`` (one HIP pass each way; the mask gradient comes back in the mask's dtype
    like the stock float cast's backward)."""

    @staticmethod
    def forward(ctx, spec, mask, channels, zero_dc, extension):
        ctx.channels, ctx.zero_dc, ctx.extension = channels, zero_dc, extension
        ctx.save_for_backward(spec, mask)
        return extension.mask_apply_forward(spec, mask, channels, zero_dc)

    @staticmethod
    def backward(ctx, grad_est):
        spec, mask = ctx.saved_tensors
        grad_mask, grad_spec = ctx.extension.mask_apply_backward(
            grad_est, spec, mask, ctx.channels, ctx.zero_dc, need_spec_grad=ctx.needs_input_grad[0])
        return grad_spec, grad_mask if ctx.needs_input_grad[1] else None, None, None, None


class _FusedAttentionGate(torch.autograd.Function):
    """fr.py:1228-1262.  With an extension that reads ``[B,N,H,Dh]`` views in place
    (``attention_gate_forward_bnhd``), the transposed SDPA output is not copied, and the attn
    gradient comes back in the layout SDPA's backward reads without a copy: dense ``[B,N,H,Dh]`` for
    16-bit tensors (the flash kernels' layout), dense ``[B,H,N,Dh]`` otherwise."""

    @staticmethod
    def forward(ctx, attn, x, weight, bias, extension):
        heads, dim_head = attn.shape[-2], attn.shape[-1]
        x_2d = x.reshape(-1, x.shape[-1])
        bnhd = attn.dim() == 4 and hasattr(extension, "attention_gate_forward_bnhd")
        if bnhd:
            out, gate, saved_attn, saved_x = extension.attention_gate_forward_bnhd(attn, x_2d, weight, bias)
        else:
            out, gate, saved_attn, saved_x = extension.attention_gate_forward(
                attn.reshape(-1, heads, dim_head), x_2d, weight, bias
            )
        ctx.attn_shape = tuple(attn.shape)
        ctx.x_shape = tuple(x.shape)
        ctx.bnhd = bnhd
        ctx.save_for_backward(saved_attn, saved_x, weight, gate)
        ctx.extension = extension
        return out.reshape(*x.shape[:-1], heads * dim_head)

    @staticmethod
    def backward(ctx, grad_out):
        saved_attn, saved_x, weight, gate = ctx.saved_tensors
        rows = gate.shape[0]
        grad_out_2d = grad_out.reshape(rows, -1)
        if ctx.bnhd:
            layout = "bnhd" if gate.dtype in (torch.float16, torch.bfloat16) else "bhnd"
            grad_attn, grad_x, grad_weight, grad_bias = ctx.extension.attention_gate_backward_bnhd(
                grad_out_2d, saved_attn, saved_x, weight, gate, out_layout=layout
            )
        else:
            grad_attn, grad_x, grad_weight, grad_bias = ctx.extension.attention_gate_backward(
                grad_out_2d, saved_attn, saved_x, weight, gate
            )
        return grad_attn.reshape(ctx.attn_shape), grad_x.reshape(ctx.x_shape), grad_weight, grad_bias, None


class _FusedRotary(torch.autograd.Function):
    """fr.py:1154-1166; ``cos``/``sin`` are the ``[..., ::2]`` views (no copy is made)."""

    @staticmethod
    def forward(ctx, t, cos, sin, extension):
        if "bhnd" in getattr(extension, "rotary_out_layouts", ()):
            # same values, written where attention reads them: its transpose(1, 2) + contiguous
            # become free, and t itself (a view into the qkv projection) is read in place
            out = extension.rotary_forward(t, cos, sin, out_layout="bhnd")
        else:
            out = extension.rotary_forward(t, cos, sin)
        ctx.save_for_backward(cos, sin)
        ctx.extension = extension
        return out

    @staticmethod
    def backward(ctx, grad_out):
        cos, sin = ctx.saved_tensors
        return ctx.extension.rotary_backward(grad_out, cos, sin), None, None, None


def _lean_rms(ext) -> bool:
    return hasattr(ext, "rms_norm_forward_lean") and hasattr(ext, "rms_norm_backward_from_input")


class _FusedRMSNorm(torch.autograd.Function):
    """gamma in x's dtype (fr.py:1169-1182)."""

    @staticmethod
    def forward(ctx, x, gamma, extension):
        ctx.input_shape = tuple(x.shape)
        ctx.extension = extension
        ctx.lean = _lean_rms(extension)
        if ctx.lean:
            xc = x.contiguous()
            out, inv_norm = extension.rms_norm_forward_lean(xc, gamma)
            ctx.save_for_backward(xc, inv_norm, gamma)
        else:
            out, normed, inv_norm = extension.rms_norm_forward(x, gamma)
            ctx.save_for_backward(normed, inv_norm, gamma)
        return out.reshape_as(x)

    @staticmethod
    def backward(ctx, grad_out):
        saved, inv_norm, gamma = ctx.saved_tensors
        go = grad_out.reshape(ctx.input_shape).to(saved.dtype)
        if ctx.lean:
            dx, dgamma = ctx.extension.rms_norm_backward_from_input(go, saved, inv_norm, gamma)
        else:
            dx, dgamma = ctx.extension.rms_norm_backward(go, saved, inv_norm, gamma)
        return dx.reshape(ctx.input_shape), dgamma, None


class _FusedRMSNormFp32Gamma(torch.autograd.Function):
    """fp32 gamma, output in x's dtype (fr.py:1185-1203)."""

    @staticmethod
    def forward(ctx, x, gamma, extension):
        ctx.input_shape = tuple(x.shape)
        ctx.extension = extension
        ctx.lean = _lean_rms(extension)
        if ctx.lean:
            xc = x.contiguous()
            out, inv_norm = extension.rms_norm_forward_lean(xc, gamma)
            ctx.save_for_backward(xc, inv_norm, gamma)
        else:
            out, normed, inv_norm = extension.rms_norm_forward_fp32_gamma(x, gamma)
            ctx.save_for_backward(normed, inv_norm, gamma)
        return out.reshape_as(x)

    @staticmethod
    def backward(ctx, grad_out):
        saved, inv_norm, gamma = ctx.saved_tensors
        go = grad_out.reshape(ctx.input_shape).to(saved.dtype)
        if ctx.lean:
            dx, dgamma = ctx.extension.rms_norm_backward_from_input(go, saved, inv_norm, gamma)
        else:
            dx, dgamma = ctx.extension.rms_norm_backward_fp32_gamma(go, saved, inv_norm, gamma)
        return dx.reshape(ctx.input_shape), dgamma, None


class _FusedRMSNormMixed(torch.autograd.Function):
    """x in 16-bit, fp32 gamma, fp32 output (fr.py:1206-1225)."""

    @staticmethod
    def forward(ctx, x, gamma, extension):
        out, normed, inv_norm = extension.rms_norm_forward_mixed(x, gamma)
        ctx.input_shape = tuple(x.shape)
        ctx.save_for_backward(normed, inv_norm, gamma, x.new_empty(0))
        ctx.extension = extension
        return out.reshape(*x.shape[:-1], x.shape[-1])

    @staticmethod
    def backward(ctx, grad_out):
        normed, inv_norm, gamma, x_meta = ctx.saved_tensors
        dx, dgamma = ctx.extension.rms_norm_backward_mixed(
            grad_out.reshape(ctx.input_shape).float(), normed, inv_norm, gamma, x_meta
        )
        return dx.reshape(ctx.input_shape), dgamma, None


_CORE_PATCH_POINTS = (
    # (module in pymsst_amd.core, owner attribute or None, patched name, marker of the saved original)
    ("transformer", None, "apply_rotary_emb_fast", "_pymsst_original_apply_rotary"),
    ("transformer", "RMSNorm", "forward", "_pymsst_original_forward"),
    ("transformer", "Attention", "forward", "_pymsst_original_forward"),
    ("bands", None, "grouped_linear", "_pymsst_original_grouped_linear"),
    ("bands", "MaskEstimator", "_forward_layer_grouped_mlp", "_pymsst_original_forward_layer_grouped_mlp"),
    ("bands", "MaskEstimator", "_get_layer_group_params", "_pymsst_original_get_layer_group_params"),
    ("bands", "BandSplit", "_get_group_params", "_pymsst_original_get_group_params"),
    ("common", "RoformerRuntimeMixin", "_estimate_masks", "_pymsst_original_estimate_masks"),
    ("mel_band_roformer", "MelBandRoformer", "_band_features", "_pymsst_original_band_features"),
    ("mel_band_roformer", "MelBandRoformer", "_spectral_mask", "_pymsst_original_spectral_mask"),
    ("bs_roformer", "BSRoformer", "_masked_spectrum", "_pymsst_original_masked_spectrum"),
    ("bs_roformer", "BSRoformer", "_mask_core", "_pymsst_original_mask_core"),
)


def restore_stock_implementations(model: torch.nn.Module | None = None) -> None:
    """Undo every patch ``apply_roformer_fused_training_backend`` made (this build's addition;
    the reference has no inverse).  Module- and class-level patches are unwound to the
    stock functions; with ``model`` its BandSplit instances get their stock
    ``_forward_grouped`` back.  Used to run stock and fused models in one process."""
    from .core import bs_roformer, mel_band_roformer

    bands, transformer, common = _core()
    modules = {"bands": bands, "transformer": transformer, "common": common, "mel_band_roformer": mel_band_roformer,
               "bs_roformer": bs_roformer}
    for mod_name, owner_name, name, marker in _CORE_PATCH_POINTS:
        owner = modules[mod_name] if owner_name is None else getattr(modules[mod_name], owner_name)
        current = getattr(owner, name)
        while getattr(current, marker, None) is not None:
            current = getattr(current, marker)
        setattr(owner, name, current)
    if model is not None:
        for module in model.modules():
            if getattr(module, "_pymsst_fused_band_split", False):
                del module._forward_grouped
                for attr in ("_pymsst_original_forward_grouped", "_pymsst_fused_extension",
                             "_pymsst_fused_band_split_bwd_mode", "_pymsst_fused_band_split"):
                    module.__dict__.pop(attr, None)


def reference_band_split_group(x, gamma, weight, bias):
    """Math statement of one band group (fr.py:1265-1271): normalise, scale, per-group Linear.

    ``x[M,G,I]``, ``gamma[G,I]``, ``weight[G,O,I]``, ``bias[G,O] | None`` -> ``[M,G,O]``.
    """
    normed = F.normalize(x, dim=-1) * (x.shape[-1] ** 0.5) * gamma.unsqueeze(0)
    out = torch.bmm(normed.transpose(0, 1), weight.transpose(1, 2).contiguous()).transpose(0, 1)
    return out + bias.unsqueeze(0) if bias is not None else out


__all__ = [
    "FusedTrainingStatus",
    "FusedKernelUnavailable",
    "RUNTIME_PRESETS",
    "apply_roformer_fused_training_backend",
    "apply_runtime_preset",
    "load_fused_band_split_extension",
    "normalize_fused_kernel_backend",
    "normalize_fused_rms_norm_mode",
    "reference_band_split_group",
    "restore_stock_implementations",
]

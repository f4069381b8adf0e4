"""Synthetic workloads: the training configurations the fused path is measured on.

Each entry restates one configuration of the benchmark (model hyper-parameters,
batch shape, sample length, stems, loss) for the restated stock models in
``pymsst_amd.core``; inputs are seeded synthetic audio, never a dataset:

* ``bsr_tiny``  - BS-RoFormer dim 64, depth 1, 4 heads x 32, 1 stem; batch 2 of
  stereo 32768 samples; L1 on the complex spectrogram.
* ``bsr_train`` - BS-RoFormer dim 192, depth 6, 8 heads x 64, 4 stems; batch 4 of
  stereo 131584 samples (258 frames); multi-resolution STFT L1; AdamW 5e-4.
* ``bsr_large`` - BS-RoFormer dim 512, depth 12, 1 stem; batch 2 of stereo 485100
  samples (948 frames); L1; activation checkpointing per axial block.
* ``mbr_train`` - Mel-band RoFormer dim 192, depth 8, 8 heads x 64, 4 stems, 60 mel bands;
  batch 4 of stereo 352800 samples (690 frames); L1 (configs[3]; transformer depths 1 and
  mask-estimator depth 2 chosen as for the BS-RoFormer configs).
* ``mbr_tiny`` - Mel-band RoFormer dim 32, depth 1, 12 bands, 2 stems (tests).

Audio: every source is i.i.d. N(0, 0.1^2) clipped to [-1, 1], drawn from its own
``torch.Generator``; the mixture is the sum of the sources and the target their
stack ``[B, stems, C, L]`` (one stem: ``[B, 1, C, L]``).
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

from .core.bs_roformer import BSRoformer
from .core.mel_band_roformer import MelBandRoformer


@dataclass(frozen=True)
class TrainWorkload:
    name: str
    model: dict
    batch: int
    length: int
    stems: int
    lr: float = 5e-4
    amp_dtype: torch.dtype | None = torch.bfloat16
    extra: dict = field(default_factory=dict)
    family: str = "bsr"  # "bsr" (BS-RoFormer) or "mbr" (Mel-band RoFormer)

    def build_model(self, device=None, seed: int = 4) -> BSRoformer:
        torch.manual_seed(seed)
        model = (MelBandRoformer if self.family == "mbr" else BSRoformer)(**self.model)
        return model.to(device) if device is not None else model


WORKLOADS = {
    "bsr_tiny": TrainWorkload(
        name="bsr_tiny",
        model=dict(dim=64, depth=1, stereo=True, num_stems=1, time_transformer_depth=1, freq_transformer_depth=1,
                   heads=4, dim_head=32, mask_estimator_depth=2, mlp_expansion_factor=4, loss="spec_l1"),
        batch=2, length=32768, stems=1, amp_dtype=None, extra={"independent_target": True},
    ),
    "bsr_train": TrainWorkload(
        name="bsr_train",
        model=dict(dim=192, depth=6, stereo=True, num_stems=4, time_transformer_depth=1, freq_transformer_depth=1,
                   heads=8, dim_head=64, mask_estimator_depth=2, mlp_expansion_factor=4, loss="multi_stft"),
        batch=4, length=131584, stems=4,
    ),
    "bsr_large": TrainWorkload(
        name="bsr_large",
        model=dict(dim=512, depth=12, stereo=True, num_stems=1, time_transformer_depth=1, freq_transformer_depth=1,
                   heads=8, dim_head=64, mask_estimator_depth=2, mlp_expansion_factor=4, loss="l1",
                   checkpoint_blocks=True),
        batch=2, length=485100, stems=1,
    ),
    "mbr_train": TrainWorkload(
        name="mbr_train",
        model=dict(dim=192, depth=8, stereo=True, num_stems=4, time_transformer_depth=1, freq_transformer_depth=1,
                   heads=8, dim_head=64, num_bands=60, mask_estimator_depth=2, mlp_expansion_factor=4, loss="l1"),
        batch=4, length=352800, stems=4, family="mbr",
    ),
    "mbr_tiny": TrainWorkload(
        name="mbr_tiny",
        model=dict(dim=32, depth=1, stereo=True, num_stems=2, time_transformer_depth=1, freq_transformer_depth=1,
                   heads=2, dim_head=32, num_bands=12, mask_estimator_depth=2, mlp_expansion_factor=2, loss="l1"),
        batch=2, length=16384, stems=2, amp_dtype=None, family="mbr",
    ),
}


def noise_sources(batch: int, stems: int, channels: int, length: int, *, seed: int = 0, device=None):
    """``stems`` independent seeded sources -> ``(target[B, stems, C, L], mixture[B, C, L])``."""
    srcs = []
    for s in range(stems):
        g = torch.Generator().manual_seed(seed + s)
        srcs.append((torch.randn(batch, channels, length, generator=g) * 0.1).clamp_(-1.0, 1.0))
    target = torch.stack(srcs, dim=1)
    mixture = target.sum(dim=1)
    if device is not None:
        target, mixture = target.to(device), mixture.to(device)
    return target, mixture


def workload_batch(workload: TrainWorkload, *, seed: int = 0, device=None):
    """``(target, mixture)`` for one step.  With ``independent_target`` the mixture is drawn
    from ``seed`` and the target from ``seed + 1`` instead of being the sources' sum."""
    if workload.extra.get("independent_target"):
        mixture = noise_sources(workload.batch, 1, 2, workload.length, seed=seed)[1]
        target = noise_sources(workload.batch, workload.stems, 2, workload.length, seed=seed + 1)[0]
        if device is not None:
            target, mixture = target.to(device), mixture.to(device)
        return target, mixture
    return noise_sources(workload.batch, workload.stems, 2, workload.length, seed=seed, device=device)


def synthetic_batches(workload: TrainWorkload, steps: int, *, seed: int = 0, device=None, distinct: bool = True):
    """One ``(target, mixture)`` batch per step (seed ``seed + 1000 * step``); ``distinct=False``
    repeats the first batch."""
    first = None
    for step in range(steps):
        if first is None or distinct:
            batch = workload_batch(workload, seed=seed + 1000 * step, device=device)
            if first is None:
                first = batch
            yield batch
        else:
            yield first


__all__ = ["TrainWorkload", "WORKLOADS", "noise_sources", "synthetic_batches", "workload_batch"]

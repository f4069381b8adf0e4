"""Runtime mixin shared by the RoFormer models (pymss-core ``common.RoformerRuntimeMixin``).

``_estimate_masks`` stacks the active mask estimators' outputs on a new stem axis;
the reference replaces it with a single-stem shortcut (fused_roformer.py:299-318).
"""

from __future__ import annotations

import torch


class RoformerRuntimeMixin:
    def _active_mask_estimators(self):
        return list(self.mask_estimators)

    def _estimate_masks(self, x: torch.Tensor) -> torch.Tensor:
        """``x[B, T, NB, dim]`` -> ``[B, stems, T, F]``."""
        return torch.stack([est(x) for est in self._active_mask_estimators()], dim=1)

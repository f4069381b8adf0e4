"""Training losses of the reference's separation module, restated.

``align_prediction_and_target``, ``masked_loss`` and ``compute_loss`` follow
src/pymsst/training/losses.py:7-68 (same arguments, shapes and error messages):
the masked loss is the per-(stem, item) MSE whose values at or above the
``q`` quantile (computed on detached values, linear interpolation) are masked
out before the mean.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def align_prediction_and_target(prediction: torch.Tensor, target: torch.Tensor):
    """Drop a singleton stem axis on whichever side has it (losses.py:7-15)."""
    if prediction.ndim == 3 and target.ndim == 4 and target.shape[1] == 1:
        target = target[:, 0]
    elif prediction.ndim == 4 and target.ndim == 3 and prediction.shape[1] == 1:
        prediction = prediction[:, 0]
    if prediction.shape != target.shape:
        raise ValueError(f"prediction shape {tuple(prediction.shape)} does not match target shape {tuple(target.shape)}")
    return prediction, target


def masked_loss(prediction: torch.Tensor, target: torch.Tensor, *, q: float = 0.95, coarse: bool = True,
                original_shape_compat: bool = False) -> torch.Tensor:
    """losses.py:18-40."""
    if original_shape_compat:
        prediction, target = torch.broadcast_tensors(prediction, target)
    else:
        prediction, target = align_prediction_and_target(prediction, target)
    if prediction.ndim == 3:
        prediction, target = prediction[:, None], target[:, None]
    err = (prediction - target).pow(2) if original_shape_compat else F.mse_loss(prediction, target, reduction="none")
    if err.ndim >= 3:
        err = err.transpose(0, 1)  # stems first
    if coarse and err.ndim >= 2:
        err = err.mean(dim=tuple(range(max(1, err.ndim - 2), err.ndim)))
    err = err.reshape(err.shape[0], -1)
    cut = torch.quantile(err.detach(), q, interpolation="linear", dim=1, keepdim=True)
    return (err * (err < cut)).mean()


def compute_loss(prediction: torch.Tensor, target: torch.Tensor, *, loss_name: str, q: float = 0.95,
                 coarse: bool = True, original_shape_compat: bool = False) -> torch.Tensor:
    """losses.py:52-68: ``masked_loss`` / ``mse_loss`` / ``l1_loss``."""
    if loss_name == "masked_loss":
        return masked_loss(prediction, target, q=q, coarse=coarse, original_shape_compat=original_shape_compat)
    prediction, target = align_prediction_and_target(prediction, target)
    if loss_name == "mse_loss":
        return F.mse_loss(prediction, target)
    if loss_name == "l1_loss":
        return F.l1_loss(prediction, target)
    raise ValueError(f"unsupported loss: {loss_name}")


__all__ = ["align_prediction_and_target", "compute_loss", "masked_loss"]

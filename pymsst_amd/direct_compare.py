"""Seeded direct training loop, loss-curve CSV and loss-curve comparison.

The harness a user of the reference runs as ``pymsst compare-direct`` to show that
the fused backend trains like the stock modules:

* ``seed_everything`` - src/pymsst/validation/direct_compare.py:472-477;
* ``run_manual_steps`` - the behaviour of the manual loop of direct_compare.py:335-392:
  autocast, GradScaler (enabled for fp16 only; bf16 needs none), gradient
  accumulation, optional clipping; ``loss_record_steps`` - the steps it records
  (1, N and every ``interval``, direct_compare.py:407-408);
* ``write_loss_curve`` / ``read_loss_curve`` - the CSV of direct_compare.py:411-440
  (header ``event,global_step,epoch,batch_idx,loss,val_loss,val_sdr``) and
  comparison.py:244-251;
* ``compare_loss_curves`` / ``summarize_comparisons`` - comparison.py:83-126 and
  223-241 (mean and max absolute difference over the overlapping points).

``run_direct_loss_curve`` runs one seeded curve of a synthetic workload with the
stock modules (``implementation="stock"``) or with the fused HIP backend
(``"fused"``), in a fresh model built from the same seed.  The reference's
second implementation is the upstream training repository; here the stock
restated modules play that role.
"""

from __future__ import annotations

import csv
import json
import random
import sys
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Callable, Iterable

import numpy as np
import torch

LOSS_CURVE_FIELDS = ("event", "global_step", "epoch", "batch_idx", "loss", "val_loss", "val_sdr")


def seed_everything(seed: int) -> None:
    random.seed(seed)
    np.random.seed(seed)
    torch.manual_seed(seed)
    if torch.cuda.is_available():
        torch.cuda.manual_seed_all(seed)


def loss_record_steps(total_steps: int, interval: int) -> frozenset[int]:
    """The 1-based steps whose loss goes into the curve.

    ``interval`` 0 keeps none; otherwise the first step, the last step and every multiple of
    ``interval`` are kept (the recording rule of direct_compare.py:407-408)."""
    if interval < 0:
        raise ValueError(f"loss_record_interval cannot be negative (got {interval})")
    if interval == 0 or total_steps < 1:
        return frozenset()
    return frozenset(range(interval, total_steps + 1, interval)) | {1, total_steps}


def _optimizer_update(model: torch.nn.Module, optimizer: torch.optim.Optimizer, scaler, grad_clip: float) -> None:
    """One parameter update from the accumulated (possibly scaled) gradients: unscale, clip, step."""
    scaler.unscale_(optimizer)
    if grad_clip:
        torch.nn.utils.clip_grad_norm_(model.parameters(), grad_clip)
    scaler.step(optimizer)  # skipped by the scaler when an fp16 gradient overflowed
    scaler.update()
    optimizer.zero_grad(set_to_none=True)


def run_manual_steps(
    *,
    model: torch.nn.Module,
    batches: Iterable,
    optimizer: torch.optim.Optimizer,
    device: torch.device,
    steps: int,
    loss_fn: Callable[[torch.nn.Module, torch.Tensor, torch.Tensor], torch.Tensor],
    amp_dtype: torch.dtype | None = None,
    grad_accum: int = 1,
    grad_clip: float = 0.0,
    loss_record_interval: int = 1,
) -> list[tuple[int, float]]:
    """Train ``steps`` steps on ``(target, mixture)`` pairs from ``batches`` and return the recorded
    ``[(step, loss)]``.

    Behaviour of the reference's manual loop (direct_compare.py:335-392): the forward runs under
    autocast in ``amp_dtype`` on a GPU (none on the CPU or with ``amp_dtype=None``); fp16 losses are
    scaled by a GradScaler (bf16 and fp32 need none); gradients of ``grad_accum`` consecutive steps are
    summed (each loss divided by ``grad_accum``) before one optimizer update, and the last step always
    updates; ``grad_clip`` > 0 clips the global gradient norm of the unscaled gradients; the recorded
    loss is the unscaled, undivided one.  Fewer batches than ``steps`` is an error.
    """
    if grad_accum < 1:
        raise ValueError(f"grad_accum must be a positive step count (got {grad_accum})")
    record = loss_record_steps(steps, loss_record_interval)
    autocast_on = amp_dtype is not None and device.type == "cuda"
    scaler = torch.amp.GradScaler(device.type, enabled=autocast_on and amp_dtype == torch.float16)
    source = iter(batches)
    curve: list[tuple[int, float]] = []
    optimizer.zero_grad(set_to_none=True)
    for step in range(1, steps + 1):
        batch = next(source, None)
        if batch is None:
            raise RuntimeError(f"the batch source ran out after {step - 1} of {steps} steps")
        target, mixture = (t.to(device, non_blocking=True) for t in batch)
        with torch.autocast(device_type=device.type, dtype=amp_dtype or torch.bfloat16, enabled=autocast_on):
            loss = loss_fn(model, mixture, target)
        if step in record:
            curve.append((step, float(loss.detach().cpu())))
        scaler.scale(loss / grad_accum).backward()
        if step % grad_accum == 0 or step == steps:
            _optimizer_update(model, optimizer, scaler, grad_clip)
    return curve


def write_loss_curve(path: str | Path, losses: list[tuple[int, float]]) -> Path:
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    with path.open("w", newline="", encoding="utf-8") as handle:
        writer = csv.DictWriter(handle, fieldnames=LOSS_CURVE_FIELDS)
        writer.writeheader()
        for step, loss in losses:
            writer.writerow({"event": "train", "global_step": step, "epoch": 0, "batch_idx": step - 1, "loss": loss,
                             "val_loss": "", "val_sdr": ""})
    return path


def read_loss_curve(path: str | Path) -> list[float]:
    """Losses of the ``train`` rows, in file order (comparison.py:244-251)."""
    out = []
    with Path(path).open(newline="", encoding="utf-8") as handle:
        for row in csv.DictReader(handle):
            if row.get("event") == "train" and row.get("loss"):
                out.append(float(row["loss"]))
    return out


@dataclass(frozen=True)
class CurveComparison:
    pymsst_points: int
    original_points: int
    compared_points: int
    mean_abs_diff: float
    max_abs_diff: float
    first_pymsst_loss: float
    first_original_loss: float
    last_pymsst_loss: float
    last_original_loss: float


def compare_loss_curves(fused_curve: str | Path, stock_curve: str | Path) -> CurveComparison:
    a, b = read_loss_curve(fused_curve), read_loss_curve(stock_curve)
    n = min(len(a), len(b))
    if n == 0:
        raise ValueError("no overlapping loss points to compare")
    diffs = [abs(a[i] - b[i]) for i in range(n)]
    return CurveComparison(len(a), len(b), n, sum(diffs) / n, max(diffs), a[0], b[0], a[n - 1], b[n - 1])


def summarize_comparisons(paths, *, min_points=None, max_mean_abs_diff=None, max_max_abs_diff=None) -> dict:
    """Aggregate saved ``CurveComparison`` JSON files against thresholds (comparison.py:83-126)."""
    if not paths:
        raise ValueError("at least one comparison path is required")
    records = []
    for p in paths:
        data = json.loads(Path(p).read_text(encoding="utf-8"))
        fails = []
        if min_points is not None and data["compared_points"] < min_points:
            fails.append(f"compared_points {data['compared_points']} < {min_points}")
        if max_mean_abs_diff is not None and data["mean_abs_diff"] > max_mean_abs_diff:
            fails.append(f"mean_abs_diff {data['mean_abs_diff']} > {max_mean_abs_diff}")
        if max_max_abs_diff is not None and data["max_abs_diff"] > max_max_abs_diff:
            fails.append(f"max_abs_diff {data['max_abs_diff']} > {max_max_abs_diff}")
        records.append({"path": str(p), **{k: data[k] for k in ("compared_points", "mean_abs_diff", "max_abs_diff")},
                        "failures": fails})
    failures = [{"path": r["path"], "failures": r["failures"]} for r in records if r["failures"]]
    return {
        "schema_version": 1,
        "thresholds": {"min_points": min_points, "max_mean_abs_diff": max_mean_abs_diff,
                       "max_max_abs_diff": max_max_abs_diff},
        "aggregate": {
            "count": len(records),
            "min_compared_points": min(r["compared_points"] for r in records),
            "max_mean_abs_diff": max(r["mean_abs_diff"] for r in records),
            "max_max_abs_diff": max(r["max_abs_diff"] for r in records),
            "passed": not failures,
        },
        "comparisons": records,
        "failures": failures,
    }


def model_loss(model, mixture, target):
    """The restated models return their training loss when given the target."""
    return model(mixture, target)


def run_direct_loss_curve(
    *,
    implementation: str,
    workload,
    steps: int,
    results_path: str | Path | None = None,
    seed: int = 0,
    device: torch.device | str = "cuda:0",
    amp_dtype: torch.dtype | None | str = "workload",
    preset: str = "hip_full",
    rms_norm_mode: str | None = "fast",
    distinct_batches: bool = True,
    loss_record_interval: int = 1,
    lr: float | None = None,
) -> dict:
    """One seeded loss curve of ``workload`` (a ``workloads.TrainWorkload``)."""
    from . import fused_roformer as fr
    from .workloads import synthetic_batches

    if implementation not in ("stock", "fused"):
        raise ValueError("implementation must be 'stock' or 'fused'")
    device = torch.device(device)
    amp = workload.amp_dtype if amp_dtype == "workload" else amp_dtype
    seed_everything(seed)
    model = workload.build_model(device, seed=seed + 4)
    model.train()
    status = None
    fr.restore_stock_implementations(model)
    if implementation == "fused":
        fr.apply_runtime_preset(preset)
        status = fr.apply_roformer_fused_training_backend(model, "hip", rms_norm_mode=rms_norm_mode)
        if status.active == "off":
            raise RuntimeError(f"fused backend inactive: {status.reason}")
    try:
        optimizer = torch.optim.AdamW(model.parameters(), lr=workload.lr if lr is None else lr)
        losses = run_manual_steps(
            model=model, batches=synthetic_batches(workload, steps, seed=seed, device=device, distinct=distinct_batches),
            optimizer=optimizer, device=device, steps=steps, loss_fn=model_loss, amp_dtype=amp,
            loss_record_interval=loss_record_interval,
        )
    finally:
        fr.restore_stock_implementations(model)
    meta = {
        "schema_version": 1,
        "implementation": implementation,
        "workload": workload.name,
        "seed": seed,
        "steps": steps,
        "amp_dtype": str(amp) if amp is not None else None,
        "fused_status": asdict(status) if status is not None else None,
        "losses": losses,
        "environment": {
            "python": sys.version.split()[0],
            "torch": torch.__version__,
            "hip": torch.version.hip,
            "device_name": torch.cuda.get_device_name(device) if device.type == "cuda" else None,
        },
    }
    if results_path is not None:
        results_path = Path(results_path)
        meta["loss_curve_path"] = str(write_loss_curve(results_path / "loss_curve.csv", losses))
        (results_path / "run_metadata.json").write_text(json.dumps(meta, indent=2, default=str), encoding="utf-8")
    return meta


__all__ = [
    "CurveComparison",
    "LOSS_CURVE_FIELDS",
    "compare_loss_curves",
    "model_loss",
    "read_loss_curve",
    "run_direct_loss_curve",
    "run_manual_steps",
    "seed_everything",
    "loss_record_steps",
    "summarize_comparisons",
    "write_loss_curve",
]

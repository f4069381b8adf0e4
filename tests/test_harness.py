"""CPU tests of the training harness: loss-curve CSV, curve comparison, threshold summary,
the seeded manual loop and the model's waveform loss (mirroring the reference's
tests/test_comparison.py:127-222)."""

from __future__ import annotations

import csv
import json
import warnings

import pytest
import torch
from pytest import approx

from pymsst_amd import direct_compare as dc
from pymsst_amd.workloads import TrainWorkload, noise_sources, synthetic_batches, workload_batch


def _write_csv(path, rows):
    with path.open("w", newline="", encoding="utf-8") as handle:
        writer = csv.DictWriter(handle, fieldnames=dc.LOSS_CURVE_FIELDS)
        writer.writeheader()
        for row in rows:
            writer.writerow(row)


def test_read_loss_curve_keeps_train_rows_only(tmp_path):
    path = tmp_path / "loss_curve.csv"
    _write_csv(path, [
        {"event": "train", "global_step": 1, "epoch": 0, "batch_idx": 0, "loss": 0.5},
        {"event": "validation", "global_step": 1, "epoch": 0, "batch_idx": "", "loss": "", "val_loss": 0.4},
        {"event": "train", "global_step": 2, "epoch": 0, "batch_idx": 1, "loss": 0.25},
    ])
    assert dc.read_loss_curve(path) == [0.5, 0.25]


def test_compare_loss_curves_known_answer(tmp_path):
    a, b = tmp_path / "a.csv", tmp_path / "b.csv"
    dc.write_loss_curve(a, [(1, 1.0), (2, 2.0)])
    dc.write_loss_curve(b, [(1, 1.25), (2, 1.75), (3, 9.0)])
    res = dc.compare_loss_curves(a, b)
    assert res.compared_points == 2 and res.pymsst_points == 2 and res.original_points == 3
    assert res.mean_abs_diff == approx(0.25)
    assert res.max_abs_diff == approx(0.25)
    assert (res.first_pymsst_loss, res.last_original_loss) == (1.0, 1.75)
    assert json.loads(json.dumps(res.__dict__))["compared_points"] == 2
    empty = tmp_path / "empty.csv"
    dc.write_loss_curve(empty, [])
    with pytest.raises(ValueError, match="no overlapping"):
        dc.compare_loss_curves(a, empty)


def test_write_loss_curve_header_and_rows(tmp_path):
    path = dc.write_loss_curve(tmp_path / "x" / "loss_curve.csv", [(1, 0.5), (3, 0.25)])
    lines = path.read_text().splitlines()
    assert lines[0] == "event,global_step,epoch,batch_idx,loss,val_loss,val_sdr"
    assert lines[1] == "train,1,0,0,0.5,,"
    assert lines[2] == "train,3,0,2,0.25,,"


def test_summarize_comparisons_thresholds(tmp_path):
    paths = []
    for name, mean_d, max_d in (("first", 0.1, 0.2), ("second", 0.05, 0.15)):
        p = tmp_path / f"{name}.json"
        p.write_text(json.dumps({"pymsst_points": 1000, "original_points": 1000, "compared_points": 1000,
                                 "mean_abs_diff": mean_d, "max_abs_diff": max_d}))
        paths.append(p)
    ok = dc.summarize_comparisons(paths, min_points=1000, max_mean_abs_diff=0.1, max_max_abs_diff=0.2)
    bad = dc.summarize_comparisons(paths, min_points=1001, max_mean_abs_diff=0.09, max_max_abs_diff=0.19)
    assert ok["aggregate"]["passed"] is True and ok["aggregate"]["count"] == 2
    assert ok["aggregate"]["max_mean_abs_diff"] == approx(0.1)
    assert ok["aggregate"]["max_max_abs_diff"] == approx(0.2)
    assert bad["aggregate"]["passed"] is False and len(bad["failures"]) == 2
    with pytest.raises(ValueError):
        dc.summarize_comparisons([])


def test_loss_record_steps():
    assert sorted(dc.loss_record_steps(10, 4)) == [1, 4, 8, 10]
    assert sorted(dc.loss_record_steps(10, 1)) == list(range(1, 11))
    assert sorted(dc.loss_record_steps(3, 5)) == [1, 3]
    assert dc.loss_record_steps(10, 0) == frozenset()
    with pytest.raises(ValueError):
        dc.loss_record_steps(10, -1)


def test_one_stem_waveform_loss_is_per_item():
    """One stem: recon is [B, C, L] and the stacked target [B, 1, C, L]; the L1 compares each item with
    its own target (no broadcast over [B, B, C, L]); the multi-resolution term likewise."""
    import torch.nn.functional as F

    from pymsst_amd.workloads import WORKLOADS

    torch.manual_seed(0)
    for loss in ("l1", "multi_stft"):
        model = WORKLOADS["bsr_tiny"].build_model(None, seed=4)
        model.loss_type = loss
        recon = torch.randn(2, 2, 4096)
        target = torch.randn(2, 1, 2, 4096)
        with warnings.catch_warnings():
            warnings.simplefilter("error")  # torch warns when l1_loss broadcasts mismatched sizes
            got = model.loss(recon, target)
            ref = model.loss(recon, target[:, 0])
        assert got.item() == approx(ref.item(), rel=1e-6)
        if loss == "l1":
            assert got.item() == approx(F.l1_loss(recon, target[:, 0]).item(), rel=1e-6)


def test_noise_sources_law_and_seeding():
    target, mixture = noise_sources(2, 4, 2, 4096, seed=0)
    assert target.shape == (2, 4, 2, 4096) and mixture.shape == (2, 2, 4096)
    assert torch.allclose(mixture, target.sum(1))
    assert target.abs().max() <= 1.0
    assert abs(target.std().item() - 0.1) < 0.005
    again, _ = noise_sources(2, 4, 2, 4096, seed=0)
    assert torch.equal(target, again)
    assert not torch.equal(target[:, 0], target[:, 1])


_TINY = TrainWorkload(
    name="cpu_tiny",
    model=dict(dim=16, depth=1, stereo=True, num_stems=1, time_transformer_depth=1, freq_transformer_depth=1,
               heads=2, dim_head=8, mask_estimator_depth=2, mlp_expansion_factor=2, loss="spec_l1",
               stft_n_fft=256, stft_hop_length=64, stft_win_length=256,
               freqs_per_bands=(2,) * 16 + (4,) * 8 + (32,) + (33,)),
    batch=1, length=2048, stems=1, amp_dtype=None, extra={"independent_target": True},
)


def test_independent_target_batches():
    target, mixture = workload_batch(_TINY, seed=3)
    assert target.shape == (1, 1, 2, 2048) and mixture.shape == (1, 2, 2048)
    assert not torch.allclose(target[:, 0], mixture)
    batches = list(synthetic_batches(_TINY, 3, seed=3, distinct=False))
    assert all(torch.equal(b[1], batches[0][1]) for b in batches)
    batches = list(synthetic_batches(_TINY, 2, seed=3))
    assert not torch.equal(batches[0][1], batches[1][1])


def test_manual_loop_is_seeded_and_deterministic_on_cpu():
    def run():
        dc.seed_everything(0)
        model = _TINY.build_model(seed=4)
        opt = torch.optim.AdamW(model.parameters(), lr=1e-3)
        return dc.run_manual_steps(model=model, batches=synthetic_batches(_TINY, 3, seed=0), optimizer=opt,
                                   device=torch.device("cpu"), steps=3, loss_fn=dc.model_loss)

    first, second = run(), run()
    assert [s for s, _ in first] == [1, 2, 3]
    assert first == second
    assert all(torch.isfinite(torch.tensor(v)) for _, v in first)


def test_manual_loop_accumulates_and_checks_batches():
    """grad_accum 2 over 3 steps updates after steps 2 and 3 (the last step always updates); each loss is
    recorded undivided; a batch source shorter than ``steps`` is an error."""
    updates = []

    class CountingSGD(torch.optim.SGD):
        def step(self, closure=None):
            updates.append([p.grad.clone() for p in self.param_groups[0]["params"] if p.grad is not None])
            return super().step(closure)

    torch.manual_seed(0)
    lin = torch.nn.Linear(3, 1)
    batches = [(torch.randn(2, 1), torch.randn(2, 3)) for _ in range(3)]

    def loss_fn(model, mixture, target):
        return ((model(mixture) - target) ** 2).mean()

    ref = torch.nn.Linear(3, 1)
    ref.load_state_dict(lin.state_dict())
    curve = dc.run_manual_steps(model=lin, batches=batches, optimizer=CountingSGD(lin.parameters(), lr=0.1),
                                device=torch.device("cpu"), steps=3, loss_fn=loss_fn, grad_accum=2)
    assert len(updates) == 2
    # the first update's gradient is the mean of the two steps' gradients at the initial weights
    g = [torch.zeros_like(p) for p in ref.parameters()]
    for target, mixture in batches[:2]:
        ref.zero_grad()
        (loss_fn(ref, mixture, target) / 2).backward()
        g = [a + p.grad for a, p in zip(g, ref.parameters())]
    assert all(torch.allclose(a, b) for a, b in zip(updates[0], g))
    assert [s for s, _ in curve] == [1, 2, 3]
    assert curve[0][1] == approx(loss_fn(ref, batches[0][1], batches[0][0]).item(), rel=1e-6)
    with pytest.raises(RuntimeError, match="ran out after 3 of 4"):
        dc.run_manual_steps(model=lin, batches=batches, optimizer=torch.optim.SGD(lin.parameters(), lr=0.1),
                            device=torch.device("cpu"), steps=4, loss_fn=loss_fn)
    with pytest.raises(ValueError):
        dc.run_manual_steps(model=lin, batches=batches, optimizer=torch.optim.SGD(lin.parameters(), lr=0.1),
                            device=torch.device("cpu"), steps=3, loss_fn=loss_fn, grad_accum=0)

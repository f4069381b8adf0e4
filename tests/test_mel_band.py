"""CPU tests of the Mel-band RoFormer restatement: the mel band layout (pinned against figures
computed independently of this code from the mel scale: 60 bands at 44.1 kHz / n_fft 2048 give 6 to 130 bins per band,
1979 (bin, band) pairs, 38 distinct widths, every bin in one or two bands), the model's stock
gather / average against the oracle, and the fused autograd Functions through a CPU stand-in of the
extension computing with the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pymsst_amd import fused_roformer as fr
from pymsst_amd.core.mel_band_roformer import MelBandRoformer, mel_band_bins, mel_filterbank


def test_mel_band_layout_matches_independent_figures():
    bins = mel_band_bins(44100, 2048, 60)
    widths = [b.size for b in bins]
    assert len(bins) == 60 and min(widths) == 6 and max(widths) == 130
    assert sum(widths) == 1979 and len(set(widths)) == 38
    cover = np.zeros(1025, dtype=int)
    for b in bins:
        cover[b] += 1
        assert np.all(np.diff(b) == 1), "a band is a contiguous run of bins"
    assert cover.min() == 1 and cover.max() == 2
    assert bins[0][0] == 0 and bins[-1][-1] == 1024


def test_mel_filterbank_shape_and_peaks():
    fb = mel_filterbank(44100, 2048, 60)
    assert fb.shape == (60, 1025) and (fb >= 0).all()
    peaks = fb.argmax(axis=1)
    assert np.all(np.diff(peaks) >= 0), "filters are ordered by frequency"


def _tiny(**kw):
    torch.manual_seed(0)
    return MelBandRoformer(16, depth=1, stereo=True, num_stems=2, heads=2, dim_head=8, num_bands=12,
                           mask_estimator_depth=2, mlp_expansion_factor=2, loss="l1", **kw)


def test_stock_gather_and_average_match_oracle():
    m = _tiny()
    spec = torch.randn(2, m.num_rows, 7, dtype=torch.complex64)
    x = m._band_features(spec)
    ref = oracle.band_rows_gather(torch.view_as_real(spec).numpy(), m.band_rows.numpy())
    assert np.allclose(x.numpy(), ref.reshape(2, 7, -1))
    mask = torch.randn(2, 2, 7, 2 * m.band_rows.numel())
    avg = torch.view_as_real(m._spectral_mask(mask))
    r = oracle.band_rows_scatter(mask.reshape(4, 7, -1, 2).numpy(), m.band_rows.numpy(), m.num_rows)
    assert np.allclose(avg.reshape(4, m.num_rows, 7, 2).numpy(), r, atol=1e-6)


class _OracleRowsExt:
    """CPU stand-in with the band-row op names, computing through the numpy oracle."""

    band_rows_plan = staticmethod(lambda rows, num_rows, device: fr_plan(rows, num_rows))

    def band_rows_gather(self, x, plan, divide=False, out_dtype=None):
        div = plan.divisor.numpy() if divide else None
        out = oracle.band_rows_gather(x.detach().double().numpy(), plan.rows.numpy(), div)
        return torch.from_numpy(out).to(out_dtype or x.dtype)

    def band_rows_scatter(self, x, plan, mean=True, out_dtype=torch.float32):
        out = oracle.band_rows_scatter(x.detach().double().numpy(), plan.rows.numpy(), plan.num_rows, mean)
        return torch.from_numpy(out).to(out_dtype)


def fr_plan(rows, num_rows):
    from pymsst_amd.extension import HipFusedExtension

    return HipFusedExtension.band_rows_plan(rows, num_rows, "cpu")


def test_fused_mel_functions_match_stock_autograd():
    m = _tiny()
    ext = _OracleRowsExt()
    plan = fr_plan(m.band_rows, m.num_rows)
    spec = torch.randn(2, m.num_rows, 6, dtype=torch.complex64)
    got = fr._FusedBandGather.apply(torch.view_as_real(spec), plan, ext).reshape(2, 6, -1)
    assert torch.allclose(got, m._band_features(spec))
    mask = torch.randn(2, 2, 6, 2 * plan.num_sel, dtype=torch.float64, requires_grad=True)
    out = fr._FusedMaskScatterMean.apply(mask, plan, ext)
    ref = torch.view_as_real(MelBandRoformer._spectral_mask(m, mask))
    assert torch.allclose(out, ref.to(out.dtype), atol=1e-6)
    g = torch.randn(out.shape, dtype=out.dtype)
    (gm,) = torch.autograd.grad(out, mask, g)
    (gr,) = torch.autograd.grad(ref, mask, g.to(ref.dtype))
    assert torch.allclose(gm.double(), gr.double(), atol=1e-6)


def test_mel_patch_and_restore(monkeypatch):
    orig = (MelBandRoformer._band_features, MelBandRoformer._spectral_mask)
    monkeypatch.setenv(fr.EXPERIMENTAL_FUSED_MEL_BANDS_ENV, "1")
    monkeypatch.setenv(fr.CORE_GROUPED_TRAIN_ENV, "")
    status = fr.apply_roformer_fused_training_backend(_tiny(), "hip", extension=_OracleRowsExt())
    assert status.patched_mel_bands
    assert getattr(MelBandRoformer._band_features, "_pymsst_fused_mel_bands", False)
    fr.restore_stock_implementations()
    assert (MelBandRoformer._band_features, MelBandRoformer._spectral_mask) == orig


def test_model_forward_and_loss_shapes():
    m = _tiny()
    audio = torch.randn(1, 2, 4096) * 0.1
    assert m(audio).shape == (1, 2, 2, 4096)
    loss = m(audio, torch.randn(1, 2, 2, 4096) * 0.1)
    loss.backward()
    assert torch.isfinite(loss)

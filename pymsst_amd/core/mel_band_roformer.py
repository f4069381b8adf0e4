"""Mel-band RoFormer for music source separation, stock PyTorch.

Restated from the public Mel-band RoFormer architecture on top of the BS-RoFormer
restatement in ``bs_roformer.py`` (same axial transformer, band split and mask
estimators).  pymss-core's mel code is not available, so the band layout follows the
public model:

* ``num_bands`` triangular mel filters (Slaney mel scale and area normalisation, the
  librosa defaults) over the ``n_fft // 2 + 1`` STFT bins; band ``b`` owns every bin
  where its filter is positive, with the first bin of the first band and the last bin
  of the last band forced on.  Adjacent bands overlap, so a bin belongs to one or two
  bands.  At 44.1 kHz, ``n_fft`` 2048 and 60 bands: 6 to 130 bins per band, 1979
  (bin, band) pairs, 38 distinct widths.
* Band features: the rows ``f * C + c`` (frequency-major, channel inner, as the STFT
  is packed) of each band's bins are gathered in band order, each row giving its real
  and imaginary parts, so band ``b`` owns ``2 * C * bins_b`` consecutive features.
* Masks: the estimators emit one complex value per gathered row; values of a bin that
  several bands cover are summed and divided by the number of bands covering it
  (scatter-add average) before multiplying the spectrum.

The gather and the scatter average are the methods ``_band_features`` and
``_spectral_mask``, which the fused backend replaces.
"""

from __future__ import annotations

import numpy as np
import torch

from .bs_roformer import BSRoformer

_F_SP = 200.0 / 3.0
_MIN_LOG_HZ = 1000.0
_MIN_LOG_MEL = _MIN_LOG_HZ / _F_SP
_LOGSTEP = float(np.log(6.4) / 27.0)


def hz_to_mel(f):
    """Slaney mel scale: linear below 1 kHz, logarithmic above."""
    f = np.asarray(f, dtype=np.float64)
    return np.where(f >= _MIN_LOG_HZ, _MIN_LOG_MEL + np.log(np.maximum(f, 1e-10) / _MIN_LOG_HZ) / _LOGSTEP, f / _F_SP)


def mel_to_hz(m):
    m = np.asarray(m, dtype=np.float64)
    return np.where(m >= _MIN_LOG_MEL, _MIN_LOG_HZ * np.exp(_LOGSTEP * (m - _MIN_LOG_MEL)), _F_SP * m)


def mel_filterbank(sample_rate: int, n_fft: int, num_bands: int) -> np.ndarray:
    """``[num_bands, n_fft // 2 + 1]`` triangular filters on the Slaney mel scale between 0 Hz and
    Nyquist, each scaled by 2 / (its band width in Hz)."""
    freqs = np.linspace(0.0, sample_rate / 2.0, 1 + n_fft // 2)
    edges = mel_to_hz(np.linspace(hz_to_mel(0.0), hz_to_mel(sample_rate / 2.0), num_bands + 2))
    widths = np.diff(edges)
    ramps = edges[:, None] - freqs[None, :]
    fb = np.zeros((num_bands, freqs.size))
    for i in range(num_bands):
        rising = -ramps[i] / widths[i]
        falling = ramps[i + 2] / widths[i + 1]
        fb[i] = np.maximum(0.0, np.minimum(rising, falling))
    return fb * (2.0 / (edges[2 : num_bands + 2] - edges[:num_bands]))[:, None]


def mel_band_bins(sample_rate: int, n_fft: int, num_bands: int) -> list[np.ndarray]:
    """Bins of each band (ascending), first and last bin forced on; every bin is covered."""
    owned = mel_filterbank(sample_rate, n_fft, num_bands) > 0
    owned[0, 0] = True
    owned[-1, -1] = True
    if not owned.any(axis=0).all():
        raise ValueError("mel bands leave some frequency bins uncovered")
    return [np.nonzero(row)[0] for row in owned]


class MelBandRoformer(BSRoformer):
    """BS-RoFormer with overlapping mel bands (see the module docstring)."""

    def __init__(self, dim: int, *, num_bands: int = 60, sample_rate: int = 44100, stft_n_fft: int = 2048,
                 stereo: bool = False, **kwargs):
        if "freqs_per_bands" in kwargs:
            raise TypeError("MelBandRoformer derives its bands from num_bands")
        channels = 2 if stereo else 1
        bins = mel_band_bins(sample_rate, stft_n_fft, num_bands)
        self.mel_band_widths = tuple(int(b.size) for b in bins)
        # BSRoformer builds band split / mask estimators from freqs_per_bands; give it widths in
        # bins whose feature counts (2 * C * bins) are those of the mel bands
        super().__init__(dim, stereo=stereo, stft_n_fft=stft_n_fft, freqs_per_bands=self.mel_band_widths,
                         _check_cover=False, **kwargs)
        rows = np.concatenate([(b[:, None] * channels + np.arange(channels)[None, :]).reshape(-1) for b in bins])
        n_freqs = stft_n_fft // 2 + 1
        counts = np.zeros(n_freqs * channels, dtype=np.int64)
        np.add.at(counts, rows, 1)
        self.register_buffer("band_rows", torch.from_numpy(rows.astype(np.int64)), persistent=False)
        self.register_buffer("bands_per_row", torch.from_numpy(counts), persistent=False)
        self.num_rows = n_freqs * channels

    def _band_features(self, spec: torch.Tensor) -> torch.Tensor:
        """Gather the band rows of ``spec[B, F*C, T]`` -> ``[B, T, rows*2]``."""
        b, _, t = spec.shape
        gathered = spec.index_select(1, self.band_rows)  # [B, rows, T]
        return torch.view_as_real(gathered).permute(0, 2, 1, 3).reshape(b, t, -1)

    def _spectral_mask(self, mask: torch.Tensor) -> torch.Tensor:
        """``[B, stems, T, rows*2]`` -> averaged complex mask ``[B, stems, F*C, T]``."""
        b, stems, t = mask.shape[:3]
        vals = mask.float().reshape(b, stems, t, -1, 2).permute(0, 1, 3, 2, 4)  # [B, S, rows, T, 2]
        idx = self.band_rows.view(1, 1, -1, 1, 1).expand(b, stems, -1, t, 2)
        summed = vals.new_zeros(b, stems, self.num_rows, t, 2).scatter_add_(2, idx, vals)
        summed = summed / self.bands_per_row.view(1, 1, -1, 1, 1).to(summed.dtype)
        return torch.view_as_complex(summed.contiguous())


__all__ = ["MelBandRoformer", "mel_band_bins", "mel_filterbank", "hz_to_mel", "mel_to_hz"]

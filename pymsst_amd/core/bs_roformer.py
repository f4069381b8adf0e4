"""BS-RoFormer (band-split RoPE transformer) for music source separation, stock PyTorch.

Restated from the public BS-RoFormer architecture in the layout pymss-core's
model exposes to the reference's patch layer (``band_split``, ``layers`` of
``(time_transformer, freq_transformer)``, ``final_norm``, ``mask_estimators``,
``RoformerRuntimeMixin._estimate_masks``).  pymss-core itself is not available,
so feature packing, rotary tables and init follow the public architecture:

* STFT (``center=True``) of each channel; the complex spectrum is packed as
  ``(freq, channel, re/im)`` so band ``b`` owns ``4 * bins_b`` consecutive
  features for stereo input.
* ``depth`` axial blocks: a time transformer over frames (batch ``B * NB``) and a
  frequency transformer over bands (batch ``B * T``), each with its own rotary
  table shared across depth; no output norm inside blocks, one ``final_norm``.
* Mask estimators: per band ``MLP(dim -> hidden -> 2 * 4 * bins_b)`` + GLU; the
  masks multiply the complex STFT and iSTFT returns the separated stems.
* Loss when ``target`` is given (``loss=``): ``"multi_stft"`` = waveform L1 plus the
  multi-resolution STFT L1 (windows 4096, 2048, 1024, 512, 256; hop 147;
  ``n_fft = max(win, 2048)``); ``"l1"`` = waveform L1; ``"spec_l1"`` = L1 between the
  estimated and the target complex spectrograms (real and imaginary parts).
* ``checkpoint_blocks=True`` recomputes each axial block in the backward.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn
from torch.utils.checkpoint import checkpoint

from .bands import BandSplit, MaskEstimator
from .common import RoformerRuntimeMixin
from .transformer import RMSNorm, RotaryEmbedding, Transformer

DEFAULT_FREQS_PER_BANDS = (2,) * 24 + (4,) * 12 + (12,) * 8 + (24,) * 8 + (48,) * 8 + (128, 129)


class BSRoformer(RoformerRuntimeMixin, nn.Module):
    def __init__(
        self,
        dim: int,
        *,
        depth: int,
        stereo: bool = False,
        num_stems: int = 1,
        time_transformer_depth: int = 2,
        freq_transformer_depth: int = 2,
        freqs_per_bands=DEFAULT_FREQS_PER_BANDS,
        dim_head: int = 64,
        heads: int = 8,
        attn_dropout: float = 0.0,
        ff_dropout: float = 0.0,
        stft_n_fft: int = 2048,
        stft_hop_length: int = 512,
        stft_win_length: int = 2048,
        stft_normalized: bool = False,
        mask_estimator_depth: int = 2,
        mlp_expansion_factor: int = 4,
        multi_stft_resolution_loss_weight: float = 1.0,
        multi_stft_resolutions_window_sizes=(4096, 2048, 1024, 512, 256),
        multi_stft_hop_size: int = 147,
        multi_stft_normalized: bool = False,
        rotary_theta: float = 10000.0,
        checkpoint_blocks: bool = False,
        loss: str = "multi_stft",
        zero_dc: bool = False,
        _check_cover: bool = True,
    ):
        super().__init__()
        if loss not in ("multi_stft", "l1", "spec_l1"):
            raise ValueError(f"unknown loss {loss!r}")
        self.loss_type = loss
        self.stereo = stereo
        self.audio_channels = 2 if stereo else 1
        self.num_stems = num_stems
        self.checkpoint_blocks = checkpoint_blocks
        self.zero_dc = zero_dc  # zero frequency bin 0 of the masked spectrum before the iSTFT
        time_rotary = RotaryEmbedding(dim_head, rotary_theta)
        freq_rotary = RotaryEmbedding(dim_head, rotary_theta)
        kw = dict(dim=dim, heads=heads, dim_head=dim_head, attn_dropout=attn_dropout, ff_dropout=ff_dropout,
                  norm_output=False)
        self.layers = nn.ModuleList(
            [
                nn.ModuleList(
                    [
                        Transformer(depth=time_transformer_depth, rotary_embed=time_rotary, **kw),
                        Transformer(depth=freq_transformer_depth, rotary_embed=freq_rotary, **kw),
                    ]
                )
                for _ in range(depth)
            ]
        )
        self.final_norm = RMSNorm(dim)
        self.stft_kwargs = dict(n_fft=stft_n_fft, hop_length=stft_hop_length, win_length=stft_win_length,
                                normalized=stft_normalized)
        self.stft_win_length = stft_win_length
        n_freqs = stft_n_fft // 2 + 1
        if _check_cover and sum(freqs_per_bands) != n_freqs:
            raise ValueError(f"freqs_per_bands must sum to {n_freqs}, got {sum(freqs_per_bands)}")
        self.freqs_per_bands = tuple(int(f) for f in freqs_per_bands)
        dims_in = tuple(2 * f * self.audio_channels for f in self.freqs_per_bands)
        self.band_split = BandSplit(dim, dims_in)
        self.mask_estimators = nn.ModuleList(
            [MaskEstimator(dim, dims_in, depth=mask_estimator_depth, mlp_expansion_factor=mlp_expansion_factor)
             for _ in range(num_stems)]
        )
        self.multi_stft_resolution_loss_weight = multi_stft_resolution_loss_weight
        self.multi_stft_resolutions_window_sizes = tuple(multi_stft_resolutions_window_sizes)
        self.multi_stft_n_fft = stft_n_fft
        self.multi_stft_kwargs = dict(hop_length=multi_stft_hop_size, normalized=multi_stft_normalized)

    # ---------------------------------------------------------------- STFT packing
    def _stft(self, audio: torch.Tensor):
        """``audio[B, C, L]`` -> complex ``[B, F*C, T]`` (frequency-major, channel inner)."""
        b, c, length = audio.shape
        window = torch.hann_window(self.stft_win_length, device=audio.device, dtype=torch.float32)
        spec = torch.stft(audio.reshape(b * c, length).float(), window=window, return_complex=True, **self.stft_kwargs)
        f, t = spec.shape[-2:]
        return spec.reshape(b, c, f, t).transpose(1, 2).reshape(b, f * c, t), window

    def _band_features(self, spec: torch.Tensor) -> torch.Tensor:
        """Complex ``spec[B, F*C, T]`` -> band-split input ``[B, T, F*C*2]`` (bands are contiguous runs of
        frequencies, so the features are the spectrum itself)."""
        b, _, t = spec.shape
        return torch.view_as_real(spec).permute(0, 2, 1, 3).reshape(b, t, -1)

    def _spectral_mask(self, mask: torch.Tensor) -> torch.Tensor:
        """Mask-estimator output ``[B, stems, T, F*C*2]`` -> complex mask ``[B, stems, F*C, T]``."""
        b, stems, t = mask.shape[:3]
        return torch.view_as_complex(mask.float().reshape(b, stems, t, -1, 2).contiguous()).transpose(-1, -2)

    def _masked_spectrum(self, spec: torch.Tensor, mask: torch.Tensor, channels: int) -> torch.Tensor:
        """Complex ``spec[B, F*C, T]`` times the stems' masks (mask-estimator output
        ``[B, stems, T, F*C*2]``) in the layout iSTFT consumes, ``[B * stems * C, F, T]``; frequency bin 0
        is zeroed when ``zero_dc`` (the layout and fill of pymsst's cached-zero iSTFT,
        ``cuda_graph.py:140-158``)."""
        b, stems, t = mask.shape[:3]
        est = spec.unsqueeze(1) * self._spectral_mask(mask)  # [B, stems, F*C, T]
        est = est.reshape(b, stems, -1, channels, t).transpose(2, 3).reshape(b * stems * channels, -1, t)
        if self.zero_dc:
            est = est.index_fill(1, torch.zeros(1, dtype=torch.long, device=est.device), 0.0)
        return est

    def _axial(self, x: torch.Tensor, time_tf: Transformer, freq_tf: Transformer) -> torch.Tensor:
        b, t, nb, d = x.shape
        x = time_tf(x.transpose(1, 2).reshape(b * nb, t, d)).reshape(b, nb, t, d).transpose(1, 2)
        x = freq_tf(x.reshape(b * t, nb, d)).reshape(b, t, nb, d)
        return x

    def forward(self, raw_audio: torch.Tensor, target: torch.Tensor | None = None):
        """``raw_audio[B, C, L]`` (or ``[B, L]``) -> separated audio ``[B, stems, C, L]`` (stems squeezed
        when 1), or the training loss when ``target`` is given."""
        if raw_audio.ndim == 2:
            raw_audio = raw_audio.unsqueeze(1)
        b, c, length = raw_audio.shape
        spec, window = self._stft(raw_audio)  # [B, F*C, T] complex
        if target is not None and self.loss_type == "spec_l1":
            return self._spec_loss(spec.unsqueeze(1) * self._spectral_mask(self._masks(spec)), target, c)
        return self._finish(self._mask_core(spec, c), window, b, c, length, target)

    def _masks(self, spec: torch.Tensor) -> torch.Tensor:
        """Complex ``spec[B, F*C, T]`` -> the stems' masks ``[B, stems, T, features]`` (band features,
        band split, axial blocks, final norm, mask estimators)."""
        return self._estimate_masks(self._mask_features(spec))

    def _mask_features(self, spec: torch.Tensor) -> torch.Tensor:
        """Complex ``spec[B, F*C, T]`` -> the mask estimators' input ``[B, T, NB, dim]`` (band features,
        band split, axial blocks, final norm)."""
        x = self._band_features(spec)  # [B, T, features]
        x = self.band_split(x)  # [B, T, NB, dim]
        for time_tf, freq_tf in self.layers:
            if self.checkpoint_blocks and self.training:
                x = checkpoint(self._axial, x, time_tf, freq_tf, use_reentrant=False)
            else:
                x = self._axial(x, time_tf, freq_tf)
        return self.final_norm(x)

    def _mask_core(self, spec: torch.Tensor, channels: int) -> torch.Tensor:
        """The part between STFT and iSTFT (pymsst's "mask core"): complex ``spec[B, F*C, T]`` -> masked
        spectrum in the iSTFT layout ``[B * stems * C, F, T]``."""
        return self._masked_spectrum(spec, self._masks(spec), channels)

    def _finish(self, est: torch.Tensor, window: torch.Tensor, batch: int, channels: int, length: int,
                target: torch.Tensor | None = None):
        """iSTFT of the masked spectrum -> audio ``[B, stems, C, L]`` (stems squeezed when 1), or the loss
        against ``target``."""
        recon = torch.istft(est, window=window, length=length, return_complex=False, **self.stft_kwargs)
        stems = est.shape[0] // (batch * channels)
        recon = recon.reshape(batch, stems, channels, length)
        if stems == 1:
            recon = recon[:, 0]
        if target is None:
            return recon
        return self.loss(recon, target)

    def _spec_loss(self, est: torch.Tensor, target: torch.Tensor, channels: int) -> torch.Tensor:
        """L1 on (re, im) of ``est[B, stems, F*C, T]`` against the STFT of ``target[B, stems, C, L]``."""
        b, stems = est.shape[:2]
        if target.ndim == 3:
            target = target.unsqueeze(1)
        tspec, _ = self._stft(target.reshape(b * stems, channels, -1))
        return F.l1_loss(torch.view_as_real(est), torch.view_as_real(tspec.reshape(est.shape)))

    def loss(self, recon: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        # one stem: recon is [B, C, L] (stem axis squeezed) and a stacked target [B, 1, C, L] drops
        # its singleton stem axis, so the loss compares item with item instead of broadcasting
        if target.ndim == recon.ndim + 1 and target.shape[1] == 1:
            target = target[:, 0]
        if target.ndim == recon.ndim - 1:
            target = target.unsqueeze(-2)
        target = target[..., : recon.shape[-1]]
        loss = F.l1_loss(recon, target)
        if self.loss_type == "l1":
            return loss
        multi = recon.new_zeros(())
        flat_r = recon.reshape(-1, recon.shape[-1]).float()
        flat_t = target.reshape(-1, target.shape[-1]).float()
        for win in self.multi_stft_resolutions_window_sizes:
            kw = dict(n_fft=max(win, self.multi_stft_n_fft), win_length=win, return_complex=True,
                      window=torch.hann_window(win, device=recon.device), **self.multi_stft_kwargs)
            multi = multi + F.l1_loss(torch.stft(flat_r, **kw), torch.stft(flat_t, **kw))
        return loss + self.multi_stft_resolution_loss_weight * multi

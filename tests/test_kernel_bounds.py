"""CPU: every HIP kernel of the fused train step stays inside its buffers and its LDS allocation at
the shapes of BASELINE.json's configs (tests/bounds_model.py replays the host dispatch and the
kernels' address arithmetic), and the replay itself detects planted addressing mistakes."""

from __future__ import annotations

import numpy as np
import pytest

import bounds_model as bm


@pytest.mark.parametrize("esz", [2, 4], ids=["16bit", "fp32"])
@pytest.mark.parametrize("config", ["configs0", "configs1", "configs3", "configs4"])
def test_fused_step_kernels_stay_in_bounds(config, esz):
    bad = {}
    for label, bnd in bm.all_replays(config, esz):
        v = bnd.violations()
        if v:
            bad[label] = v
    assert not bad, bad


def test_configs4_shapes_named_in_the_review_are_covered():
    """Band split at O = 512 over the 62 bands, M = 1896; grouped linear 512 -> 2048; mask final at
    H = 2048 (8-wave dx blocks); qkv rotary at [124, 948, 8, 64]; the gate at D = 512."""
    labels = [label for label, _ in bm.all_replays("configs4", 2)]
    for want in ("band_split_fwd", "band_split_bwd", "grouped_linear_fwd", "grouped_linear_bwd",
                 "mask_final_fwd", "mask_final_bwd", "rotary_qkv[124, 948, 8, 64]",
                 "attention_gate[124, 948, 8, 64]"):
        assert want in labels
    b = bm.replay_mask_final_backward(bm.BSR_WIDTHS, 1896, 2048, 2, tanh_in=True)
    assert b.sizes["lds"] == 3 * (32 * 256 * 2 + 8192)  # the 8-wave (HC = 256) dx kernel's ring
    assert not b.violations()


def test_replay_flags_a_short_buffer():
    b = bm.replay_band_split_forward(bm.BSR_WIDTHS, 1032, 192, 2)
    assert not b.violations()
    b.sizes["out"] -= 2
    assert any(v.startswith("out:") for v in b.violations())


def test_replay_flags_a_wrong_swizzle(monkeypatch):
    """A K-unit swizzle that names units past the four 16-byte units of a 64-byte K chunk makes the
    mask forward's DMA read past the last row of x and W; the replay catches it (the planted
    mistake is in the replay, on the CPU)."""
    assert not bm.replay_mask_final_forward(bm.BSR_WIDTHS, 1032, 768, 2).violations()
    monkeypatch.setattr(bm, "swz_k", lambda r: 4 + (r & 3))
    v = bm.replay_mask_final_forward(bm.BSR_WIDTHS, 1032, 768, 2).violations()
    assert any(x.startswith("x:") for x in v) and any(x.startswith("weight:") for x in v)


def test_replay_flags_a_schedule_that_skips_units():
    units = lambda b: 3  # noqa: E731
    sc = bm.build_band_sched(62, 9, units)
    bnd = bm.Bounds({})
    bm.sched_decode(sc, 62, units, False, bnd, "ok")
    assert not bnd.violations()
    sc.gs[3] += 1  # XCD 2 runs one block more, XCD 3 one less: a unit runs twice
    bnd = bm.Bounds({})
    bm.sched_decode(sc, 62, units, False, bnd, "tampered")
    assert any("exactly once" in v for v in bnd.violations())


def test_replay_flags_an_unclamped_row():
    """The row clamp of the register loaders is what keeps the last row tile in bounds: with
    rows_valid set past the real rows the replay reports it."""
    b = bm.Bounds({"x": 100 * 64 * 2})
    tid = np.arange(bm.GEMM_THREADS)
    bm.krow_loader(b, "x", 2, 64 * 64, 64, 36, 64, 64, True, 0, 2, tid)
    assert not b.violations()
    bm.krow_loader(b, "x", 2, 64 * 64, 64, 64, 64, 64, True, 0, 2, tid)
    assert b.violations()


def test_mixed_band_split_replay_covers_its_buffers_and_flags_mistakes(monkeypatch):
    """The fp32-input band split's row-sum and column passes touch exactly their buffers at configs[1];
    a short features buffer and a band lookup that returns the next band are caught."""
    reps = dict(bm.replay_band_split_mixed(bm.BSR_WIDTHS, 1032, 192))
    for label, b in reps.items():
        assert not b.violations(), (label, b.violations())
    norm = reps["band_split_mixed_fwd_norm"]
    assert norm.hi["features"] == norm.sizes["features"] and norm.hi["x"] == norm.sizes["x"]
    b = dict(bm.replay_band_split_mixed(bm.BSR_WIDTHS, 1032, 192))["band_split_mixed_fwd_norm"]
    b.sizes["features"] -= 2
    assert any(v.startswith("features:") for v in b.violations())
    real = bm.np.searchsorted
    monkeypatch.setattr(bm.np, "searchsorted", lambda a, v, side="left": real(a, v, side=side) + 1)
    v = dict(bm.replay_band_split_mixed(bm.BSR_WIDTHS, 1032, 192))["band_split_mixed_fwd_norm"].violations()
    assert v


def test_grouped_dw_192_column_tiles_stay_in_bounds():
    """The grouped-linear dW on 192 output columns per block (chosen when it takes fewer rounds of
    resident blocks), with a partly filled last column tile (776 = 4 x 192 + 8)."""
    assert bm.dw_jt(100, 192, 776) == 192 and bm.dw_jt(62, 192, 768) == 192 and bm.dw_jt(62, 512, 2048) == 128
    b = bm.replay_band_split_backward([192] * 100, 100, 776, 2, grouped=True)
    assert b.sizes["lds_dw"] == 3 * 32 * 2 * (64 + 192)
    assert not b.violations()


def test_mask_mlp_row_tiles_stay_in_bounds():
    """The one-pass MLP's row tile: one wave's rows less than the block where the full tile would
    leave a last tile of at most an eighth (M = 1032 at dim 192: 4 x 224 + 136 rows), the full
    tile elsewhere; every tile height that is a multiple of 16 replays clean, others are refused."""
    widths = [8] * 24 + [16] * 12 + [48] * 8 + [96] * 8 + [192] * 8 + [512, 516]
    assert bm.mlp_row_tile(1032, 2, 8) == 224 and bm.mlp_row_tile(1033, 2, 8) == 224
    assert bm.mlp_row_tile(1024, 2, 8) == 256 and bm.mlp_row_tile(1896, 2, 8) == 256
    assert bm.mlp_row_tile(4104, 2, 8) == 256  # 224-row tiles would need two more
    assert bm.mlp_row_tile(140, 2, 4) == 96 and bm.mlp_row_tile(300, 2, 4) == 128
    for M, D, H in ((1032, 192, 768), (257, 192, 768), (140, 512, 2048), (31, 192, 768)):
        assert not bm.replay_mask_mlp_forward(widths, M, D, H, 2).violations(), (M, D)
    for rb in (160, 176, 192, 208, 224, 240, 256):
        assert not bm.replay_mask_mlp_forward(widths, 1032, 192, 768, 2, rb=rb).violations(), rb
    assert bm.replay_mask_mlp_forward(widths, 1032, 192, 768, 2, rb=200).violations()
    assert bm.replay_mask_mlp_forward(widths, 1032, 192, 768, 2, rb=272).violations()


def test_grouped_dx_row_tiles_stay_in_bounds():
    """glin_dx's 48-row-wave form takes the smallest multiple of 16 rows that keeps the grid in the
    full tile's block rounds (configs[1]: 8 tiles of 144 rows in one round of 2 x 256 blocks); every
    tile height up to the block's 192 rows replays clean, others are refused."""
    assert bm.gdx_tiles(192, 62, 1032)[1] == 3 and bm.gdx_row_tile(1032, 62, 3) == 144
    assert 62 * bm.cdiv(1032, 144) <= bm.GDX_SLOTS < 62 * bm.cdiv(1032, 128)
    assert bm.gdx_row_tile(2760, 60, 3) == 176 and bm.gdx_row_tile(1032, 62, 2) == 128

    def replay(M, G, rb=None):
        b = bm.Bounds({"dy": M * G * 768 * 2, "weight": G * 768 * 192 * 2, "dx": M * G * 192 * 2,
                       "lds_gdx": 0})
        bm._replay_glin_dx(b, G, 192, 768, M, rb=rb)
        return b.violations()

    for M, G in ((1032, 62), (1033, 62), (2760, 60)):
        assert not replay(M, G), (M, G)
    for rb in range(16, 193, 16):
        assert not replay(1032, 62, rb), rb
    assert replay(1032, 62, 200) and replay(1032, 62, 208)

"""The CPU bounds replay (``tests/bounds_model.py``) restates the launchers' tile tables and the
kernels' ring and tile constants.  These tests read the same values out of the HIP sources, so a
change to a kernel's shape that is not mirrored in the replay fails here instead of going unseen.
Each check names the source line it parses; a pattern that no longer matches fails too."""

from __future__ import annotations

import re
from pathlib import Path

import pytest

import bounds_model as bm

CSRC = Path(__file__).resolve().parent.parent / "pymsst_amd" / "csrc"


def _src(name: str) -> str:
    return (CSRC / name).read_text()


def _one(pattern: str, text: str, what: str) -> re.Match:
    found = list(re.finditer(pattern, text))
    assert len(found) == 1, f"{what}: pattern {pattern!r} matched {len(found)} times"
    return found[0]


def _const(name: str, src: str) -> int:
    return int(_one(rf"constexpr int {name} = (\d+);", _src(src), name).group(1))


def _define(name: str, src: str) -> int:
    return int(_one(rf"#define {name} (\d+)", _src(src), name).group(1))


def test_shared_constants():
    assert _const("kChunkK", "mfma.h") == bm.CHUNK_K
    assert _const("kGemmThreads", "gemm.h") == bm.GEMM_THREADS
    assert _const("kRowSumMaxF", "band_split.hip") == bm.ROWSUM_MAX_F


def test_mask_mlp_tile_table_and_ring():
    """mask_mlp.hip launch_mlp_fwd: dim -> launch_dk<T, DK, NT[, WV = 4]>; kMlpJ; mlp_stages."""
    s = _src("mask_mlp.hip")
    table = {int(d): (int(dk), int(nt), int(wv or 4))
             for d, dk, nt, wv in re.findall(r"case (\d+): return launch_dk<T, (\d+), (\d+)(?:, (\d+))?>", s)}
    assert table == bm.MLP_TILES
    assert _const("kMlpJ", "mask_mlp.hip") == 64
    m = _one(r"return DK >= (\d+) \? (\d+) : (\d+);", s, "mlp_stages")
    assert tuple(int(v) for v in m.groups()) == (12, 2, 3)  # S, J = (2 if DK >= 12 else 3), 64 in the replay
    # the row tile rule: full - 32 where the last full tile holds at most an eighth of a tile
    _one(r"const int64_t alt = full - 32;", s, "mlp_row_tile")
    _one(r"if \(M > full && tail <= full / 8 && \(M \+ alt - 1\) / alt == tiles\) return alt;", s, "mlp_row_tile")
    assert bm.mlp_row_tile(1032, 2, 8) == 224 and bm.mlp_row_tile(1024, 2, 8) == 256


def test_grouped_dx_tile_table_and_row_tile():
    """grouped_dx.hip launch_grouped_dx: in_features -> launch<T, DT, NT, S>, the two forms at 192."""
    s = _src("grouped_dx.hip")
    plain = {int(i): (int(dt), int(nt), int(st))
             for i, dt, nt, st in re.findall(r"case (\d+): return launch<T, (\d+), (\d+), (\d+)>", s)}
    assert plain == {k: v for k, v in bm.GDX_TILES.items() if k != 192}
    forms = set(re.findall(r"launch<T, 12, (\d+), (\d+)>", s))
    assert forms == {("3", "3"), ("2", "4")}
    assert bm.GDX_TILES[192] == (12, 2, 4)
    assert bm.gdx_tiles(192, 62, 1032) == (12, 3, 3)
    _one(r"if \(rounds\(192\) \* 3 <= rounds\(128\) \* 2\)", s, "48-row form rule")
    _one(r"const int64_t rb = \(\(M \+ tiles - 1\) / tiles \+ 15\) / 16 \* 16;", s, "gdx_row_tile")
    _one(r"const int64_t slots = 2 \* static_cast<int64_t>\(num_cus\(\)\);", s, "two blocks per CU")
    assert bm.GDX_SLOTS == 2 * 256


def test_mask_dz_ring_and_instances():
    s = _src("mask_dz.hip")
    assert _const("kDzStages", "mask_dz.hip") == 4
    assert set(re.findall(r"return launch<T, (\d+), (\d+)>", s)) == {("12", "2"), ("8", "2")}
    # the replay's block cost: K chunks + 5
    _one(r"\[&\]\(int b\) \{ return \(2 \* dim_inputs\[b\] \+ 31\) / 32 \+ 5; \}", s, "dz block cost")
    src_replay = Path(bm.__file__).read_text()
    assert "lambda b: cdiv(2 * widths[b], 32) + 5" in src_replay
    assert "S, HT = 4, 16 * DT" in src_replay


def test_mask_estimator_dpre_and_dw_rules():
    s = _src("mask_estimator.hip")
    assert _const("kDpreFlatRows", "mask_estimator.hip") == 4
    assert _const("kDpreFlatMaxBands", "mask_estimator.hip") == 4096
    m = _one(r"ring128 = (\d+) \* kChunkK \* 2 \* \(64 \+ 128\), ring192 = (\d+) \* kChunkK \* 2 \* \(64 \+ 192\)",
             s, "dW ring sizes")
    assert m.groups() == ("3", "3")
    _one(r"const int jt = rounds\(192, ring192\) < rounds\(128, ring128\) \? 192 : 128;", s, "dW tile rule")
    assert bm.dw_jt(62, 192, 768) == 192


def test_band_split_dw_ring():
    assert _define("PMSST_BS_DWD_STAGES", "band_split.hip") == 3
    assert _define("PMSST_BS_DWD_KS", "band_split.hip") == 2
    assert "S, KS = 3, 2" in Path(bm.__file__).read_text()


@pytest.mark.parametrize("mistake", ["table", "constant"])
def test_a_planted_mismatch_is_caught(monkeypatch, mistake):
    """A replay table or constant that no longer matches the source fails the checks above."""
    if mistake == "table":
        monkeypatch.setitem(bm.MLP_TILES, 192, (6, 2, 4))
        with pytest.raises(AssertionError):
            test_mask_mlp_tile_table_and_ring()
    else:
        monkeypatch.setattr(bm, "CHUNK_K", 64)
        with pytest.raises(AssertionError):
            test_shared_constants()

"""The autotuner's winner rule and the tile search's local refinement, host side (no GPU)."""
from __future__ import annotations

import importlib.util
from pathlib import Path

from factorized_inference import tilegen
from factorized_inference.tilegen import Tile

ROOT = Path(__file__).resolve().parents[1]
spec = importlib.util.spec_from_file_location(
    "autotune", ROOT / "kernel-task_amd" / "benchmarks" / "autotune.py")
autotune = importlib.util.module_from_spec(spec)
spec.loader.exec_module(autotune)

O = (2, 1, 0)
T8 = Tile(1, 1, 2, 12, 8, 4, 1)            # on all 8 XCDs
T4 = Tile(1, 1, 2, 12, 8, 4, 1, XL=4)      # the same tile on 4
T1 = Tile(1, 1, 10, 12, 8, 4, 1, 0, 16, 8, XL=1)
TILES = {"x8": (O, T8), "x4": (O, T4), "xl": (O, T1)}


def test_fastest_tile_wins():
    assert autotune.winner({"x8": 3.00, "x4": 3.20, "xl": 3.40}, TILES) == "x8"


def test_ties_go_to_fewer_xcds():
    # within 1 %: the 4-XCD copy wins over the 8-XCD tile even when it reads 0.5 % slower
    assert autotune.winner({"x8": 3.000, "x4": 3.015, "xl": 3.40}, TILES) == "x4"
    assert autotune.winner({"x8": 3.000, "x4": 3.015, "xl": 3.02}, TILES) == "xl"
    # beyond 1 %: speed decides
    assert autotune.winner({"x8": 3.00, "x4": 3.04}, TILES) == "x8"


def test_neighbours_are_valid_register_resident_tiles():
    shape = next(s for s in tilegen.BASELINE if s.key == "bf16_16x28x32_16x16x16_r16")
    base = Tile(2, 1, 16, 16, 2, 1, 2, 8, 32, 8, 1)
    nb = tilegen.neighbours(shape, O, base)
    assert nb and base not in nb.values()
    for t in nb.values():
        assert t.WIDE == base.WIDE and t.SC == base.SC and t.IC == base.IC
        assert not tilegen.geometry(shape, O, t)["reject"]
    got = {(t.TT, t.FC, t.PIPE) for t in nb.values()}
    assert {(1, 1, 1), (1, 2, 1), (2, 1, 0)} <= got
    # a tile that is not register-resident has no neighbours here
    assert tilegen.neighbours(shape, O, Tile(1, 1, 1, 16, 2, 8, 1, 0, 16, 8, 1)) == {}

"""CPU checks of the tile generator (factorized_inference/tilegen.py).

- The generator's mirror of the kernel's compile-time geometry agrees with the compiled
  library: for every MFMA variant of every plan (hand-written and generated tables) the LDS
  bytes match and the kernel's constraints accept the tile.
- The committed generated sources are what the generator writes now.
- Every declared shape gets MFMA variants whose default token ranges cover every token
  count, in the chain order the generator chose.
- Planted mistakes in a tile (a rank that is not a power of two, FC*TT not dividing 16 on a
  16x16 stage-2 tile, IC not dividing the last core's input mode, LDS over budget, a
  pipelined tile of one step, a pipelined tile whose doubled slices no longer fit) are
  rejected; FC*TT = 3 is accepted on a 32x32 stage-2 tile.
"""
from __future__ import annotations

from dataclasses import replace

import numpy as np
import pytest

from factorized_inference import _lib, tilegen

HAND = [
    tilegen.ShapeDecl("r8", (8, 12, 20), (12, 10, 24), 8, "f16"),
    tilegen.ShapeDecl("r16", (8, 12, 20), (12, 10, 24), 16, "f16"),
    tilegen.ShapeDecl("up", (16, 16, 16), (16, 28, 32), 8, "bf16"),
    tilegen.ShapeDecl("down", (16, 28, 32), (16, 16, 16), 16, "bf16"),
]
DT = {"f16": _lib.DTYPE_F16, "bf16": _lib.DTYPE_BF16, "f32": _lib.DTYPE_F32}


def parse(name: str):
    return tilegen.parse_variant_name(name)


def test_variant_names_parse_back_to_their_tiles():
    assert parse("ring3_mfma<210,1,1,2,12,8,4,1>") == ((2, 1, 0), tilegen.Tile(1, 1, 2, 12, 8, 4, 1))
    assert parse("ring3_mfma_w8<210,1,1,1,12,4,8,1>") == (
        (2, 1, 0), tilegen.Tile(1, 1, 1, 12, 4, 8, 1, 0, 16, 8))
    assert parse("ring3_mfma_wide8x32w8<012,4,1,28,32,4,1,2>") == (
        (0, 1, 2), tilegen.Tile(4, 1, 28, 32, 4, 1, 2, 8, 32, 8))
    assert parse("ring3_mfma_wide2<210,4,1,8,16,1,2,1>")[1].MF2 == 16
    assert parse("ring3_mfma_wide8x32w8p<210,8,1,10,12,1,1,2>")[1] == tilegen.Tile(
        8, 1, 10, 12, 1, 1, 2, 8, 32, 8, 1)
    assert parse("ring3_mfma_w8_p<210,1,1,1,12,4,8,1>")[1] == tilegen.Tile(
        1, 1, 1, 12, 4, 8, 1, 0, 16, 8, 1)
    assert parse("ring3_mfma_p<210,1,1,10,12,2,1,2>")[1].PIPE == 1
    assert parse("ring3_mfma_p2<210,1,1,10,12,2,1,2>")[1].PIPE == 2
    assert parse("ring3_mfma_wide8x32w8p2<210,2,1,16,16,1,1,2>")[1] == tilegen.Tile(
        2, 1, 16, 16, 1, 1, 2, 8, 32, 8, 2)
    assert parse("ring3_mfma_w8_xl<210,1,1,10,12,8,4,1>")[1] == tilegen.Tile(
        1, 1, 10, 12, 8, 4, 1, 0, 16, 8, XL=1)
    assert parse("ring3_mfma_wide8x32w8p_s4_xl<210,4,1,10,12,2,2,1>")[1] == tilegen.Tile(
        4, 1, 10, 12, 2, 2, 1, 8, 32, 8, 1, 4, 1)
    assert parse("ring3_mfma_x4<210,1,1,2,12,8,4,1>")[1] == tilegen.Tile(
        1, 1, 2, 12, 8, 4, 1, XL=4)
    assert parse("ring3_mfma_p_x2<210,1,1,5,12,8,1,2>")[1] == tilegen.Tile(
        1, 1, 5, 12, 8, 1, 2, PIPE=1, XL=2)
    assert parse("ring3_mfma_wide4x32_sl<210,1,1,10,12,4,2,1>")[1] == tilegen.Tile(
        1, 1, 10, 12, 4, 2, 1, 4, 32, 4, SL=1)
    assert parse("ring3_mfma_wide8x32w8p_s4_g_sl<210,1,2,16,16,2,2,1>")[1] == tilegen.Tile(
        1, 2, 16, 16, 2, 2, 1, 8, 32, 8, 1, 4, YM=1, SL=1)
    assert parse("ring3_mfma_x4_sl<210,1,1,2,12,8,4,1>")[1] == tilegen.Tile(
        1, 1, 2, 12, 8, 4, 1, XL=4, SL=1)
    assert parse("ring3_mfma_wide8x32w8p_sl_tp<210,1,3,10,12,2,4,1>")[1] == tilegen.Tile(
        1, 3, 10, 12, 2, 4, 1, 8, 32, 8, 1, SL=1, TP=1)
    with pytest.raises(ValueError):
        parse("ring3_generic<012,rc=8>")


def test_xcd_placed_tiles_emit_every_trailing_argument():
    # XL is the last argument of tile(shape, ...), so an XCD-local tile spells out the
    # defaults before it
    assert tilegen.Tile(1, 1, 10, 12, 8, 4, 1, 0, 16, 8, XL=1).args() == \
        "1, 1, 10, 12, 8, 4, 1, 0, 16, 8, 0, 0, 1"
    assert tilegen.Tile(1, 1, 2, 12, 8, 4, 1).args() == "1, 1, 2, 12, 8, 4, 1"
    # so do a tile whose second-core slice is read late (SL) and one with tail priority (TP,
    # the last argument)
    assert tilegen.Tile(1, 3, 10, 12, 2, 4, 1, 8, 32, 8, 1, SL=1).args() == \
        "1, 3, 10, 12, 2, 4, 1, 8, 32, 8, 1, 0, 0, 0, 1"
    assert tilegen.Tile(1, 3, 10, 12, 2, 4, 1, 8, 32, 8, 1, TP=1).args() == \
        "1, 3, 10, 12, 2, 4, 1, 8, 32, 8, 1, 0, 0, 0, 0, 1"
    # the headline shape's table carries an XCD-local tile, index-only, beside its winners
    shape = tilegen.BASELINE[0]
    xl = [(n, t, lo, hi) for n, _, t, lo, hi in tilegen.table(shape) if t.XL == 1]
    assert xl and all((lo, hi) == (0, 0) for *_, lo, hi in xl)
    # and the extended search offers single-token tiles on 1, 2 and 4 XCDs; those on 2 and 4
    # only where a token tile's workgroups fit those XCDs' CUs
    placed = [(o, t) for o, t in tilegen.search_candidates(shape, extended=True).values() if t.XL]
    assert {t.XL for _, t in placed} == {1, 2, 4}
    for o, t in placed:
        nblk = tilegen.geometry(shape, o, t)["NBLK"]
        assert t.TT == 1 and nblk % t.XL == 0 and (t.XL == 1 or nblk <= 32 * t.XL)
    plan = _lib.Plan(shape.ins, shape.outs, shape.rank, DT[shape.dtype])
    v = next(v for v in plan.variants(1) if "_xl<" in v["name"])
    assert v["grid"][0] == 8 * 24 and v["t_min"] == 0
    # the tuned single-token winner runs on 4 XCDs: 120 working workgroups in a grid of 240
    v = plan.describe(-1, 1)
    assert "_x4<" in v["name"] and v["grid"][0] == 2 * 120


@pytest.mark.parametrize("shape", tilegen.DECLARED, ids=lambda s: s.key)
def test_variant_names_are_unique_and_name_their_tiles(shape):
    # the autotuner and the trace summaries key timings by name: two different tiles of one
    # plan may not share one (a tile serving several token ranges is registered once per
    # range, under one name), and each name parses back to a tile the table compiled
    plan = _lib.Plan(shape.ins, shape.outs, shape.rank, DT[shape.dtype])
    names = {v["name"] for v in plan.variants(1) if v["kind"] == "mfma"}
    compiled = {(o, t) for _, o, t, _, _ in tilegen.table(shape)}
    assert len(names) == len(compiled)
    assert {parse(n) for n in names} == compiled


@pytest.mark.parametrize("shape", HAND + tilegen.DECLARED, ids=lambda s: s.key)
def test_geometry_mirror_matches_the_library(shape):
    plan = _lib.Plan(shape.ins, shape.outs, shape.rank, DT[shape.dtype])
    mfma = [v for v in plan.variants(1) if v["kind"] == "mfma"]
    assert mfma
    for v in mfma:
        order, tile = parse(v["name"])
        g = tilegen.geometry(shape, order, tile)
        assert g["LDS_BYTES"] == v["lds_bytes"], v["name"]
        # the hand tables hold a few register-heavy sweep variants beyond the generator's
        # register budget; every other constraint holds for all compiled tiles
        assert g["reject"] in ("", "register-resident slices too large"), (v["name"], g["reject"])
        assert list(order) == v["order"]


def test_generated_sources_are_current(tmp_path):
    written = tilegen.write_all(out_dir=tmp_path)
    for p in written:
        committed = tilegen.GEN_DIR / p.name
        assert committed.exists(), f"{p.name} is not generated in csrc/gen"
        assert committed.read_text() == p.read_text(), f"{p.name} is stale: rerun tilegen"


@pytest.mark.parametrize("shape", tilegen.DECLARED, ids=lambda s: s.key)
def test_declared_shapes_are_covered(shape):
    rows = tilegen.table(shape)
    plan = _lib.Plan(shape.ins, shape.outs, shape.rank, DT[shape.dtype])
    for T in (1, 2, 3, 7, 8, 16, 17, 33, 64, 65, 128, 256, 4096):
        info = plan.describe(-1, T)
        assert info["kind"] == "mfma", (shape.key, T)
        # the selected tile is the table's tile for T, in that row's chain order
        covering = [r for r in rows if r[3] <= T <= r[4]]
        assert len(covering) == 1, (shape.key, T)
        name, order, tile, _, _ = covering[0]
        assert tuple(info["order"]) == order
        assert tilegen.parse_variant_name(info["name"]) == (order, tile), (name, info["name"])
    for _, order, tile, lo, hi in rows:
        assert not tilegen.geometry(shape, order, tile)["reject"]
        assert (lo, hi) == (0, 0) or 1 <= lo <= hi


def test_every_table_row_is_registered():
    # a plan holds a bounded number of variants: none of a shape's tiles may be dropped
    for shape in tilegen.DECLARED:
        plan = _lib.Plan(shape.ins, shape.outs, shape.rank, DT[shape.dtype])
        names = [v["name"] for v in plan.variants(1) if v["kind"] == "mfma"]
        assert len(names) == len(tilegen.table(shape)), shape.key
        key = lambda ot: (ot[0], tuple(vars(ot[1]).values()))  # noqa: E731
        assert sorted(map(tilegen.parse_variant_name, names), key=key) == sorted(
            ((order, tile) for _, order, tile, _, _ in tilegen.table(shape)), key=key)


def test_search_orders():
    for shape in tilegen.DECLARED:
        orders = tilegen.search_orders(shape, extended=True)
        assert orders[0] == tilegen.choose_order(shape) == tilegen.search_orders(shape)[0]
        assert len(set(orders)) == len(orders)
        least = min(tilegen.padded_work(shape, o)[0] for o in tilegen.ORDERS)
        for o in orders[1:]:
            assert tilegen.padded_work(shape, o)[0] <= tilegen.ALT_ORDER_SLACK * least
    # candidates of another order carry its tag and parse back to that order
    cands = tilegen.search_candidates(HAND[3], extended=True)
    tagged = [n for n in cands if "@" in n]
    assert tagged and all(cands[n][0] == tuple(int(c) for c in n.split("@")[1]) for n in tagged)


def test_order_choice_prefers_least_padded_work():
    for shape in tilegen.DECLARED + HAND:
        best = tilegen.choose_order(shape)
        if shape.order is not None:  # an explicit order (measured faster) wins
            assert best == tuple(shape.order)
            continue
        work = {o: tilegen.padded_work(shape, o) for o in tilegen.ORDERS}
        assert work[best] == min(work.values())
    # the chosen order never does more unpadded work than twice the least
    for shape in tilegen.DECLARED:
        unpadded = [tilegen.padded_work(shape, o)[1] for o in tilegen.ORDERS]
        assert tilegen.padded_work(shape, tilegen.choose_order(shape))[1] <= 2 * min(unpadded)


@pytest.mark.parametrize("shape,tile,why", [
    (tilegen.ShapeDecl("r12", (8, 12, 20), (12, 10, 24), 12), tilegen.Tile(1, 1, 2, 12, 8, 4, 1),
     "power of two"),
    (HAND[0], tilegen.Tile(3, 1, 2, 12, 8, 4, 1), "divide 16"),
    (HAND[0], tilegen.Tile(1, 1, 2, 12, 3, 1, 1), "IC must divide"),
    (HAND[1], tilegen.Tile(1, 1, 10, 12, 8, 1, 1), "LDS"),
    (HAND[0], tilegen.Tile(1, 1, 2, 12, 8, 3, 1), "KS3"),
    (HAND[0], tilegen.Tile(1, 1, 2, 12, 8, 4, 1, PIPE=1), "two steps"),
    (HAND[1], tilegen.Tile(1, 1, 5, 12, 4, 1, 2, PIPE=1), "LDS"),  # fits with one buffer
    (HAND[0], tilegen.Tile(1, 1, 2, 12, 8, 4, 1, XL=4, YM=1), "YM"),
    (HAND[0], tilegen.Tile(1, 1, 2, 12, 8, 4, 1, SL=2), "SL"),
    # tail priority on a tile whose stage 2 has no tail waves (8 row tiles on 8 waves)
    (HAND[3], tilegen.Tile(1, 2, 16, 16, 2, 2, 1, 8, 32, 8, 1, 4, TP=1), "TP"),
])
def test_planted_tile_mistakes_are_rejected(shape, tile, why):
    assert why in tilegen.geometry(shape, (2, 1, 0), tile)["reject"]


def test_first_core_chunks_beyond_powers_of_two_only_on_32x32_stage2():
    # TT*FC = 3: the 32x32 stage-2 stores compute their column offsets per lane, so the
    # register-resident 32x32 tiles take it; the 16x16 stage-2 tiles keep the split offsets
    # and need TT*FC to divide 16
    r16 = HAND[1]
    wide32 = tilegen.Tile(1, 3, 10, 12, 2, 4, 1, 8, 32, 8, 1)
    assert tilegen.geometry(r16, (2, 1, 0), wide32)["reject"] == ""
    assert tilegen.geometry(r16, (2, 1, 0), wide32)["NBLK"] == 8  # 24 first-core digits / 3
    lds16 = tilegen.Tile(1, 3, 2, 12, 4, 4, 1)
    assert "divide 16" in tilegen.geometry(r16, (2, 1, 0), lds16)["reject"]
    wide16 = tilegen.Tile(1, 3, 10, 12, 2, 4, 1, 8, 16, 8)
    assert "divide 16" in tilegen.geometry(r16, (2, 1, 0), wide16)["reject"]
    # the extended search offers the family on the 24-digit first core only
    names = tilegen.candidates(r16, (2, 1, 0), extended=True)
    assert any(t.FC == 3 and t.TT == 1 for t in names.values())
    assert not any(t.FC * t.TT not in (1, 2, 4, 8, 16)
                   for t in tilegen.candidates(HAND[3], (2, 1, 0), extended=True).values())


def test_extended_search_offers_the_chip_filling_one_token_tiles():
    # one-token register-resident tiles that split the second core in two or four, and ones
    # that cross first-core chunks of 2-8 digits with those splits: the families the tuned
    # tables took at Llama down T=3-8, R16 T=3-4, Llama up from 65 tokens and R8 from 129
    down = tilegen.candidates(HAND[3], (2, 1, 0), extended=True).values()
    assert {8, 4} <= {t.SC for t in down if t.TT == 1 and t.FC == 1 and t.MF2 == 32}
    r16 = tilegen.candidates(HAND[1], (2, 1, 0), extended=True).values()
    assert any(t.TT == 1 and t.FC == 1 and t.SC == 5 and t.MF2 == 32 for t in r16)
    up = tilegen.candidates(HAND[2], (0, 1, 2), extended=True).values()
    assert any(t.TT == 1 and t.FC == 8 and t.SC == 28 and t.MF2 == 32 for t in up)
    r8 = tilegen.candidates(HAND[0], (2, 1, 0), extended=True).values()
    assert any(t.TT == 1 and t.FC == 8 and t.SC == 10 and t.WIDE == 4 and t.NW == 8 for t in r8)
    # every offered tile passes the kernel's constraints
    for shape, order, tiles in ((HAND[3], (2, 1, 0), down), (HAND[1], (2, 1, 0), r16)):
        assert all(tilegen.geometry(shape, order, t)["reject"] == "" for t in tiles)


def test_extended_search_offers_the_winners_with_late_slices_and_tail_priority():
    # every winner of a tuned table comes back with SL=1 and the same tile otherwise, the
    # register-resident and the LDS-staged ones alike
    tuned = tilegen.load_tuned()
    for shape in tilegen.BASELINE:
        rows = tilegen.table(shape, tuned, all_candidates=True, extended=True)
        late = {(o, t) for _, o, t, _, _ in rows if t.SL}
        prio = {(o, t) for _, o, t, _, _ in rows if t.TP}
        for r in tuned[shape.key]["ranges"]:
            t = tilegen.Tile(**r["tile"])
            order = tuple(r.get("order", tuned[shape.key]["order"]))
            assert t.SL or (order, replace(t, SL=1)) in late, (shape.name, r["name"])
            # and those whose stage 2 has tail waves also with the tail waves' priority
            tail = tilegen.geometry(shape, order, t)["TAIL"]
            assert t.TP or ((order, replace(t, TP=1)) in prio) == tail, (shape.name, r["name"])


def test_rule_ranges_cover_everything():
    for names in (["t1_s1", "mid_half", "mid_all", "wide8x32w8"], ["t1_s2", "mid_all"],
                  ["t1_s1"]):
        ranges = tilegen.rule_ranges(names)
        covered = np.zeros(300, bool)
        for lo, hi in ranges.values():
            covered[lo:min(hi, 299) + 1] = True
        assert covered[1:].all(), names



def test_candidates_with_one_name_keep_both_tiles():
    # shortened names of two refined winners can agree: the second tile gets a numbered
    # name instead of replacing the first; an identical tile is not added twice
    order = (2, 1, 0)
    t1, t2 = tilegen.Tile(1, 1, 10, 12, 4, 2, 1), tilegen.Tile(1, 1, 10, 12, 2, 2, 1)
    cands = {}
    assert tilegen.add_candidate(cands, "w~t1", order, t1) == "w~t1"
    assert tilegen.add_candidate(cands, "w~t1", order, t2) == "w~t1#2"
    assert tilegen.add_candidate(cands, "w~t1", order, t1) is None
    assert tilegen.add_candidate(cands, "w~t1", (0, 1, 2), t1) == "w~t1#3"
    assert cands == {"w~t1": (order, t1), "w~t1#2": (order, t2), "w~t1#3": ((0, 1, 2), t1)}

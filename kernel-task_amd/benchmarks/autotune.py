"""Autotuner of the generated MFMA variant tables: measure every compiled tile of every
declared shape over a grid of token counts and write the fastest per token range.

    python -m factorized_inference.tilegen --all   # compile every candidate (from kernel-task_amd/)
    python -m factorized_inference.build_ext
    python kernel-task_amd/benchmarks/autotune.py --out OUT/tuned.json    # on an MI355X
        (the winners' table; the raw timings of every candidate go to --measurements, a file
        outside the source tree, and never into the tables)
    cp OUT/tuned.json kernel-task_amd/csrc/gen/tuned.json
    python -m factorized_inference.tilegen && python -m factorized_inference.build_ext

Role of the reference's tools/qwen_sweep.py and tools/gen_v3g_tuned.py (a sweep of V3G
tilings per Qwen shape and token count, reduced to the fastest correct tiling per token
count, src/factorized_inference/v3g_tuned.py:4-17). Timing, median of three blocks:
- HIP events around the replay of a HIP graph of back-to-back calls of one tile. This gives
  the GPU time per call without the host's per-call cost (6-8 us through run_variant), which
  would hide the differences between fast tiles;
- for tiles that take 12 us or more (--eager-from-us; 0 re-times every tile), HIP events
  around back-to-back eager calls on the stream instead, as bench.py times them: the plan
  routed to the tile and called through its per-call path, whose host cost (~2.4 us a call)
  stays hidden behind the kernels. Graph replays ranked some tiles differently from eager
  calls (Llama up T=128: a graph put two tiles 1 % apart, eager calls 7 % apart the other
  way; tiles numbered over the whole launch, Tile.YM, won graph replays at 1920->2880 R8
  T=8-32 and lost eager calls by ~1 us).

Every variant's output is checked against the shape's default variant before it may win (bitwise equality
is not expected across tiles: the stage-3 summation order differs). Timings within 1 % count
as equal, and then the tile on the fewest XCDs wins (Tile.XL).

Candidates span every chain order the generator searches (tilegen.search_orders); each
range records its winner's order. Token counts measured: 1, 2, 4, 8, 16, 32, 64, 128, 256. The winner at T serves the range
(previous measured T, T]; 256's winner serves everything above.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from dataclasses import asdict
from pathlib import Path

os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "0")  # as bench.py
PACKAGE_ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(PACKAGE_ROOT))

import torch  # noqa: E402

from factorized_inference import TRSpec, make_cores, prepare_optimized, tilegen  # noqa: E402

GRID = (1, 2, 4, 8, 16, 32, 64, 128, 256)


def graph_us(fn, calls: int, blocks: int = 3) -> float:
    """GPU time per call of `calls` back-to-back calls captured in one HIP graph (no host
    cost in the timed region, so tiles that finish faster than a call's host work still
    rank correctly), median of `blocks` replays."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    out = []
    for _ in range(blocks):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        graph.replay()
        e.record()
        e.synchronize()
        out.append(s.elapsed_time(e) * 1000.0 / calls)
    del graph
    return statistics.median(out)


def eager_us(fn, calls: int, blocks: int = 3) -> float:
    """Stream time per call of `calls` back-to-back eager calls, median of `blocks` blocks."""
    out = []
    for _ in range(blocks):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(calls):
            fn()
        e.record()
        e.synchronize()
        out.append(s.elapsed_time(e) * 1000.0 / calls)
    return statistics.median(out)


EAGER_FROM_US = 12.0  # tiles this slow (graph-timed) are re-timed with eager calls (--eager-from-us)
PLACEMENT_TIE = 0.01  # timings this close count as equal: the fewer XCDs win


def xcds(tile: tilegen.Tile) -> int:
    """XCDs a tile's launch runs on (Tile.XL; 0 means all 8)."""
    return tile.XL or 8


def winner(row: dict[str, float], tiles: dict) -> str:
    """The fastest tile of one token count; among tiles within PLACEMENT_TIE of it, the one
    on the fewest XCDs (less HBM traffic and L2 write-back for the same latency, and the
    other XCDs stay free for concurrent work)."""
    best = min(row, key=row.get)
    close = [n for n in row if row[n] <= row[best] * (1 + PLACEMENT_TIE)]
    return min(close, key=lambda n: (xcds(tiles[n][1]), row[n]))


def tune_shape(shape: tilegen.ShapeDecl, budget_s: float,
               eager_from_us: float = EAGER_FROM_US) -> tuple[dict, dict]:
    dtype = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[shape.dtype]
    tol = 1e-4 if dtype is torch.float32 else 0.02  # the acceptance rule of the dtype
    spec = TRSpec(shape.ins, shape.outs, shape.rank)
    cores = make_cores(spec, device="cuda", dtype=dtype, seed=0, init="uniform")
    run = prepare_optimized(cores, spec)
    variants = [(i, v) for i, v in enumerate(run.variants()) if v["kind"] == "mfma"]
    names, tiles = {}, {}
    cands = tilegen.search_candidates(shape, extended=True)
    for i, v in variants:
        key = tilegen.parse_variant_name(v["name"])
        names[i] = next((n for n, c in cands.items() if c == key), v["name"])
        tiles[names[i]] = key
    measured: dict[int, dict[str, float]] = {}
    t_end = time.perf_counter() + budget_s
    default = {T: run.plan.select(T) for T in GRID}  # before any routing below
    for T in GRID:
        x = torch.randn(T, spec.in_features, device="cuda", dtype=dtype,
                        generator=torch.Generator(device="cuda").manual_seed(T))
        ref = run.run_variant(x, default[T]).float()
        scale = ref.abs().max().item()
        row = {}
        for i, v in variants:
            y = run.run_variant(x, i).float()
            torch.cuda.synchronize()
            err = (y - ref).abs().max().item()
            if not (err <= tol * scale + tol):  # a tile that disagrees never wins
                print(f"  {shape.key} T={T} {v['name']}: disagrees ({err:.3e}), skipped",
                      flush=True)
                continue
            fn = lambda i=i: run.run_variant(x, i)  # noqa: E731
            fn()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            torch.cuda.synchronize()
            one = (time.perf_counter() - t0) * 1e6
            calls = max(5, min(50, int(2e3 / max(one, 1.0))))
            us = graph_us(fn, calls)
            if us >= eager_from_us:
                # the per-call path of bench.py with the plan routed to this tile: its host
                # cost (~2.4 us a call) stays below the kernels, unlike run_variant's
                run.plan.set_variant(1, 1 << 30, i)
                fast = lambda: run(x)  # noqa: E731
                # blocks of ~20 ms: short blocks of a few-us kernel vary by several percent
                n = max(calls, min(4000, int(2e4 / max(us, 1.0))))
                for _ in range(n):  # the clock settles under load first
                    fast()
                us = eager_us(fast, n)
            row[names[i]] = us
        measured[T] = row
        best = winner(row, tiles)
        print(f"{shape.key} T={T:4d}: " + "  ".join(
            f"{n} {us:7.2f}{'*' if n == best else ''}" for n, us in sorted(row.items())),
            flush=True)
        if time.perf_counter() > t_end:
            print(f"  {shape.key}: time budget spent after T={T}", flush=True)
            break
    # winners per range (previous T, T]; the last measured T serves everything above
    ranges = []
    lo = 1
    done = sorted(measured)
    for k, T in enumerate(done):
        row = measured[T]
        best = winner(row, tiles)
        hi = (1 << 30) if k == len(done) - 1 else T
        if ranges and ranges[-1]["name"] == best:
            ranges[-1]["t_max"] = hi
        else:
            ranges.append({"name": best, "t_min": lo, "t_max": hi})
        lo = T + 1
    order = tilegen.choose_order(shape)
    for r in ranges:
        r["order"] = list(tiles[r["name"]][0])
        r["tile"] = asdict(tiles[r["name"]][1])
    return ({"order": list(order), "device": torch.cuda.get_device_name(0), "ranges": ranges},
            {str(T): row for T, row in measured.items()})


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", type=Path, required=True)
    ap.add_argument("--shapes", default="", help="comma-separated shape keys (default: all)")
    ap.add_argument("--seconds-per-shape", type=float, default=60.0)
    ap.add_argument("--eager-from-us", type=float, default=EAGER_FROM_US,
                    help="re-time with eager calls every tile whose graph time reaches this (0: "
                         "every tile). Graph replays keep the L2 warm across kernels where eager "
                         "launches do not, which ranked tiles differently on MI355X: one that "
                         "shares fewer core slices per XCD won graph replays and lost eager calls")
    ap.add_argument("--measurements", type=Path, default=Path("gpurun_out/autotune_us.json"),
                    help="where the raw per-candidate timings go (not part of the tables)")
    args = ap.parse_args()
    if not torch.cuda.is_available():
        print("autotune.py needs a ROCm GPU", file=sys.stderr)
        return 1
    wanted = set(filter(None, args.shapes.split(",")))
    result = json.loads(args.out.read_text()) if args.out.exists() else {}
    raw = json.loads(args.measurements.read_text()) if args.measurements.exists() else {}
    with torch.inference_mode():
        # bring the GPU to its working clock first (the first timings would read slow)
        a = torch.randn(4096, 4096, device="cuda", dtype=torch.float16)
        t_end = time.perf_counter() + 0.5
        while time.perf_counter() < t_end:
            for _ in range(20):
                a @ a
            torch.cuda.synchronize()
        del a
        for shape in tilegen.DECLARED:
            if wanted and shape.key not in wanted:
                continue
            prev = result.get(shape.key) or tilegen.load_tuned().get(shape.key) or {}
            result[shape.key], raw[shape.key] = tune_shape(shape, args.seconds_per_shape,
                                                           args.eager_from_us)
            if prev.get("extra"):  # index-only alternatives outlive a retune
                result[shape.key]["extra"] = prev["extra"]
            for path, data in ((args.out, result), (args.measurements, raw)):
                path.parent.mkdir(parents=True, exist_ok=True)
                path.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")
    print(f"wrote {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Summaries of rocprofv3 csv output: `--pmc` runs of `bench.py --traffic-probe`, and
kernel traces.

    # HBM traffic per launch (one FETCH_SIZE run and one WRITE_SIZE run of the same probe)
    python kernel-task_amd/benchmarks/counters.py traffic --fetch DIR --write DIR --out FILE.json
    # per-dispatch means of every counter of the probed kernel, one or more runs
    python kernel-task_amd/benchmarks/counters.py means DIR [DIR ...]
    # back-to-back blocks of one kernel in a --kernel-trace run (e.g. bench.py's timed block)
    python kernel-task_amd/benchmarks/counters.py blocks TRACE.csv --kernel REGEX [--grid N]
    # durations per (tensor-ring kernel, grid) in a --kernel-trace run: one kernel serves
    # several token counts (grids), which rocprofv3's --stats summary lumps together; each
    # row also gives the longest back-to-back block of that kernel and grid
    python kernel-task_amd/benchmarks/counters.py grids TRACE.csv [--out FILE.json]
    # one row per bench.py case: its kernel's durations in a traced bench.py run, beside the
    # case's stream time from that run's details file (bench.py's DETAILS)
    python kernel-task_amd/benchmarks/counters.py cases TRACE.csv DETAILS.json [--out FILE]

A probe run (bench.py --traffic-probe CALLS) launches one tensor-ring kernel CALLS times and
then copies a 512 MiB buffer 5 times. The copy is larger than every L2 and the 256 MB MALL,
so its bytes all cross from HBM: the counted KiB per copy against the 512 MiB it moves give
the scale between a counter and bytes (FETCH_SIZE counts 2x on MI355X at this writing,
WRITE_SIZE 1x), which is applied to the kernel's per-dispatch mean.

Role of the reference's tools/measure_kernels.py (profiler-derived rates of the fused kernel)
for the counters it has no equivalent of on its hardware.
"""
from __future__ import annotations

import argparse
import csv
import json
import re
import sys
from collections import defaultdict
from pathlib import Path

COPY_BYTES = 512 << 20  # bench.py traffic_probe: torch.ones(256 << 20, float16) copied


def _rows(run_dir: Path) -> list[dict]:
    files = sorted(Path(run_dir).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {run_dir}")
    with open(files[0], newline="") as f:
        return list(csv.DictReader(f))


def kernel_label(name: str) -> str | None:
    """'ring3<KCfg fields>' for a tensor-ring kernel, 'copy' for the runtime's buffer copy,
    None for anything else (allocation fills, packing, random inputs)."""
    if "ring3_mfma" in name:
        m = re.search(r"KCfg\{([^}]*)\}", name)
        return "ring3<" + (m.group(1).replace(" ", "") if m else "?") + ">"
    if "ring3_generic" in name:
        return "ring3_generic"
    if "copyBuffer" in name:
        return "copy"
    return None


def means(run_dir: Path) -> dict[str, dict[str, dict]]:
    """{kernel label: {counter: {"dispatches": n, "mean": per-dispatch mean}}}."""
    acc: dict = defaultdict(lambda: defaultdict(list))
    for r in _rows(run_dir):
        label = kernel_label(r["Kernel_Name"])
        if label is not None:
            acc[label][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return {k: {c: {"dispatches": len(v), "mean": sum(v) / len(v)} for c, v in cs.items()}
            for k, cs in acc.items()}


def probed_kernel(m: dict) -> str:
    """The tensor-ring kernel a probe launched (the most dispatched one)."""
    ring = [k for k in m if k.startswith("ring3")]
    if not ring:
        raise SystemExit("no tensor-ring kernel in the run")
    return max(ring, key=lambda k: max(v["dispatches"] for v in m[k].values()))


def traffic(fetch_dir: Path, write_dir: Path, algorithmic_bytes: float | None) -> dict:
    out = {"counters": {}}
    total = 0.0
    for counter, d in (("FETCH_SIZE", fetch_dir), ("WRITE_SIZE", write_dir)):
        m = means(d)
        kernel = probed_kernel(m)
        ring = m[kernel][counter]
        copy = m["copy"][counter]
        scale = COPY_BYTES / (copy["mean"] * 1024.0)
        nbytes = ring["mean"] * 1024.0 * scale
        out["kernel"] = kernel
        out["counters"][counter] = {
            "ring_kib_per_dispatch_mean": ring["mean"], "ring_dispatches": ring["dispatches"],
            "copy_kib_per_dispatch_mean": copy["mean"], "copy_dispatches": copy["dispatches"],
            "copy_bytes_actual": COPY_BYTES, "scale": scale, "ring_bytes_per_dispatch": nbytes}
        total += nbytes
    out["hbm_bytes_per_launch"] = total
    if algorithmic_bytes:
        out["algorithmic_bytes_per_launch"] = algorithmic_bytes
        out["ratio_to_algorithmic"] = total / algorithmic_bytes
    return out


def blocks(trace: Path, pattern: str, grid: int | None = None, max_gap_us: float = 30.0,
           min_len: int = 10) -> list[dict]:
    """Runs of consecutive dispatches of the kernels matching `pattern` (and grid size
    `grid`, in threads) whose gaps from the previous dispatch's end stay under max_gap_us:
    bench.py's timed blocks, told apart from isolated calls. Per run: dispatches, mean and
    min duration, first start (us from the first dispatch)."""
    with open(trace, newline="") as f:
        rows = [r for r in csv.DictReader(f) if re.search(pattern, r["Kernel_Name"]) and
                (grid is None or int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) == grid)]
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    if not rows:
        return []
    t0 = int(rows[0]["Start_Timestamp"])
    runs, cur, prev_end = [], [], None
    for r in rows:
        s, e = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        if prev_end is not None and (s - prev_end) / 1e3 > max_gap_us:
            runs.append(cur)
            cur = []
        cur.append((s, e))
        prev_end = e
    runs.append(cur)
    out = []
    for run in runs:
        if len(run) >= min_len:
            d = [(e - s) / 1e3 for s, e in run]
            out.append({"dispatches": len(run), "mean_us": sum(d) / len(d), "min_us": min(d),
                        "start_us": (run[0][0] - t0) / 1e3})
    return out


def _longest_block(spans: list[tuple[int, int]], max_gap_us: float) -> list[tuple[int, int]]:
    """The longest run of consecutive (start, end) spans whose gaps from the previous end stay
    under max_gap_us (spans sorted by start)."""
    best, cur, prev_end = [], [], None
    for s, e in spans:
        if prev_end is not None and (s - prev_end) / 1e3 > max_gap_us:
            cur = []
        cur.append((s, e))
        prev_end = e
        if len(cur) > len(best):
            best = list(cur)
    return best


def grids(trace: Path, max_gap_us: float = 30.0) -> list[dict]:
    """Per (tensor-ring or empty kernel, grid in workgroups x * y): dispatches and mean, min
    and median duration in us over every dispatch, most dispatched first; and the longest
    back-to-back block of that kernel and grid (dispatches whose gaps stay under max_gap_us:
    bench.py's timed blocks and its per-dispatch kernel timing), with its mean duration and
    its period (first start to last end over dispatches)."""
    acc: dict = defaultdict(list)
    with open(trace, newline="") as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            label = kernel_label(name) or ("empty" if "empty" in name else None)
            if label is None:
                continue
            if label == "empty":
                label = name.replace("(anonymous namespace)::", "").split("(")[0].split("::")[-1]
            wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"])
            g = (int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]),
                 int(r["Grid_Size_Y"]) // int(r["Workgroup_Size_Y"]))
            acc[(label, g, wg)].append((int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    out = []
    for (label, g, wg), spans in acc.items():
        spans.sort()
        d = sorted((e - s) / 1e3 for s, e in spans)
        block = _longest_block(spans, max_gap_us)
        bd = [(e - s) / 1e3 for s, e in block]
        out.append({"kernel": label, "grid": list(g), "threads": wg, "dispatches": len(d),
                    "mean_us": sum(d) / len(d), "min_us": d[0], "median_us": d[len(d) // 2],
                    "block_dispatches": len(block), "block_mean_us": sum(bd) / len(bd),
                    "block_period_us": (block[-1][1] - block[0][0]) / 1e3 / len(block)})
    return sorted(out, key=lambda r: -r["dispatches"])


def kcfg_of(label: str) -> tuple[tuple, tuple] | None:
    """(chain order, tile fields TT..TP) of a 'ring3<KCfg fields>' label; fields the
    compiler's name leaves out at the end are zero."""
    m = re.fullmatch(r"ring3<([-0-9,]*)>", label)
    if not m:
        return None
    f = [int(v) for v in m.group(1).split(",") if v]
    f += [0] * (27 - len(f))
    return tuple(f[1:4]), tuple(f[11:27])


def cases(trace: Path, details: dict, max_gap_us: float = 30.0) -> list[dict]:
    """Per bench.py case (details["cases"], from the traced run): the kernel of its variant at
    its grid in the trace, with dispatches, mean / min / median duration and the longest
    back-to-back block (grids()), the case's stream time in the same run, and the roofline
    fractions of the trace mean (algorithmic bytes / 8 TB/s, chain-order flops / peak)."""
    import dataclasses

    sys.path.insert(0, str(Path(__file__).resolve().parents[1]))
    from factorized_inference import tilegen

    peaks = {"float16": 2500.0, "bfloat16": 2500.0, "float32": 157.3}
    by_cfg: dict = {}
    for r in grids(trace, max_gap_us):
        key = kcfg_of(r["kernel"])
        if key is not None:
            by_cfg[(key, tuple(r["grid"]))] = r
    out = []
    for c in details["cases"]:
        order, tile = tilegen.parse_variant_name(c["variant"])
        key = ((tuple(order), dataclasses.astuple(tile)), tuple(c["grid"][:2]))
        r = by_cfg.get(key)
        row = {"case": c["case"], "tokens": c["tokens"], "variant": c["variant"],
               "grid": c["grid"][:2], "stream_us": c["ours_stream_us"]}
        if r is not None:
            mean = r["mean_us"]
            row.update({"trace_dispatches": r["dispatches"], "trace_mean_us": mean,
                        "trace_min_us": r["min_us"], "trace_median_us": r["median_us"],
                        "trace_block_dispatches": r["block_dispatches"],
                        "trace_block_mean_us": r["block_mean_us"],
                        "trace_block_period_us": r["block_period_us"],
                        "trace_frac_hbm": c["bytes"] / (mean * 1e-6) / 1e9 / 8000.0,
                        "trace_frac_mfma": c["flops"] / (mean * 1e-6) / 1e12 / peaks[c["dtype"]]})
        out.append(row)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", type=Path, required=True)
    t.add_argument("--write", type=Path, required=True)
    t.add_argument("--algorithmic-bytes", type=float, default=None)
    t.add_argument("--workload", default="")
    t.add_argument("--out", type=Path)
    mp = sub.add_parser("means")
    mp.add_argument("dirs", type=Path, nargs="+")
    bp = sub.add_parser("blocks")
    bp.add_argument("trace", type=Path)
    bp.add_argument("--kernel", required=True, help="regular expression on the kernel name")
    bp.add_argument("--grid", type=int, default=None, help="grid size in threads (x * y)")
    bp.add_argument("--max-gap-us", type=float, default=30.0)
    gp = sub.add_parser("grids")
    gp.add_argument("trace", type=Path)
    gp.add_argument("--out", type=Path)
    cp = sub.add_parser("cases")
    cp.add_argument("trace", type=Path)
    cp.add_argument("details", type=Path)
    cp.add_argument("--out", type=Path)
    args = ap.parse_args()
    if args.cmd == "cases":
        res = {"trace": str(args.trace), "rows": cases(args.trace, json.loads(args.details.read_text()))}
        text = json.dumps(res, indent=1) + "\n"
        if args.out:
            args.out.write_text(text)
        print(text, end="")
        return 0
    if args.cmd == "grids":
        text = json.dumps(grids(args.trace), indent=1) + "\n"
        if args.out:
            args.out.write_text(text)
        else:
            print(text, end="")
        return 0
    if args.cmd == "blocks":
        print(json.dumps(blocks(args.trace, args.kernel, args.grid, args.max_gap_us), indent=1))
        return 0
    if args.cmd == "traffic":
        res = traffic(args.fetch, args.write, args.algorithmic_bytes)
        if args.workload:
            res["workload"] = args.workload
        text = json.dumps(res, indent=1) + "\n"
        if args.out:
            args.out.write_text(text)
        print(text, end="")
        return 0
    merged: dict = {}
    for d in args.dirs:
        m = means(d)
        kernel = probed_kernel(m)
        merged.setdefault(kernel, {}).update({c: v["mean"] for c, v in m[kernel].items()})
    print(json.dumps(merged, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())

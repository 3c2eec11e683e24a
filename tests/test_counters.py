"""The counter summarizer (kernel-task_amd/benchmarks/counters.py) on synthetic rocprofv3 csv
output: calibration against the 512 MiB copy, per-dispatch means, the probed kernel."""
from __future__ import annotations

import csv
import importlib.util
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
spec = importlib.util.spec_from_file_location(
    "counters", ROOT / "kernel-task_amd" / "benchmarks" / "counters.py")
counters = importlib.util.module_from_spec(spec)
spec.loader.exec_module(counters)

RING = ("void trk::(anonymous namespace)::ring3_mfma_kernel<trk::(anonymous namespace)::"
        "KCfg{0, 2, 1, 0, 8, 12, 20, 12, 10, 24, 8, 1, 1, 2, 12, 8, 4, 1, 0, 16, 4}, false>"
        "(unsigned short const*)")


def write_run(d: Path, counter: str, ring_values, copy_values):
    d.mkdir(parents=True)
    with open(d / "p_counter_collection.csv", "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        i = 0
        for v in ring_values:
            i += 1
            w.writerow([i, RING, 30720, counter, v])
        w.writerow([i + 1, "void at::native::vectorized_elementwise_kernel<8>", 6144, counter, 9.0])
        for v in copy_values:
            i += 1
            w.writerow([i, "__amd_rocclr_copyBuffer", 131072, counter, v])


def test_traffic_scales_by_the_copy(tmp_path):
    # FETCH counted at half the copy's bytes (scale 2), WRITE exactly (scale 1)
    write_run(tmp_path / "f", "FETCH_SIZE", [100.0, 102.0], [262144.0] * 5)
    write_run(tmp_path / "w", "WRITE_SIZE", [5.0, 7.0], [524288.0] * 5)
    t = counters.traffic(tmp_path / "f", tmp_path / "w", 1024.0)
    assert t["kernel"].startswith("ring3<0,2,1,0,8,12,20")
    assert t["counters"]["FETCH_SIZE"]["scale"] == pytest.approx(2.0)
    assert t["counters"]["FETCH_SIZE"]["ring_bytes_per_dispatch"] == pytest.approx(101 * 1024 * 2)
    assert t["counters"]["WRITE_SIZE"]["ring_bytes_per_dispatch"] == pytest.approx(6 * 1024)
    assert t["hbm_bytes_per_launch"] == pytest.approx(101 * 2048 + 6 * 1024)
    assert t["ratio_to_algorithmic"] == pytest.approx((101 * 2048 + 6 * 1024) / 1024.0)


def test_means_ignore_other_kernels(tmp_path):
    write_run(tmp_path / "s", "SQ_WAVES", [1536.0, 1536.0, 1536.0], [2048.0])
    m = counters.means(tmp_path / "s")
    assert set(m) == {counters.probed_kernel(m), "copy"}
    assert m[counters.probed_kernel(m)]["SQ_WAVES"] == {"dispatches": 3, "mean": 1536.0}


def write_trace(path: Path, rows):
    """A --kernel-trace csv: rows of (name, grid_x_threads, grid_y, wg_threads, start, end)."""
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Workgroup_Size_X",
                    "Workgroup_Size_Y", "Grid_Size_X", "Grid_Size_Y"])
        for name, gx, gy, wg, s, e in rows:
            w.writerow([name, s, e, wg, 1, gx, gy])


def test_grids_split_one_kernel_by_launch_shape(tmp_path):
    # one kernel at two token counts (grids 240 x 1 and 240 x 16 workgroups), an empty
    # kernel, and a library kernel that is not summarized
    empty = "trk::(anonymous namespace)::ring3_empty_args_kernel(void const*)"
    rows = [(RING, 240 * 256, 1, 256, 0, 3000), (RING, 240 * 256, 1, 256, 5000, 7000),
            (RING, 240 * 256, 16, 256, 9000, 19000), (empty, 64, 1, 64, 20000, 21500),
            ("Cijk_Alik_Bljk_HHS", 64, 1, 64, 22000, 30000)]
    write_trace(tmp_path / "t.csv", rows)
    g = {(r["kernel"], tuple(r["grid"])): r for r in counters.grids(tmp_path / "t.csv")}
    ring = counters.kernel_label(RING)
    assert set(g) == {(ring, (240, 1)), (ring, (240, 16)), ("ring3_empty_args_kernel", (1, 1))}
    one = g[(ring, (240, 1))]
    assert one["dispatches"] == 2 and one["mean_us"] == pytest.approx(2.5)
    assert one["min_us"] == pytest.approx(2.0) and one["threads"] == 256
    assert g[(ring, (240, 16))]["mean_us"] == pytest.approx(10.0)
    assert g[("ring3_empty_args_kernel", (1, 1))]["mean_us"] == pytest.approx(1.5)


def test_blocks_split_at_gaps(tmp_path):
    # 12 back-to-back dispatches, a 100 us gap, 12 more, then 3 isolated ones (too few)
    rows, t = [], 0
    for run in (12, 12):
        for _ in range(run):
            rows.append((RING, 30720, 1, 256, t, t + 3000))
            t += 3500
        t += 100000
    for _ in range(3):
        rows.append((RING, 30720, 1, 256, t, t + 3000))
        t += 200000
    write_trace(tmp_path / "t.csv", rows)
    b = counters.blocks(tmp_path / "t.csv", r"KCfg\{0, 2, 1, 0", grid=30720)
    assert [r["dispatches"] for r in b] == [12, 12]
    assert b[0]["mean_us"] == pytest.approx(3.0) and b[1]["start_us"] > b[0]["start_us"]
    assert counters.blocks(tmp_path / "t.csv", r"KCfg", grid=61440) == []


def test_grids_report_the_longest_back_to_back_block(tmp_path):
    # 3 isolated long dispatches (the tracer's spaced-out calls), then 20 back to back with
    # 2.5 us duration and 3.0 us period: the block figures come from the 20 only
    rows, t = [], 0
    for _ in range(3):
        rows.append((RING, 30720, 1, 256, t, t + 4000))
        t += 100000
    for _ in range(20):
        rows.append((RING, 30720, 1, 256, t, t + 2500))
        t += 3000
    write_trace(tmp_path / "t.csv", rows)
    (r,) = counters.grids(tmp_path / "t.csv")
    assert r["dispatches"] == 23 and r["block_dispatches"] == 20
    assert r["block_mean_us"] == pytest.approx(2.5)
    assert r["block_period_us"] == pytest.approx((19 * 3000 + 2500) / 1e3 / 20)
    assert r["mean_us"] == pytest.approx((3 * 4.0 + 20 * 2.5) / 23)


def test_cases_match_each_bench_case_to_its_kernel_and_grid(tmp_path):
    # the headline case's variant at grid 240 x 1; the same kernel at another grid and an
    # unrelated kernel stay out of its row; a case with no traced kernel keeps its stream time
    rows = [(RING, 240 * 256, 1, 256, 0, 3000), (RING, 240 * 256, 1, 256, 20000, 22000),
            (RING, 240 * 256, 8, 256, 40000, 50000),
            (RING.replace("8, 4, 1, 0, 16, 4}", "8, 4, 1, 0, 16, 8}"), 240 * 512, 1, 512,
             60000, 70000)]
    write_trace(tmp_path / "t.csv", rows)
    details = {"cases": [
        {"case": "r8", "tokens": 1, "variant": "ring3_mfma<210,1,1,2,12,8,4,1>",
         "grid": [240, 1, 1], "ours_stream_us": 3.1, "bytes": 98688.0, "flops": 32.4e6,
         "dtype": "float16"},
        {"case": "r8", "tokens": 32, "variant": "ring3_mfma_wide4x32<210,1,2,10,12,4,2,1>",
         "grid": [120, 32, 1], "ours_stream_us": 5.0, "bytes": 2e5, "flops": 1e9,
         "dtype": "float16"}]}
    head, other = counters.cases(tmp_path / "t.csv", details)
    assert head["trace_dispatches"] == 2 and head["trace_mean_us"] == pytest.approx(2.5)
    assert head["trace_frac_hbm"] == pytest.approx(98688 / 2.5e-6 / 1e9 / 8000)
    assert head["stream_us"] == 3.1
    assert "trace_mean_us" not in other and other["stream_us"] == 5.0
    assert counters.kcfg_of(counters.kernel_label(RING)) == (
        (2, 1, 0), (1, 1, 2, 12, 8, 4, 1, 0, 16, 4, 0, 0, 0, 0, 0, 0))

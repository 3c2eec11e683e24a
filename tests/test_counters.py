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

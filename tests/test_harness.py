"""The benchmark harness CLI (the reference's tests/test_benchmark.py:9-27, ported)."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

SCRIPT = Path(__file__).resolve().parents[1] / "kernel-task_amd" / "benchmarks" / "benchmark.py"


def run_harness(tmp_path, *extra):
    out = tmp_path / "results.json"
    done = subprocess.run([sys.executable, str(SCRIPT), "--input-modes", "2,2,2", "--output-modes",
                           "2,3,2", "--rank", "2", "--tokens", "1", "--warmup", "1",
                           "--iterations", "2", "--output", str(out), *extra],
                          capture_output=True, text=True)
    assert done.returncode == 0, done.stdout + done.stderr
    return json.loads(out.read_text())


def test_cpu_harness_runs_isolated_methods(tmp_path):
    results = run_harness(tmp_path, "--device", "cpu", "--dtype", "float32")
    assert results["schema_version"] == 2
    assert results["spec"]["dense_parameters"] == 96
    methods = results["cases"][0]["methods"]
    assert set(methods) == {"dense", "factorized_reference", "factorized_optimized"}
    assert "unavailable" in methods["factorized_optimized"]   # no CPU fallback of the HIP path
    for name in ("dense", "factorized_reference"):
        res = methods[name]
        assert len(res["host_synchronized_samples_ms"]) == 2
        assert res["cuda_event_stream_median_ms"] is None
        assert res["memory"]["cuda_memory"] is None
        assert res["correctness"]["max_absolute_error"] < 1e-4
    assert methods["dense"]["memory"]["representation_logical_bytes"] == 96 * 4
    assert methods["factorized_reference"]["memory"]["representation_logical_bytes"] == 56 * 4


@pytest.mark.gpu
def test_gpu_harness_runs_every_method(tmp_path):
    results = run_harness(tmp_path, "--device", "cuda", "--dtype", "float16")
    methods = results["cases"][0]["methods"]
    for name in ("dense", "factorized_reference", "factorized_optimized"):
        res = methods[name]
        assert res["cuda_event_stream_median_ms"] > 0
        assert res["correctness"]["max_absolute_error"] < 2e-2
        assert res["memory"]["steady_peak_allocated_bytes"] > 0
    assert methods["factorized_optimized"]["kernel"]["variant"].startswith("ring3_")

"""bench.py's driver line, built on the CPU from synthetic case records: it stays under the
size the driver's stdout capture keeps whole, carries the headline, roofline and CPU baseline
fields the contract names, and is the last line on stdout."""
from __future__ import annotations

import importlib.util
import json
import os

import pytest

from conftest import ROOT


@pytest.fixture(scope="module")
def bench():
    saved = dict(os.environ)
    try:
        spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
    finally:  # importing bench.py sets HIP_FORCE_DEV_KERNARG for its own process only
        os.environ.clear()
        os.environ.update(saved)
    return mod


def synthetic_case(label, tokens, i):
    return {
        "case": label, "tokens": tokens, "rank": 16, "dtype": "bfloat16",
        "modes": [[16, 28, 32], [16, 16, 16]],
        "variant": f"ring3_mfma_wide8x32w8p2_s4_x4<210,{i},2,10,12,4,2,1>#{i}",
        "grid": [240, 12, 1], "lds_bytes": 65536, "ours_stream_us": 3.123456789 + i,
        "dense_stream_us": 19.87654321, "speedup_vs_dense": 6.123456, "ours_host_us": 12.3456,
        "dense_host_us": 31.23456, "ours_submit_us": 2.4567, "flops": 39813120.0 * tokens,
        "bytes": 98688.0 + 9600.0 * tokens, "max_abs_err_vs_fp32": 0.0012345678,
        "max_abs_ref": 3.98765, "prepare_ms": 12.3456, "packed_bytes": 942080,
        "prepare_held_bytes": 942080, "prepare_peak_bytes": 1234567, "call_extra_bytes": 0,
        "dense_weight_bytes": 117440512, "passed": True, "achieved_GBps": 31.5987654,
        "frac_hbm": 0.0039498765, "achieved_TFLOPs": 12.7654321, "frac_mfma": 0.005106172,
        "reference_flops": 55296000.0, "frac_mfma_reference_flops": 0.0070912345,
    }


def synthetic_inputs():
    labels = [("r8", t) for t in (1, 8, 32)] + [("r16", t) for t in (1, 32)]
    labels += [("llama_up_r8", t) for t in (1, 8, 32, 128)]
    labels += [("llama_down_r16", t) for t in (1, 32, 256)]
    labels += [("r8_fp32", t) for t in (1, 8, 32)]
    cases = [synthetic_case(lbl, t, i) for i, (lbl, t) in enumerate(labels)]
    floors = {"host_empty_c_call_us": 0.0712, "host_empty_launch_us": 1.8765,
              "stream_empty_launch_us": 1.6012, "host_empty_launch_args_us": 2.0123,
              "stream_empty_launch_args_us": 2.6789, "stream_handle": True}
    cpu = {"value": 313.456, "unit": "us/call", "cores": 16, "kind": "port",
           "sample": "config 1 (1920->2880, R8, fp32, T=1, per-core sigma, seed 0): median of "
                     "12345 calls of tr_forward_reference on the CPU (the reference's three "
                     "contractions in its order, torch CPU BLAS, 16 threads)",
           "torch_reference_path_us": {str(n): {"us": 500.0 / n, "calls": 1000}
                                       for n in (1, 2, 4, 8, 16)},
           "oracle_port_us": 339.123, "oracle_port_calls": 29000, "oracle_port_threads": 1,
           "host_threads": 16,
           "cpu_model": "AMD EPYC 9575F 64-Core Processor (family 26, model 2, stepping 1)"}
    xcd = {"variant": "ring3_mfma_w8_xl<210,1,1,10,12,8,4,1>", "value": 3.4123,
           "default_variant": cases[0]["variant"], "default_value": 3.2123, "unit": "us/call",
           "protocol": "median of 9 blocks of 20 calls, alternating with the default",
           "passed": True, "max_abs_err_vs_fp32": 0.0015, "traffic": 174000,
           "traffic_kernel": "x", "traffic_ratio_to_algorithmic": 1.76}
    runtime = {"value": 4.81, "median_of_9_blocks": 5.2, "submit_us": 4.5, "passed": True,
               "hip_force_dev_kernarg": None}
    return cases, floors, xcd, cpu, runtime


def test_line_fits_the_driver_capture_and_carries_the_contract_fields(bench):
    cases, floors, xcd, cpu, runtime = synthetic_inputs()
    assert len(cases) == 15
    line = bench.build_line(20, 5, cases, floors, xcd, cpu, runtime, 281361,
                            "gpurun_out/bench_details.json", 8000.0)
    text = json.dumps(line)
    assert len(text) < 8000
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step",
                "higher_is_better", "scaling", "vs_baseline", "dtype", "data", "config",
                "roofline", "cpu_baseline"):
        assert key in line, key
    assert line["value"] == cases[0]["ours_stream_us"] and line["steps"] == 20
    assert "workload" in line["config"]
    roof = line["roofline"]
    assert {"bound", "achieved", "peak", "unit", "frac", "traffic"} <= set(roof)
    assert roof["frac"] == pytest.approx(roof["achieved"] / roof["peak"])
    assert {"value", "unit", "cores", "kind", "sample"} <= set(line["cpu_baseline"])
    # one row per case, in the declared columns
    cols = line["case_columns"]
    assert len(line["cases"]) == 15 and all(len(r) == len(cols) for r in line["cases"])
    row = dict(zip(cols, line["cases"][4]))
    assert row["case"] == "r16" and row["T"] == 32 and row["extra_bytes"] == 0
    assert row["ours_us"] == pytest.approx(cases[4]["ours_stream_us"], rel=1e-2)
    assert row["host_us"] == pytest.approx(cases[4]["ours_host_us"], rel=1e-2)
    # host latency and preparation cost of the headline operator
    assert line["host_us"] == cases[0]["ours_host_us"]
    assert line["prepare"]["ms"] == cases[0]["prepare_ms"]
    assert line["prepare"]["peak_bytes"] == cases[0]["prepare_peak_bytes"]


def test_line_sheds_optional_fields_before_exceeding_the_limit(bench):
    cases, floors, xcd, cpu, runtime = synthetic_inputs()
    for c in cases:  # very long variant names
        c["variant"] = c["variant"] * 12
    line = bench.build_line(20, 5, cases, floors, xcd, cpu, runtime, None, None, 8000.0)
    assert len(json.dumps(line)) < 8000
    assert "roofline" in line and "cpu_baseline" in line and line["value"] > 0


def test_emit_prints_one_line_last(bench, capsys):
    cases, floors, xcd, cpu, runtime = synthetic_inputs()
    print("stdout before the line")
    bench.emit(bench.build_line(20, 5, cases, floors, xcd, cpu, runtime, None, None, 8000.0))
    out = capsys.readouterr().out.splitlines()
    assert json.loads(out[-1])["n_gpus"] == 1
    assert out[-1] == out[-1].strip() and len(out) == 2


def test_traffic_figure_only_for_the_variant_it_was_measured_on(bench):
    data = json.loads((ROOT / "profiles" / "traffic_r8_t1.json").read_text())
    measured = data["workload"].split("(", 1)[1].split(":", 1)[0]
    assert bench.traffic_figure(measured) == data["hbm_bytes_per_launch"]
    assert bench.traffic_figure(measured.replace("ring3_mfma", "ring3_mfma_other")) is None

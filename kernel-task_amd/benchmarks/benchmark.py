"""Per-method benchmark of the tensor-ring operator, one fresh interpreter per case.

Measures what the reference's harness measures (benchmarks/benchmark.py:78-286; its CLI
flags and its JSON schema 2 are the interface kept here) for the three methods: the dense
GEMM on the materialised weight, the reference's factorized path and the HIP operator.
Per (method, token count) case, in an interpreter of its own:
  preparation and first call   host wall clock, synchronized
  host latency                 `--iterations` synchronized single calls after `--warmup`
  stream latency               5 HIP-event blocks of `--event-block` back-to-back calls
  memory                       torch allocator counters around preparation and the calls
  correctness                  after timing, against a float32 dense oracle rebuilt from
                               freshly drawn (pristine) cores of the same seed
  profile (optional)           a torch.profiler trace of 3 calls at tokens = 1

Additions to the reference's flags: `--dtype bfloat16`, `--init uniform` (the benchmark
configs' sigma). On a CPU device the HIP method is recorded as unavailable: the operator
has no CPU path.

    python kernel-task_amd/benchmarks/benchmark.py --device cuda --dtype float16 --rank 8 \\
        --tokens 1,8,32 --output results.json
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import multiprocessing as mp
import os
import platform
import statistics
import subprocess
import sys
import time
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parents[1]
if str(PACKAGE_ROOT) not in sys.path:
    sys.path.insert(0, str(PACKAGE_ROOT))

METHODS = ("dense", "factorized_reference", "factorized_optimized")
TOLERANCE = {"float16": 2e-2, "bfloat16": 2e-2, "float32": 1e-4}
NOTES = [
    "Each method/token case runs in a fresh interpreter (multiprocessing spawn).",
    "Host timing includes dispatch and synchronization; HIP events measure block stream time.",
    "Memory is the PyTorch allocator's; the HIP operator allocates nothing outside it.",
    "Correctness is checked after measurement against an fp32 dense oracle.",
]


@dataclasses.dataclass(frozen=True)
class Case:
    """Everything one isolated measurement needs (picklable, sent to the child as is)."""
    method: str
    tokens: int
    device: str
    dtype: str
    input_modes: tuple
    output_modes: tuple
    rank: int
    init: str
    seed: int
    warmup: int
    iterations: int
    event_block: int
    cpu_threads: int
    profile_dir: str | None


# ---- what each method prepares (the dense W exists only in the dense method) ------------
def _prepare_dense(spec, cores):
    from factorized_inference import dense_forward, materialize_dense_weight

    weight = materialize_dense_weight(cores, spec)
    return (lambda v: dense_forward(v, weight)), weight.numel() * weight.element_size(), None


def _prepare_reference(spec, cores):
    from factorized_inference import tr_forward_reference

    size = sum(c.numel() * c.element_size() for c in cores)
    return (lambda v: tr_forward_reference(v, cores, spec)), size, None


def _prepare_optimized(spec, cores):
    from factorized_inference import prepare_optimized

    run = prepare_optimized(cores, spec)
    size = sum(c.numel() * c.element_size() for c in cores)
    return run, size, run


PREPARE = {"dense": _prepare_dense, "factorized_reference": _prepare_reference,
           "factorized_optimized": _prepare_optimized}


def _environment(torch, device, case: Case) -> dict:
    on_gpu = device.type == "cuda"
    smi = None
    if on_gpu:
        try:
            smi = subprocess.run(["rocm-smi", "--showproductname"], capture_output=True,
                                 text=True, timeout=10).stdout.strip() or "unavailable"
        except (OSError, subprocess.SubprocessError):
            smi = "unavailable"
    props = torch.cuda.get_device_properties(device) if on_gpu else None
    return {
        "python": sys.version, "platform": platform.platform(), "cpu": platform.processor(),
        "cpu_count": os.cpu_count(), "torch": torch.__version__,
        "hip_runtime": getattr(torch.version, "hip", None), "rocm_smi": smi,
        "device": str(device), "device_name": props.name if props else "CPU",
        "gcn_arch": props.gcnArchName if props else None,
        "dtype": case.dtype, "init": case.init, "cpu_threads": torch.get_num_threads(),
    }


class _Allocator:
    """Allocator snapshots on a ROCm device (None on the CPU)."""

    def __init__(self, torch, device):
        self.torch, self.device = torch, device
        self.on = device.type == "cuda"

    def allocated(self):
        return self.torch.cuda.memory_allocated(self.device) if self.on else None

    def peak(self):
        return self.torch.cuda.max_memory_allocated(self.device) if self.on else None

    def reset_peak(self):
        if self.on:
            self.torch.cuda.reset_peak_memory_stats(self.device)


def measure(case: Case) -> dict:
    """One isolated case (runs in the child interpreter)."""
    import torch

    from factorized_inference import TRSpec, dense_forward, make_cores, materialize_dense_weight
    from factorized_inference import measure as m

    device = torch.device(case.device)
    if device.type == "cuda":
        device = torch.device("cuda", device.index if device.index is not None
                              else torch.cuda.current_device())
        torch.cuda.set_device(device)
    torch.set_num_threads(case.cpu_threads)
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    on_gpu = device.type == "cuda"
    result = {"method": case.method, "tokens": case.tokens,
              "environment": _environment(torch, device, case)}
    if case.method == "factorized_optimized" and not on_gpu:
        return {**result, "unavailable": "the HIP operator needs a ROCm GPU"}

    def sync():
        if on_gpu:
            torch.cuda.synchronize(device)

    def wall_ms(fn):
        sync()
        t0 = time.perf_counter_ns()
        out = fn()
        sync()
        return out, (time.perf_counter_ns() - t0) / 1e6

    dtype = getattr(torch, case.dtype)
    spec = TRSpec(case.input_modes, case.output_modes, case.rank)
    mem = _Allocator(torch, device)
    with torch.inference_mode():
        torch.empty(1, device=device)      # context first, so the baseline excludes it
        sync()
        if on_gpu:
            torch.cuda.empty_cache()
        base = mem.allocated()
        mem.reset_peak()
        cores = make_cores(spec, device=device, dtype=dtype, seed=case.seed, init=case.init)
        x = torch.randn(case.tokens, spec.in_features, dtype=dtype, device=device,
                        generator=torch.Generator(device=device).manual_seed(case.seed + case.tokens))
        (fn, representation, prepared), prep_ms = wall_ms(lambda: PREPARE[case.method](spec, cores))
        if case.method == "dense":
            del cores                      # the dense method keeps only its weight
        call = lambda: fn(x)  # noqa: E731
        _, first_ms = wall_ms(call)
        for _ in range(case.warmup):
            call()
        sync()
        x_bytes = x.numel() * x.element_size()
        setup_peak, resident = mem.peak(), mem.allocated()
        mem.reset_peak()
        host = [t / 1000.0 for t in m.host_us(call, case.iterations, sync=sync)]
        steady_peak = mem.peak()
        stream = ([t / 1000.0 for t in m.stream_us(call, case.event_block, blocks=5)]
                  if on_gpu else [])
        # correctness after timing: fp32 dense oracle from cores drawn again from the seed
        pristine = make_cores(spec, device=device, dtype=dtype, seed=case.seed, init=case.init)
        oracle = dense_forward(x.float(), materialize_dense_weight(
            tuple(c.float() for c in pristine), spec))
        got = call().float()
        tol = TOLERANCE[case.dtype]
        torch.testing.assert_close(got, oracle, rtol=tol, atol=tol)
        diff = (got - oracle).abs()
        ref_max = oracle.abs().max().item()
        correctness = {
            "rtol": tol, "atol": tol,
            "max_absolute_error": diff.max().item(), "mean_absolute_error": diff.mean().item(),
            "relative_l2_error": (diff.norm() / oracle.norm().clamp_min(1e-12)).item(),
            "max_abs_over_max_ref": diff.max().item() / max(ref_max, 1e-12),
        }
        trace = None
        if case.profile_dir and case.tokens == 1:
            trace = Path(case.profile_dir) / f"{case.method}_rank{case.rank}_tokens1.json"
            trace.parent.mkdir(parents=True, exist_ok=True)
            activities = [torch.profiler.ProfilerActivity.CPU]
            if on_gpu:
                activities.append(torch.profiler.ProfilerActivity.CUDA)
            with torch.profiler.profile(activities=activities, record_shapes=True) as prof:
                for _ in range(3):
                    with torch.profiler.record_function(case.method):
                        call()
                sync()
            prof.export_chrome_trace(str(trace))

    if on_gpu:
        memory = {
            "context_baseline_allocated_bytes": base,
            "input_logical_bytes": x_bytes,
            "representation_logical_bytes": representation,
            "resident_after_warmup_allocated_bytes": resident,
            "extra_resident_allocated_bytes": max(0, resident - base - x_bytes - representation),
            "preparation_and_warmup_peak_allocated_bytes": setup_peak,
            "steady_peak_allocated_bytes": steady_peak,
            "incremental_workspace_and_output_bytes": steady_peak - resident,
            "steady_peak_reserved_bytes": torch.cuda.max_memory_reserved(device),
        }
    else:
        memory = {"input_logical_bytes": x_bytes, "representation_logical_bytes": representation,
                  "cuda_memory": None}
    kernel = None
    if prepared is not None:
        info = prepared.selected(case.tokens)
        kernel = {"variant": info["name"], "grid": info["grid"], "lds_bytes": info["lds_bytes"],
                  "packed_bytes": prepared.packed_bytes, "flops": info["flops"],
                  "compulsory_bytes": info["bytes"]}
    return {
        **result, "preparation_ms": prep_ms, "first_call_ms": first_ms,
        "host_synchronized_median_ms": statistics.median(host),
        "host_synchronized_samples_ms": host,
        "cuda_event_stream_median_ms": statistics.median(stream) if stream else None,
        "cuda_event_stream_samples_ms": stream,
        "memory": memory, "correctness": correctness, "kernel": kernel,
        "profiler_trace": str(trace) if trace else None,
    }


def _child(case: Case, queue) -> None:
    try:
        queue.put(("ok", measure(case)))
    except BaseException as exc:  # reported to the parent, which fails the run
        queue.put(("error", f"{type(exc).__name__}: {exc}"))


def run_isolated(case: Case) -> dict:
    """measure(case) in a fresh interpreter; raises if the child fails."""
    ctx = mp.get_context("spawn")
    queue = ctx.Queue()
    proc = ctx.Process(target=_child, args=(case, queue))
    proc.start()
    status, payload = queue.get()
    proc.join()
    if status != "ok" or proc.exitcode != 0:
        raise RuntimeError(f"{case.method} tokens={case.tokens} failed: {payload}")
    return payload


def _modes(text: str) -> tuple:
    try:
        modes = tuple(int(v) for v in text.split(","))
    except ValueError:
        modes = ()
    if len(modes) != 3 or min(modes) < 1:
        raise argparse.ArgumentTypeError("Use three positive integers")
    return modes


def parse_args(argv=None):
    from factorized_inference import TRSpec

    default = TRSpec()
    ap = argparse.ArgumentParser(description="Isolated per-method tensor-ring benchmark")
    ap.add_argument("--device", default="cuda")
    ap.add_argument("--dtype", choices=tuple(TOLERANCE), default="float16")
    ap.add_argument("--input-modes", type=_modes, default=default.input_modes)
    ap.add_argument("--output-modes", type=_modes, default=default.output_modes)
    ap.add_argument("--rank", type=int, default=8)
    ap.add_argument("--init", choices=("per_core", "uniform"), default="per_core")
    ap.add_argument("--tokens", default="1,8,32")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--iterations", type=int, default=100)
    ap.add_argument("--event-block", type=int, default=20)
    ap.add_argument("--cpu-threads", type=int, default=1)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--output", type=Path, default=Path("benchmark_results.json"))
    ap.add_argument("--profile-dir", type=Path)
    args = ap.parse_args(argv)
    positive = ("rank", "warmup", "iterations", "event_block", "cpu_threads")
    if any(getattr(args, name) < 1 for name in positive):
        ap.error("rank, warmup, iterations, event-block and cpu-threads must be positive")
    if args.device.startswith("cpu") and args.dtype != "float32":
        ap.error("use float32 on the CPU")
    try:
        args.token_counts = [int(t) for t in args.tokens.split(",")]
    except ValueError:
        args.token_counts = []
    if not args.token_counts or min(args.token_counts) < 1:
        ap.error("tokens must be comma-separated positive integers")
    return args


def main(argv=None) -> None:
    from factorized_inference import TRSpec

    args = parse_args(argv)
    spec = TRSpec(args.input_modes, args.output_modes, args.rank)
    report = {
        "schema_version": 2,
        "spec": {"input_modes": spec.input_modes, "output_modes": spec.output_modes,
                 "rank": spec.rank, "dense_parameters": spec.dense_parameters,
                 "factor_parameters": spec.factor_parameters},
        "settings": {k: (str(v) if isinstance(v, Path) else v) for k, v in vars(args).items()
                     if k != "token_counts"},
        "measurement_notes": NOTES,
        "cases": [],
    }
    for tokens in args.token_counts:
        methods = {}
        for method in METHODS:
            case = Case(method, tokens, args.device, args.dtype, tuple(args.input_modes),
                        tuple(args.output_modes), args.rank, args.init, args.seed, args.warmup,
                        args.iterations, args.event_block, args.cpu_threads,
                        str(args.profile_dir.resolve()) if args.profile_dir else None)
            res = run_isolated(case)
            methods[method] = res
            if "unavailable" in res:
                print(f"tokens={tokens} {method}: {res['unavailable']}", flush=True)
            else:
                stream = res["cuda_event_stream_median_ms"]
                print(f"tokens={tokens} {method}: host={res['host_synchronized_median_ms']:.4f} ms; "
                      f"stream={'N/A' if stream is None else f'{stream:.4f}'} ms", flush=True)
        report["cases"].append({"tokens": tokens, "methods": methods})
    args.output.parent.mkdir(parents=True, exist_ok=True)
    args.output.write_text(json.dumps(report, indent=2) + "\n")
    print(f"Wrote {args.output}")


if __name__ == "__main__":
    main()

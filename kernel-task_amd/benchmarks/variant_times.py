"""Per-variant timing of one operator shape: every MFMA variant of the plan, launched through
trk_forward_variant at the given token counts, in one process (so that variants compare on
the same GPU clocks and caches), with each output checked against the default variant's.

    python kernel-task_amd/benchmarks/variant_times.py --case r16 --tokens 32 64
    python kernel-task_amd/benchmarks/variant_times.py --case llama_up_r8 --tokens 128 --out t.json

Cases are bench.py's (label, modes, rank, dtype). Time per call: HIP events around blocks of
400 back-to-back launches on the current stream, median of 5 blocks after 300 untimed
launches. The launches go through the CPython fast-call binding, whose host cost (~1-2 us a
call) stays below the kernels timed here. The default variant (trk_plan_select) is marked *.

This is how the variants of a table are compared in isolation. The tuned tables come from
benchmarks/autotune.py, which times tiles the same way through the per-call path of
bench.py.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
from pathlib import Path

os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "0")  # as bench.py
PACKAGE_ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(PACKAGE_ROOT))

import torch  # noqa: E402

from factorized_inference import TRSpec, make_cores, prepare_optimized  # noqa: E402
from factorized_inference.tr_kernel import _fast_forward  # noqa: E402

CASES = {  # bench.py's cases: modes, rank, dtype, init
    "r8": ((8, 12, 20), (12, 10, 24), 8, torch.float16, "per_core"),
    "r16": ((8, 12, 20), (12, 10, 24), 16, torch.float16, "per_core"),
    "llama_up_r8": ((16, 16, 16), (16, 28, 32), 8, torch.bfloat16, "uniform"),
    "llama_down_r16": ((16, 28, 32), (16, 16, 16), 16, torch.bfloat16, "uniform"),
    "r8_fp32": ((8, 12, 20), (12, 10, 24), 8, torch.float32, "per_core"),
}


def block_us(fn, calls: int = 400, blocks: int = 5) -> float:
    out = []
    for _ in range(blocks):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(calls):
            fn()
        b.record()
        b.synchronize()
        out.append(a.elapsed_time(b) * 1000.0 / calls)
    return statistics.median(out)


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--case", required=True, choices=sorted(CASES))
    ap.add_argument("--tokens", type=int, nargs="+", required=True)
    ap.add_argument("--out", type=Path, default=None, help="also write the timings as JSON")
    args = ap.parse_args()
    if not torch.cuda.is_available():
        print("variant_times.py needs a ROCm GPU", file=sys.stderr)
        return 1
    ins, outs, rank, dtype, init = CASES[args.case]
    spec = TRSpec(ins, outs, rank)
    cores = make_cores(spec, device="cuda", dtype=dtype, seed=0, init=init)
    run = prepare_optimized(cores, spec)
    _, forward_variant, _ = _fast_forward()
    stream = torch.cuda.current_stream().cuda_stream
    result = {}
    for tokens in args.tokens:
        x = torch.randn(tokens, spec.in_features, device="cuda", dtype=dtype,
                        generator=torch.Generator(device="cuda").manual_seed(tokens))
        default = run.plan.select(tokens)
        ref = run.run_variant(x, default).float()
        scale = ref.abs().max().item()
        rows = {}
        for i, info in enumerate(run.variants(tokens)):
            if info["kind"] != "mfma":
                continue
            y = torch.empty(tokens, spec.out_features, device="cuda", dtype=dtype)
            fn = lambda i=i, y=y: forward_variant(run.plan.handle, i, run.packed.data_ptr(),  # noqa: E731
                                                  x.data_ptr(), y.data_ptr(), tokens, stream)
            if fn() != 0:
                continue
            torch.cuda.synchronize()
            diff = (y.float() - ref).abs().max().item() / scale
            for _ in range(300):
                fn()
            torch.cuda.synchronize()
            us = block_us(fn)
            rows[info["name"]] = {"us": us, "grid": info["grid"][:2], "lds_bytes": info["lds_bytes"],
                                  "max_diff_to_default": diff, "default": i == default}
            print(f"{args.case} T={tokens:4d} {i:3d}{'*' if i == default else ' '} "
                  f"{info['name']:56s} grid={info['grid'][:2]} {us:8.2f} us  "
                  f"diff {diff:.1e}", flush=True)
        result[tokens] = rows
    if args.out is not None:
        args.out.parent.mkdir(parents=True, exist_ok=True)
        args.out.write_text(json.dumps(result, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""The operator on the Qwen3.8-27B layer shapes (bf16, ranks 8 and 16): ours vs the dense GEMM.

    python kernel-task_amd/benchmarks/qwen_bench.py --out qwen.json [--tokens 1,8,32,128]
        [--dtype bfloat16|float16] [--ranks 8,16]

The library carries tuned MFMA tables for these shapes in bf16 at ranks 8 and 16. Other
dtypes and ranks (fp16; rank 12, which runs the rank-16 kernels on zero-padded links) get
the variant modules built at prepare time (factorized_inference/jit.py; TRK_JIT=0 runs the
generic kernel instead, for comparison). Each row records which kind of plan served it.

Role of the reference's tools/qwen_bench.py (shapes from tools/qwen_shapes.py:20-27, bf16,
seed 0, harness protocol): per shape, rank and token count, the HIP-event stream latency of
the prepared operator (the generated, autotuned MFMA tables) and of F.linear on the
materialised weight, timed the same way in one process, with the relative L2 error of
both against an fp64 dense product on a subset of token rows, and the algorithmic rates
(flops of the contraction order the kernel runs, compulsory bytes).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "0")  # as bench.py
PACKAGE_ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(PACKAGE_ROOT))

import torch  # noqa: E402

from factorized_inference import (  # noqa: E402
    TRSpec, dense_forward, make_cores, materialize_dense_weight, prepare_optimized, tilegen,
)

PEAK_TFLOPS, PEAK_GBS = 2500.0, 8000.0


def stream_us(fn, calls: int, blocks: int = 5) -> float:
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


def calls_for(fn) -> int:
    fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    fn()
    torch.cuda.synchronize()
    one = (time.perf_counter() - t0) * 1e6
    return max(5, min(100, int(3e3 / max(one, 1.0))))


def rel_l2(y, ref) -> float:
    d = y.double() - ref
    return (d.norm() / ref.norm()).item()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", type=Path, required=True)
    ap.add_argument("--tokens", default="1,8,32,128")
    ap.add_argument("--dtype", default="bfloat16", choices=("bfloat16", "float16"))
    ap.add_argument("--ranks", default="8,16")
    args = ap.parse_args()
    dtype = getattr(torch, args.dtype)
    ranks = [int(r) for r in args.ranks.split(",")]
    if not torch.cuda.is_available():
        print("qwen_bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    tokens = [int(t) for t in args.tokens.split(",")]
    torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    rows = []
    shapes = [tilegen.ShapeDecl(f"qwen_{name}", ins, outs, rank)
              for name, (ins, outs) in tilegen.QWEN.items() for rank in ranks]
    with torch.inference_mode():
        for shape in shapes:
            spec = TRSpec(shape.ins, shape.outs, shape.rank)
            cores = make_cores(spec, device="cuda", dtype=dtype, seed=0)
            t0 = time.perf_counter()
            run = prepare_optimized(cores, spec)
            torch.cuda.synchronize()
            prepare_ms = (time.perf_counter() - t0) * 1e3
            w = materialize_dense_weight(cores, spec)
            w64 = materialize_dense_weight([c.double() for c in cores], spec)
            for T in tokens:
                x = torch.randn(T, spec.in_features, device="cuda", dtype=dtype,
                                generator=torch.Generator(device="cuda").manual_seed(T))
                ours = lambda: run(x)  # noqa: E731
                dense = lambda: dense_forward(x, w)  # noqa: E731
                ours_us = stream_us(ours, calls_for(ours))
                dense_us = stream_us(dense, calls_for(dense))
                sub = x[: min(T, 8)]
                ref = sub.double() @ w64.T
                info = run.selected(T)
                row = {"shape": shape.name, "key": shape.key, "rank": shape.rank, "tokens": T,
                       "dtype": args.dtype, "kernel_rank": run.plan.kernel_rank,
                       "modules": run.plan.modules, "kind": info["kind"],
                       "prepare_ms": prepare_ms,
                       "in_features": spec.in_features, "out_features": spec.out_features,
                       "variant": info["name"], "ours_us": ours_us, "dense_us": dense_us,
                       "dense_over_ours": dense_us / ours_us,
                       "ours_tflops": info["flops"] / ours_us / 1e6,
                       "ours_frac_mfma": info["flops"] / ours_us / 1e6 / PEAK_TFLOPS,
                       "dense_gbs": 2 * spec.in_features * spec.out_features / dense_us / 1e3,
                       "rel_l2_ours": rel_l2(run(sub), ref),
                       "rel_l2_dense": rel_l2(dense_forward(sub, w), ref)}
                rows.append(row)
                print(f"{shape.name:18s} R{shape.rank:2d} T{T:4d}: ours {ours_us:8.2f} us  dense "
                      f"{dense_us:8.2f} us  ({row['dense_over_ours']:.2f}x)  relL2 "
                      f"{row['rel_l2_ours']:.1e} / {row['rel_l2_dense']:.1e}  {info['name']}",
                      flush=True)
            del run, w, w64
            torch.cuda.empty_cache()
    args.out.parent.mkdir(parents=True, exist_ok=True)
    args.out.write_text(json.dumps({"device": torch.cuda.get_device_name(0),
                                    "trk_jit": os.environ.get("TRK_JIT", "1"), "rows": rows},
                                   indent=1) + "\n")
    print(f"wrote {args.out}", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Measurements beyond single uncaptured calls: HIP graphs, chains of distinct layers, cold
caches and a SwiGLU MLP block with fused epilogues. One MI355X.

    python kernel-task_amd/benchmarks/graph_bench.py --part single --out single.json
    python kernel-task_amd/benchmarks/graph_bench.py --part chain  --out chain.json
    python kernel-task_amd/benchmarks/graph_bench.py --part cold   --out cold.json
    python kernel-task_amd/benchmarks/graph_bench.py --part mlp    --out mlp.json

Role of the reference's tools/graph_bench.py (:1-27, parts single / chain / cold) and
tools/v3g_fp32out.py (the MLP block with fp32-output consumers), measured the same way:
HIP events around a block of calls, median of repetitions.

Parts:
  single  every BASELINE case, ours and the dense GEMM: G back-to-back eager calls, and the
          same G calls captured in one HIP graph and replayed. The captured output is
          checked against an fp64 dense reference after the timed replays.
  chain   L distinct operators (different weights) applied one after another on one stream,
          eager and captured, per-layer us. With L = 128 the dense weights (11 MB each,
          1.4 GB) exceed the 256 MB Infinity Cache; the ring's packed cores (0.2-0.9 MB
          each) still fit.
  cold    one call after a 1 GiB read-modify-write that evicts the L2s and the Infinity
          Cache, timed by HIP events around the call only, next to the warm call (after a
          bounded spin kernel instead of the flush). Both calls are queued behind the busy
          GPU, so the events time the call's GPU work without the host's launch latency.
  mlp     h + down(silu(gate(x)) * up(x)) with the Llama-3-8B shapes (gate/up 4096->14336
          rank 8, down 14336->4096 rank 16, bf16), one block and a chain of 8 blocks:
            unfused  gate, up, down, then torch silu, mul and the residual add
            consume  accumulate() x3 with the standalone consumers (the reference's
                     fp32-output chain, consume_silu_mul / consume_add)
            fused    gate.accumulate, up.forward_silu_mul, down.forward_add: 3 launches
            dense    the same block on the materialised weights (F.linear)
          eager and captured; outputs checked against an fp64 reference of the block.
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
from pathlib import Path

os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "0")  # as bench.py: kernel arguments in host memory
PACKAGE_ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(PACKAGE_ROOT))

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

from factorized_inference import (  # noqa: E402
    TRSpec, dense_forward, make_cores, materialize_dense_weight, prepare_optimized,
)
from factorized_inference.tr_kernel import consume_add, consume_silu_mul  # noqa: E402

DEFAULT = ((8, 12, 20), (12, 10, 24))
LLAMA_UP = ((16, 16, 16), (16, 28, 32))
LLAMA_DOWN = ((16, 28, 32), (16, 16, 16))
CASES = [  # (label, modes, rank, dtype, init, tokens)
    ("r8", DEFAULT, 8, torch.float16, "per_core", (1, 8, 32)),
    ("r16", DEFAULT, 16, torch.float16, "per_core", (1, 32)),
    ("llama_up_r8", LLAMA_UP, 8, torch.bfloat16, "uniform", (1, 8, 32, 128)),
    ("llama_down_r16", LLAMA_DOWN, 16, torch.bfloat16, "uniform", (1, 32, 256)),
]
MIB = 1 << 20


def log(msg: str) -> None:
    print(msg, flush=True)


def events_us(run, n_inner: int, reps: int = 7) -> float:
    """HIP events around run() (n_inner calls); us per call, median of reps."""
    for _ in range(2):
        run()
    torch.cuda.synchronize()
    out = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        run()
        e.record()
        e.synchronize()
        out.append(s.elapsed_time(e) * 1000.0 / n_inner)
    return statistics.median(out)


def capture(body):
    """Warm body up on a side stream, then capture it in one HIP graph; returns (graph,
    what the captured body returned)."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            body()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = body()
    torch.cuda.synchronize()
    return graph, out


def reference64(x, cores, spec):
    w = materialize_dense_weight([c.double() for c in cores], spec)
    return x.double() @ w.T


def err(y, ref) -> dict:
    d = (y.double() - ref).abs()
    return {"max_abs": d.max().item(),
            "rel_l2": (d.norm() / ref.norm().clamp_min(1e-30)).item(),
            "within_tol": bool((d <= 0.02 + 0.02 * ref.abs()).all())}


def make_method(method: str, cores, spec):
    if method == "dense":
        w = materialize_dense_weight(cores, spec)
        return lambda x: dense_forward(x, w)  # noqa: E731
    return prepare_optimized(cores, spec)


# ---------------------------------------------------------------------------------- single
def part_single(G: int = 20) -> list:
    rows = []
    for label, (ins, outs), R, dtype, init, tokens in CASES:
        spec = TRSpec(ins, outs, R)
        cores = make_cores(spec, device="cuda", dtype=dtype, seed=0, init=init)
        for m in ("ours", "dense"):
            fn = make_method(m, cores, spec)
            for T in tokens:
                x = torch.randn(T, spec.in_features, device="cuda", dtype=dtype,
                                generator=torch.Generator(device="cuda").manual_seed(T))

                def eager():
                    for _ in range(G):
                        fn(x)

                def body():
                    y = None
                    for _ in range(G):
                        y = fn(x)
                    return y

                eager_us = events_us(eager, G)
                graph, y_static = capture(body)
                graph_us = events_us(graph.replay, G)
                graph.replay()
                torch.cuda.synchronize()
                e = err(y_static, reference64(x, cores, spec))
                rows.append({"case": label, "rank": R, "tokens": T, "method": m,
                             "dtype": str(dtype).replace("torch.", ""), "calls_per_graph": G,
                             "eager_us_per_call": eager_us, "graph_us_per_call": graph_us,
                             "graph_output_error": e})
                log(f"single {label:15s} T={T:3d} {m:5s} eager {eager_us:8.2f}  graph "
                    f"{graph_us:8.2f} us/call  max|err| {e['max_abs']:.2e} "
                    f"{'ok' if e['within_tol'] else 'FAIL'}")
                del graph, y_static
            del fn
            torch.cuda.empty_cache()
    return rows


# ----------------------------------------------------------------------------------- chain
def part_chain(ranks=(8, 16), tokens=(1, 8), layers=(1, 8, 32, 128)) -> list:
    rows = []
    for R in ranks:
        spec = TRSpec(*DEFAULT, R)
        Lmax = max(layers)
        all_cores = [make_cores(spec, device="cuda", dtype=torch.float16, seed=1000 + i)
                     for i in range(Lmax)]
        for m in ("ours", "dense"):
            fns = [make_method(m, cores, spec) for cores in all_cores]
            weight_bytes = (spec.in_features * spec.out_features * 2 if m == "dense"
                            else fns[0].packed_bytes)
            for T in tokens:
                x = torch.randn(T, spec.in_features, device="cuda", dtype=torch.float16,
                                generator=torch.Generator(device="cuda").manual_seed(T))
                for L in layers:
                    sub = fns[:L]

                    def eager():
                        for f in sub:
                            f(x)

                    def body():
                        return [f(x) for f in sub]

                    eager_us = events_us(eager, L, reps=5)
                    graph, ys = capture(body)
                    graph_us = events_us(graph.replay, L, reps=5)
                    graph.replay()
                    torch.cuda.synchronize()
                    e0 = err(ys[0], reference64(x, all_cores[0], spec))
                    e1 = err(ys[-1], reference64(x, all_cores[L - 1], spec))
                    ok = e0["within_tol"] and e1["within_tol"]
                    rows.append({"rank": R, "tokens": T, "layers": L, "method": m,
                                 "eager_us_per_layer": eager_us, "graph_us_per_layer": graph_us,
                                 "weight_bytes_per_layer": weight_bytes,
                                 "err_first": e0, "err_last": e1})
                    log(f"chain R={R:2d} T={T:2d} L={L:4d} {m:5s} eager {eager_us:8.2f}  graph "
                        f"{graph_us:8.2f} us/layer  weights {weight_bytes / MIB:7.2f} MiB/layer "
                        f"{'ok' if ok else 'FAIL'}")
                    del graph, ys
            del fns
            torch.cuda.empty_cache()
    return rows


# ------------------------------------------------------------------------------------ cold
def part_cold(calls: int = 30, flush_mib: int = 1024) -> list:
    flush = torch.ones(flush_mib * MIB // 4, device="cuda", dtype=torch.float32)
    rows = []
    for label, (ins, outs), R, dtype, init, tokens in CASES:
        spec = TRSpec(ins, outs, R)
        cores = make_cores(spec, device="cuda", dtype=dtype, seed=0, init=init)
        for m in ("ours", "dense"):
            fn = make_method(m, cores, spec)
            for T in tokens:
                x = torch.randn(T, spec.in_features, device="cuda", dtype=dtype)
                fn(x)
                warm, cold = [], []
                for _ in range(calls):
                    for samples, do_flush in ((warm, False), (cold, True)):
                        # keep the GPU busy first, so that the call is queued before its
                        # start event runs and the events time the GPU work only
                        if do_flush:
                            flush.mul_(1.0)  # read + write 1 GiB: evicts L2 and Infinity Cache
                        else:
                            torch.cuda._sleep(100_000)  # a bounded spin: caches stay warm
                        s, e = (torch.cuda.Event(enable_timing=True),
                                torch.cuda.Event(enable_timing=True))
                        s.record()
                        fn(x)
                        e.record()
                        e.synchronize()
                        samples.append(s.elapsed_time(e) * 1000.0)
                row = {"case": label, "rank": R, "tokens": T, "method": m,
                       "warm_us": statistics.median(warm), "cold_us": statistics.median(cold)}
                rows.append(row)
                log(f"cold {label:15s} T={T:3d} {m:5s} warm {row['warm_us']:8.2f}  cold "
                    f"{row['cold_us']:8.2f} us/call")
            del fn
            torch.cuda.empty_cache()
    return rows


# ------------------------------------------------------------------------------------- mlp
def part_mlp(tokens=(1, 8, 32), blocks=(1, 8)) -> list:
    dtype = torch.bfloat16
    s_up, s_down = TRSpec(*LLAMA_UP, 8), TRSpec(*LLAMA_DOWN, 16)
    nmax = max(blocks)
    weights = []
    for b in range(nmax):
        cg = make_cores(s_up, device="cuda", dtype=dtype, seed=10 * b + 1, init="uniform")
        cu = make_cores(s_up, device="cuda", dtype=dtype, seed=10 * b + 2, init="uniform")
        cd = make_cores(s_down, device="cuda", dtype=dtype, seed=10 * b + 3, init="uniform")
        weights.append((cg, cu, cd))
    ring = [tuple(prepare_optimized(c, s) for c, s in ((cg, s_up), (cu, s_up), (cd, s_down)))
            for cg, cu, cd in weights]
    dense = [tuple(materialize_dense_weight(c, s) for c, s in ((cg, s_up), (cu, s_up),
                                                                (cd, s_down)))
             for cg, cu, cd in weights]

    def unfused(b, x, h):
        g, u, d = ring[b]
        return h + d(F.silu(g(x)) * u(x))

    def consume(b, x, h):
        g, u, d = ring[b]
        return consume_add(h, d.accumulate(consume_silu_mul(g.accumulate(x), u.accumulate(x),
                                                            dtype)))

    def fused(b, x, h):
        g, u, d = ring[b]
        return d.forward_add(u.forward_silu_mul(x, g.accumulate(x)), h)

    def dense_block(b, x, h):
        wg, wu, wd = dense[b]
        return h + F.linear(F.silu(F.linear(x, wg)) * F.linear(x, wu), wd)

    methods = {"unfused": unfused, "consume": consume, "fused": fused, "dense": dense_block}
    rows = []
    for T in tokens:
        x = torch.randn(T, 4096, device="cuda", dtype=dtype,
                        generator=torch.Generator(device="cuda").manual_seed(T))
        h = torch.randn(T, 4096, device="cuda", dtype=dtype,
                        generator=torch.Generator(device="cuda").manual_seed(100 + T))
        # fp64 reference of block 0 (rounded inputs, no intermediate rounding)
        w64 = [materialize_dense_weight([c.double() for c in cs], s)
               for cs, s in zip(weights[0], (s_up, s_up, s_down))]
        xd = x.double()
        ref0 = h.double() + (F.silu(xd @ w64[0].T) * (xd @ w64[1].T)) @ w64[2].T
        del w64
        for nb in blocks:
            for name, fn in methods.items():
                # a chain of nb blocks: each block's output is the next one's x and h
                def chain():
                    y = x
                    for b in range(nb):
                        y = fn(b, y, y if b else h)
                    return y

                eager_us = events_us(chain, 1, reps=9)
                graph, y_static = capture(chain)
                graph_us = events_us(graph.replay, 1, reps=9)
                row = {"tokens": T, "blocks": nb, "method": name, "eager_us": eager_us,
                       "graph_us": graph_us}
                if nb == 1:
                    graph.replay()
                    torch.cuda.synchronize()
                    row["error_vs_fp64"] = err(y_static, ref0)
                rows.append(row)
                extra = (f"  rel-L2 {row['error_vs_fp64']['rel_l2']:.2e}" if nb == 1 else "")
                log(f"mlp T={T:3d} blocks={nb} {name:8s} eager {eager_us:8.2f}  graph "
                    f"{graph_us:8.2f} us{extra}")
                del graph, y_static
        torch.cuda.empty_cache()
    return rows


PARTS = {"single": part_single, "chain": part_chain, "cold": part_cold, "mlp": part_mlp}


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--part", choices=sorted(PARTS), required=True)
    ap.add_argument("--out", type=Path, required=True)
    args = ap.parse_args()
    if not torch.cuda.is_available():
        print("graph_bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    torch.backends.cuda.matmul.allow_fp16_reduced_precision_reduction = False
    torch.backends.cuda.matmul.allow_bf16_reduced_precision_reduction = False
    with torch.inference_mode():
        rows = PARTS[args.part]()
    info = {"part": args.part, "device": torch.cuda.get_device_name(0),
            "torch": torch.__version__, "hip": torch.version.hip,
            "hip_force_dev_kernarg": os.environ.get("HIP_FORCE_DEV_KERNARG"), "rows": rows}
    args.out.parent.mkdir(parents=True, exist_ok=True)
    args.out.write_text(json.dumps(info, indent=1) + "\n")
    log(f"wrote {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())

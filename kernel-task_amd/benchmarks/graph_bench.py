"""Measurements beyond single uncaptured calls: HIP graphs, chains of distinct layers, cold
caches and a SwiGLU MLP block with fused epilogues. One MI355X.

    python kernel-task_amd/benchmarks/graph_bench.py --part single --out single.json
    python kernel-task_amd/benchmarks/graph_bench.py --part chain  --out chain.json
    python kernel-task_amd/benchmarks/graph_bench.py --part cold   --out cold.json
    python kernel-task_amd/benchmarks/graph_bench.py --part mlp    --out mlp.json

Covers what the reference measures in tools/graph_bench.py (parts single / chain / cold,
:1-27) and tools/v3g_fp32out.py (an MLP block on fp32-output consumers). Every figure is
HIP-event time around a block of work (factorized_inference.measure.stream_us), median of
several blocks, per call or per layer.

A "program" is a list of zero-argument thunks run in order on the current stream. Each
part builds programs and measures them two ways (`eager_and_graph`): launched one by one
from the host, and captured once into a HIP graph (`Captured`) and replayed. Outputs of the
last replay are checked against the float64 factorized path (tr_forward_reference on
float64 copies of the same cores; no dense weight is formed for the check).

Parts:
  single  every BASELINE case, ours and the dense GEMM: a program of G calls.
  chain   L distinct operators (different weights) on one input, eager and captured, per
          layer. At L = 128 the dense weights (11 MB each, 1.4 GB) exceed the 256 MB Infinity
          Cache; the ring's packed cores (0.25-0.9 MB each) still fit.
  cold    one call after a 1 GiB read-modify-write that evicts the L2s and the Infinity
          Cache, next to the same call after a bounded spin kernel (caches stay warm). The
          call is queued behind the busy GPU, so its events time the GPU work without the
          host's launch latency.
  mlp     h + down(silu(gate(x)) * up(x)) with the Llama-3-8B shapes (gate/up 4096->14336
          rank 8, down 14336->4096 rank 16, bf16), one block and a chain of 8 blocks:
            unfused  gate, up, down, then torch silu, mul and the residual add
            consume  accumulate() x3 with the standalone consumers (the reference's
                     fp32-output chain, consume_silu_mul / consume_add)
            fused    gate.accumulate, up.forward_silu_mul, down.forward_add: 3 launches
            pair     forward_swiglu(gate, up) (gate and up in one launch), down.forward_add:
                     2 launches
            dense    the same block on the materialised weights (F.linear)
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Callable, Sequence

os.environ.setdefault("HIP_FORCE_DEV_KERNARG", "0")  # as bench.py: kernel arguments in host memory
PACKAGE_ROOT = Path(__file__).resolve().parents[1]
if str(PACKAGE_ROOT) not in sys.path:
    sys.path.insert(0, str(PACKAGE_ROOT))

import torch  # noqa: E402
import torch.nn.functional as F  # noqa: E402

from factorized_inference import (  # noqa: E402
    TRSpec, dense_forward, make_cores, materialize_dense_weight, prepare_optimized,
    tr_forward_reference,
)
from factorized_inference import measure as m  # noqa: E402
from factorized_inference.tr_kernel import (  # noqa: E402
    consume_add, consume_silu_mul, forward_swiglu,
)

MIB = 1 << 20
TOL = 0.02  # the 16-bit acceptance rule |y - y_ref| <= TOL + TOL |y_ref|


@dataclass(frozen=True)
class Shape:
    label: str
    ins: tuple
    outs: tuple
    rank: int
    dtype: torch.dtype
    init: str
    tokens: tuple

    def spec(self) -> TRSpec:
        return TRSpec(self.ins, self.outs, self.rank)


SHAPES = [
    Shape("r8", (8, 12, 20), (12, 10, 24), 8, torch.float16, "per_core", (1, 8, 32)),
    Shape("r16", (8, 12, 20), (12, 10, 24), 16, torch.float16, "per_core", (1, 32)),
    Shape("llama_up_r8", (16, 16, 16), (16, 28, 32), 8, torch.bfloat16, "uniform", (1, 8, 32, 128)),
    Shape("llama_down_r16", (16, 28, 32), (16, 16, 16), 16, torch.bfloat16, "uniform", (1, 32, 256)),
]


def log(msg: str) -> None:
    print(msg, flush=True)


Program = Sequence[Callable[[], torch.Tensor]]


class Captured:
    """A program captured into one HIP graph. Capture needs the program's allocations
    settled first, so it runs twice on a side stream before the capture (PyTorch's
    documented order for torch.cuda.graph); `outputs` are the captured calls' static
    results, rewritten by every replay."""

    def __init__(self, program: Program):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                for step in program:
                    step()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.outputs = [step() for step in program]
        torch.cuda.synchronize()

    def replay(self) -> None:
        self.graph.replay()


def per_call_us(block: Callable[[], None], calls_in_block: int, blocks: int) -> float:
    """Median over `blocks` HIP-event-timed runs of `block`, per call inside it."""
    block()                                  # one untimed run
    return statistics.median(m.stream_us(block, 1, blocks=blocks)) / calls_in_block


def eager_and_graph(program: Program, blocks: int = 7) -> tuple[float, float, list]:
    """(eager us per step, captured us per step, the captured outputs after a replay)."""
    def run_eager():
        for step in program:
            step()

    eager = per_call_us(run_eager, len(program), blocks)
    captured = Captured(program)
    graphed = per_call_us(captured.replay, len(program), blocks)
    captured.replay()
    torch.cuda.synchronize()
    outputs = captured.outputs
    del captured
    return eager, graphed, outputs


def reference_fp64(x: torch.Tensor, cores, spec: TRSpec) -> torch.Tensor:
    return tr_forward_reference(x.double(), [c.double() for c in cores], spec)


def compare(y: torch.Tensor, ref: torch.Tensor) -> dict:
    d = (y.double() - ref).abs()
    return {"max_abs": d.max().item(),
            "rel_l2": (d.norm() / ref.norm().clamp_min(1e-30)).item(),
            "within_tol": bool((d <= TOL + TOL * ref.abs()).all())}


def operator(method: str, cores, spec: TRSpec) -> Callable[[torch.Tensor], torch.Tensor]:
    """The HIP operator, or the dense GEMM on the materialised weight (comparator only)."""
    if method == "ours":
        return prepare_optimized(cores, spec)
    weight = materialize_dense_weight(cores, spec)
    return lambda x: dense_forward(x, weight)


def seeded_x(tokens: int, features: int, dtype, seed: int) -> torch.Tensor:
    return torch.randn(tokens, features, device="cuda", dtype=dtype,
                       generator=torch.Generator(device="cuda").manual_seed(seed))


# ---------------------------------------------------------------------------------- single
def part_single(calls: int = 20) -> list:
    rows = []
    for shape in SHAPES:
        spec = shape.spec()
        cores = make_cores(spec, device="cuda", dtype=shape.dtype, seed=0, init=shape.init)
        for method in ("ours", "dense"):
            op = operator(method, cores, spec)
            for T in shape.tokens:
                x = seeded_x(T, spec.in_features, shape.dtype, T)
                eager, graphed, outs = eager_and_graph([lambda: op(x)] * calls)
                check = compare(outs[-1], reference_fp64(x, cores, spec))
                rows.append({"case": shape.label, "rank": shape.rank, "tokens": T,
                             "method": method, "dtype": str(shape.dtype).replace("torch.", ""),
                             "calls_per_graph": calls, "eager_us_per_call": eager,
                             "graph_us_per_call": graphed, "graph_output_error": check})
                log(f"single {shape.label:15s} T={T:3d} {method:5s} eager {eager:8.2f}  graph "
                    f"{graphed:8.2f} us/call  max|err| {check['max_abs']:.2e} "
                    f"{'ok' if check['within_tol'] else 'FAIL'}")
            del op
            torch.cuda.empty_cache()
    return rows


# ----------------------------------------------------------------------------------- chain
def part_chain(ranks=(8, 16), tokens=(1, 8), depths=(1, 8, 32, 128)) -> list:
    rows = []
    for R in ranks:
        spec = TRSpec((8, 12, 20), (12, 10, 24), R)
        layers = [make_cores(spec, device="cuda", dtype=torch.float16, seed=1000 + i)
                  for i in range(max(depths))]
        for method in ("ours", "dense"):
            ops = [operator(method, cores, spec) for cores in layers]
            held = (spec.in_features * spec.out_features * 2 if method == "dense"
                    else ops[0].packed_bytes)
            for T in tokens:
                x = seeded_x(T, spec.in_features, torch.float16, T)
                for depth in depths:
                    program = [(lambda op=op: op(x)) for op in ops[:depth]]
                    eager, graphed, outs = eager_and_graph(program, blocks=5)
                    first = compare(outs[0], reference_fp64(x, layers[0], spec))
                    last = compare(outs[-1], reference_fp64(x, layers[depth - 1], spec))
                    rows.append({"rank": R, "tokens": T, "layers": depth, "method": method,
                                 "eager_us_per_layer": eager, "graph_us_per_layer": graphed,
                                 "weight_bytes_per_layer": held,
                                 "err_first": first, "err_last": last})
                    good = first["within_tol"] and last["within_tol"]
                    log(f"chain R={R:2d} T={T:2d} L={depth:4d} {method:5s} eager {eager:8.2f}  "
                        f"graph {graphed:8.2f} us/layer  weights {held / MIB:7.2f} MiB/layer "
                        f"{'ok' if good else 'FAIL'}")
            del ops
            torch.cuda.empty_cache()
    return rows


# ------------------------------------------------------------------------------------ cold
def part_cold(samples: int = 30, flush_mib: int = 1024) -> list:
    """Warm and cold single calls. Before each timed call the GPU is kept busy, by a bounded
    spin (warm) or by rewriting a buffer larger than every cache (cold), so the call's
    events are queued behind that work and time only the call on the GPU."""
    flush = torch.ones(flush_mib * MIB // 4, device="cuda", dtype=torch.float32)
    busy = {"warm": lambda: torch.cuda._sleep(100_000), "cold": lambda: flush.mul_(1.0)}
    rows = []
    for shape in SHAPES:
        spec = shape.spec()
        cores = make_cores(spec, device="cuda", dtype=shape.dtype, seed=0, init=shape.init)
        for method in ("ours", "dense"):
            op = operator(method, cores, spec)
            for T in shape.tokens:
                x = seeded_x(T, spec.in_features, shape.dtype, T)
                op(x)
                times = {"warm": [], "cold": []}
                for _ in range(samples):
                    for kind, before in busy.items():
                        before()
                        times[kind].append(_queued_call_us(lambda: op(x)))
                row = {"case": shape.label, "rank": shape.rank, "tokens": T, "method": method,
                       "warm_us": statistics.median(times["warm"]),
                       "cold_us": statistics.median(times["cold"])}
                rows.append(row)
                log(f"cold {shape.label:15s} T={T:3d} {method:5s} warm {row['warm_us']:8.2f}  "
                    f"cold {row['cold_us']:8.2f} us/call")
            del op
            torch.cuda.empty_cache()
    return rows


def _queued_call_us(call: Callable[[], object]) -> float:
    """HIP events around one call recorded behind work already queued (no synchronize
    first, unlike measure.stream_us)."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    call()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) * 1000.0


# ------------------------------------------------------------------------------------- mlp
@dataclass
class Block:
    """One Llama-3-8B-shaped SwiGLU MLP block: cores, the prepared operators, dense weights."""
    cores: tuple
    ring: tuple
    dense: tuple


def _mlp_blocks(count: int, s_up: TRSpec, s_down: TRSpec) -> list[Block]:
    blocks = []
    for b in range(count):
        cores = tuple(make_cores(s, device="cuda", dtype=torch.bfloat16, seed=10 * b + k,
                                 init="uniform")
                      for k, s in ((1, s_up), (2, s_up), (3, s_down)))
        specs = (s_up, s_up, s_down)
        blocks.append(Block(cores, tuple(prepare_optimized(c, s) for c, s in zip(cores, specs)),
                            tuple(materialize_dense_weight(c, s) for c, s in zip(cores, specs))))
    return blocks


MLP_FORMS = {
    "unfused": lambda b, x, h: h + b.ring[2](F.silu(b.ring[0](x)) * b.ring[1](x)),
    "consume": lambda b, x, h: consume_add(h, b.ring[2].accumulate(
        consume_silu_mul(b.ring[0].accumulate(x), b.ring[1].accumulate(x), torch.bfloat16))),
    "fused": lambda b, x, h: b.ring[2].forward_add(b.ring[1].forward_silu_mul(
        x, b.ring[0].accumulate(x)), h),
    "pair": lambda b, x, h: b.ring[2].forward_add(forward_swiglu(b.ring[0], b.ring[1], x), h),
    "dense": lambda b, x, h: h + F.linear(F.silu(F.linear(x, b.dense[0]))
                                          * F.linear(x, b.dense[1]), b.dense[2]),
}


def part_mlp(tokens=(1, 8, 32), depths=(1, 8)) -> list:
    s_up = TRSpec((16, 16, 16), (16, 28, 32), 8)
    s_down = TRSpec((16, 28, 32), (16, 16, 16), 16)
    blocks = _mlp_blocks(max(depths), s_up, s_down)
    rows = []
    for T in tokens:
        x = seeded_x(T, 4096, torch.bfloat16, T)
        h = seeded_x(T, 4096, torch.bfloat16, 100 + T)
        # float64 reference of block 0 from the factorized path (no intermediate rounding)
        b0 = blocks[0]
        gate, up = (reference_fp64(x, c, s_up) for c in b0.cores[:2])
        ref0 = h.double() + tr_forward_reference(F.silu(gate) * up,
                                                 [c.double() for c in b0.cores[2]], s_down)
        for depth in depths:
            for name, form in MLP_FORMS.items():
                def chain(form=form, depth=depth):
                    y = x
                    for b in range(depth):
                        y = form(blocks[b], y, y if b else h)
                    return y

                eager, graphed, outs = eager_and_graph([chain], blocks=9)
                row = {"tokens": T, "blocks": depth, "method": name, "eager_us": eager,
                       "graph_us": graphed}
                note = ""
                if depth == 1:
                    row["error_vs_fp64"] = compare(outs[0], ref0)
                    note = f"  rel-L2 {row['error_vs_fp64']['rel_l2']:.2e}"
                rows.append(row)
                log(f"mlp T={T:3d} blocks={depth} {name:8s} eager {eager:8.2f}  graph "
                    f"{graphed:8.2f} us{note}")
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
    report = {"part": args.part, "device": torch.cuda.get_device_name(0),
              "torch": torch.__version__, "hip": torch.version.hip,
              "hip_force_dev_kernarg": os.environ.get("HIP_FORCE_DEV_KERNARG"), "rows": rows}
    args.out.parent.mkdir(parents=True, exist_ok=True)
    args.out.write_text(json.dumps(report, indent=1) + "\n")
    log(f"wrote {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Persistent multi-layer stack: build and run stack_bench.hip in its two forms.

    python kernel-task_amd/benchmarks/stack_bench.py --build            (any machine with hipcc)
    python kernel-task_amd/benchmarks/stack_bench.py --out stack.json [--tokens 1] [--layers 8,32,128]
    python kernel-task_amd/benchmarks/stack_bench.py --parallel 8 --out par.json   (P stacks side by side)

Builds kernel-task_amd/benchmarks/_bin/stack_bench_{all,xcd} against libtrk.so (the same
compiler flags as the library) and, on an MI355X, runs both: every XCD with a device-scope
barrier, and one XCD with an L2 barrier (with and without prefetching the next layer's core
slices across it). Each line compares the stack with the same tiles launched once per layer,
eagerly and in a HIP graph, and checks that the stack's output equals theirs bit for bit.
--parallel P runs P one-XCD stacks at once, stack k on XCD k (P sequences through the same
layers), against one stack alone and the same tiles launched per layer for a batch of P
tokens.

Role of the reference's stack experiment and its one-GPU measurement plan
(kernel_work/stack/tr_stack.cu:1-40, kernel-design/WEIGHT_STATIONARY.md:104-147).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from factorized_inference import build_ext  # noqa: E402

SOURCE = HERE / "stack_bench.hip"
BIN = HERE / "_bin"
FORMS = {"all": 0, "xcd": 1}


def binary(form: str) -> Path:
    return BIN / f"stack_bench_{form}"


def build(verbose: bool = False) -> list[Path]:
    """Compile both forms (rank 8) into _bin/; raises with hipcc's message on failure."""
    BIN.mkdir(exist_ok=True)
    lib = build_ext.PACKAGE
    out = []
    for form, xcd in FORMS.items():
        cmd = [build_ext._hipcc(), *build_ext.HIPCC_FLAGS, f"-DSTACK_XCD={xcd}", "-DSTACK_RANK=8",
               str(SOURCE), "-o", str(binary(form)), f"-L{lib}", "-l:libtrk.so",
               # found relative to the binary, so a copy of the tree uses its own library
               f"-Wl,-rpath,$ORIGIN/{os.path.relpath(lib, BIN)}"]
        if verbose:
            print(" ".join(cmd), flush=True)
        done = subprocess.run(cmd, capture_output=True, text=True)
        if done.returncode != 0:
            raise RuntimeError(f"hipcc failed on {SOURCE.name} ({form}):\n{done.stderr[-4000:]}")
        out.append(binary(form))
    return out


def run(form: str, tokens: int, layers: list[int], timeout: float = 240.0,
        parallel: int = 0, dump: Path | None = None) -> list[dict]:
    """Run one form (with `parallel` > 0: that many one-XCD stacks side by side); returns its
    JSON lines. With `dump`, the program writes x, each layer's cores and every checked
    output into that directory (raw fp16: x.bin, core_l<l>_k<k>.bin, y_<form>_T<T>_L<L>_pf<p>.bin,
    yref_<form>_T<T>_L<L>.bin; side by side ypar<k>_L<L>.bin and yref_L<L>.bin). Raises if the
    program fails or reports an error."""
    path = binary(form)
    if not path.exists():
        raise RuntimeError(f"{path} is not built; run with --build first")
    env = dict(os.environ)
    if parallel:
        env["STACK_PAR"] = str(parallel)
    if dump is not None:
        Path(dump).mkdir(parents=True, exist_ok=True)
        env["STACK_DUMP"] = str(dump)
    done = subprocess.run([str(path), str(tokens), *map(str, layers)], capture_output=True,
                          text=True, timeout=timeout, env=env)
    rows = [json.loads(ln) for ln in done.stdout.splitlines() if ln.startswith("{")]
    if done.returncode != 0 or any("error" in r for r in rows):
        raise RuntimeError(f"{path.name} failed ({done.returncode}):\n{done.stdout}\n{done.stderr}")
    return rows


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--build", action="store_true", help="compile the two forms and exit")
    ap.add_argument("--out", type=Path)
    ap.add_argument("--tokens", type=int, default=1)
    ap.add_argument("--layers", default="8,32,128")
    ap.add_argument("--parallel", type=int, default=0, metavar="P",
                    help="run P one-XCD stacks side by side (1-8) instead of the two forms")
    args = ap.parse_args()
    if args.build:
        for p in build(verbose=True):
            print(p)
        return 0
    layers = [int(v) for v in args.layers.split(",")]
    rows = []
    if args.parallel:
        for r in run("xcd", 1, layers, parallel=args.parallel):
            rows.append(r)
            L, P = r["layers"], r["stacks"]
            print(f"{P} one-XCD stacks L={L:4d}: {r['parallel_us'] / L:.3f} us per layer for all "
                  f"{P} ({r['parallel_us'] / L / P:.3f} per sequence-layer), one stack "
                  f"{r['one_stack_us'] / L:.3f}, per-layer launches of {P} tokens "
                  f"{r['batched_per_layer_us'] / L:.3f}; outputs differing "
                  f"{r['outputs_differing']} of {r['outputs']}; XCDs {r['xcd_ids']}", flush=True)
        if args.out:
            args.out.parent.mkdir(parents=True, exist_ok=True)
            args.out.write_text(json.dumps({"rows": rows}, indent=1) + "\n")
        return 0
    for form in FORMS:
        for r in run(form, args.tokens, layers):
            rows.append(r)
            print(f"{r['form']:8s} prefetch={str(r['prefetch']):5s} T={r['tokens']} L={r['layers']:4d}: "
                  f"stack {r['stack_us'] / r['layers']:.3f} us/layer, barriers "
                  f"{r['barriers_only_us'] / r['layers']:.3f}, per-layer eager "
                  f"{r['per_layer_eager_us'] / r['layers']:.3f}, graph "
                  f"{r['per_layer_graph_us'] / r['layers']:.3f}; outputs differing "
                  f"{r['outputs_differing']} of {r['outputs']}"
                  + (f"; XCDs {r['xcd_ids']}" if r["xcd_ids"] else ""), flush=True)
    if args.out:
        args.out.parent.mkdir(parents=True, exist_ok=True)
        args.out.write_text(json.dumps({"rows": rows}, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    sys.exit(main())

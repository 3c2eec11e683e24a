"""Compile-time guard of the MFMA kernels: an accumulation chain that mixes 16x16x32 and
16x16x16 MFMAs on one accumulator must not compile (trk_mfma_kernel.h, struct Acc).

A mixed chain gave wrong sums on gfx950 in one schedule; the kernels avoid it by finishing a
K that ends in 16 with a half-zero 16x16x32 MFMA. This checks, with hipcc's device-only syntax
pass (no GPU needed), that the accumulator types make the mistake a compile error."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

SNIPPET = """
#include "trk_mfma_kernel.h"
using namespace trk;
__global__ void chain(float *out) {{
    using O = Ops<TRK_DTYPE_F16>;
    O::V8 a8{{}}, b8{{}};
    O::V4 a4{{}}, b4{{}};
    Acc<{first}> d{{}};
    d = O::k{first}({args_first}, d);
    {second}
    out[threadIdx.x] = d.v[0];
}}
"""


def compile_snippet(tmp_path, first: int, second: str) -> subprocess.CompletedProcess:
    args = "a8, b8" if first == 32 else "a4, b4"
    src = tmp_path / "guard.hip"
    src.write_text(SNIPPET.format(first=first, args_first=args, second=second))
    return subprocess.run(
        [HIPCC, "--offload-arch=gfx950", "-std=c++20", "--cuda-device-only", "-fsyntax-only",
         f"-I{ROOT / 'include'}", f"-I{ROOT / 'kernel-task_amd' / 'csrc'}", str(src)],
        capture_output=True, text=True)


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not installed")
def test_single_shape_chains_compile(tmp_path):
    for first, second in ((32, "d = O::k32(a8, b8, d);"), (16, "d = O::k16(a4, b4, d);")):
        done = compile_snippet(tmp_path, first, second)
        assert done.returncode == 0, done.stderr[-2000:]


@pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc not installed")
def test_mixed_shape_chains_do_not_compile(tmp_path):
    for first, second in ((32, "d = O::k16(a4, b4, d);"), (16, "d = O::k32(a8, b8, d);")):
        done = compile_snippet(tmp_path, first, second)
        assert done.returncode != 0, f"a {first}-then-other chain compiled"
        assert "no viable conversion" in done.stderr or "no matching" in done.stderr, done.stderr[-2000:]

"""Build recipe for the oracle's C restatement (test infrastructure only).

    python oracle/build.py        ->  oracle/libring_oracle.so

The reference's own implementation of this path is Python on torch
(src/factorized_inference/reference.py) and its native code is sm_90 CUDA that nvcc would
have to build; neither compiles here from a few C/C++ sources, so there is no oracle/_ref
build. The oracle is pinned without it (tests/test_oracle.py).
"""
from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "ring_oracle.c"
LIBRARY = HERE / "libring_oracle.so"


def build(verbose: bool = False) -> Path:
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-o", str(LIBRARY), str(SOURCE)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv[1:]))

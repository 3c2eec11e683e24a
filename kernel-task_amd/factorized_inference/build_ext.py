"""Build libtrk.so, the HIP library behind prepare_optimized, for gfx950.

    python -m factorized_inference.build_ext      (from kernel-task_amd/)

The library is built in-tree next to this file so that it travels with the source tree; it
is never built lazily at import or call time (a missing library is an error).
"""
from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE.parent / "csrc"
INCLUDE = PACKAGE.parents[1] / "include"
LIBRARY = PACKAGE / "libtrk.so"
FASTCALL = PACKAGE / ("_trkcall" + sysconfig.get_config_var("EXT_SUFFIX"))
OBJ_DIR = PACKAGE.parent / "_build"
ARCH = "gfx950"

# -packed-fp32-ops: no packed fp32 VALU ops (v_pk_*_f32) anywhere in the device code.
# -amdgpu-kernarg-preload-count: kernel arguments arrive in SGPRs at wave start instead of
# being fetched from memory first (a memory latency off the front of every launch).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall",
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else "hipcc"


def build(verbose: bool = False, jobs: int = 8) -> Path:
    OBJ_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()

    def compile_one(src: Path) -> Path:
        obj = OBJ_DIR / (src.stem + ".o")
        cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        done = subprocess.run(cmd, capture_output=True, text=True)
        if done.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{done.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objects = list(pool.map(compile_one, sources()))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objects)]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIBRARY)
    # the CPython fast-call binding of trk_forward, linked against libtrk.so next to it
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-std=c11", f"-I{INCLUDE}",
           f"-I{sysconfig.get_paths()['include']}", str(CSRC / "trk_pycall.c"),
           "-o", str(FASTCALL), f"-L{PACKAGE}", "-l:libtrk.so", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv[1:]))

"""Build libtrk.so, the HIP library behind prepare_optimized, for gfx950.

    python -m factorized_inference.build_ext      (from kernel-task_amd/)

The library is built in-tree next to this file so that it travels with the source tree; it
is never built lazily at import or call time (a missing library is an error).
"""
from __future__ import annotations

import json
import os
import re
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
TORCHCALL = PACKAGE / ("_trktorch" + sysconfig.get_config_var("EXT_SUFFIX"))
OBJ_DIR = PACKAGE.parent / "_build"
# per-kernel register, scratch and LDS use reported by the compiler (a build artifact)
RESOURCES = PACKAGE / "kernel_resources.json"
ARCH = "gfx950"

# -packed-fp32-ops: no packed fp32 VALU ops (v_pk_*_f32) anywhere in the device code.
# -amdgpu-kernarg-preload-count: kernel arguments arrive in SGPRs at wave start instead of
# being fetched from memory first (a memory latency off the front of every launch).
# -amdgpu-mfma-vgpr-form: MFMA results go to ordinary VGPRs, so the epilogues that convert
# and store them need no accumulator-register reads (measured faster for both kernel families).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++20", "-fPIC", "-Wall",
    "-mllvm", "-amdgpu-kernarg-preload-count=16", "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


# Per-source additions to HIPCC_FLAGS (the two MFMA kernel families are separate
# translation units so that each can be tuned on its own).
FILE_FLAGS: dict[str, list[str]] = {}


def sources() -> list[Path]:
    """Every HIP source: the hand-written ones and the generated variant tables (csrc/gen/,
    rewritten from tilegen.py's declared shapes and tuned table first)."""
    from . import tilegen

    tilegen.write_all()
    return sorted(CSRC.glob("*.hip")) + sorted((CSRC / "gen").glob("*.hip"))


def _newest_dependency() -> float:
    """Modification time of the newest header and of this build script (a change to either
    recompiles every source)."""
    deps = [*CSRC.glob("*.h"), *INCLUDE.glob("*.h"), Path(__file__)]
    return max(p.stat().st_mtime for p in deps)


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else "hipcc"


def build(verbose: bool = False, jobs: int = 8, incremental: bool = False) -> Path:
    """Compile every source and link libtrk.so and the two bindings. incremental=True
    (development only) reuses objects newer than their source, the headers and this script."""
    OBJ_DIR.mkdir(exist_ok=True)
    hipcc = _hipcc()

    def compile_one(src: Path) -> Path:
        obj = OBJ_DIR / (src.stem + ".o")
        report = obj.with_suffix(".resources.json")
        if (incremental and obj.exists() and report.exists()
                and obj.stat().st_mtime > max(_newest_dependency(), src.stat().st_mtime)):
            return obj
        cmd = [hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []),
               "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        done = subprocess.run(cmd, capture_output=True, text=True)
        if done.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src.name}:\n{done.stderr}")
        report.write_text(json.dumps(parse_resource_remarks(done.stderr)))
        return obj

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        objects = list(pool.map(compile_one, sources()))
    resources = {}
    for obj in objects:
        resources.update(json.loads(obj.with_suffix(".resources.json").read_text()))
    RESOURCES.write_text(json.dumps(resources, indent=0, sort_keys=True) + "\n")
    tmp = LIBRARY.with_suffix(".so.tmp")
    # the SONAME lets the variant modules' dependency on libtrk.so resolve to the copy this
    # process already loaded, wherever the tree lives (they carry no path to it)
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-soname,libtrk.so",
           "-o", str(tmp), *map(str, objects), "-ldl"]
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
    _build_torchcall(verbose)
    return LIBRARY


_REMARK = re.compile(r"remark: +(Function Name|[A-Za-z][A-Za-z /]*?)(?: \[[^\]]*\])?: (\S+) "
                     r"\[-Rpass-analysis=kernel-resource-usage\]")


def parse_resource_remarks(stderr: str) -> dict[str, dict[str, str]]:
    """{kernel: {"VGPRs": .., "AGPRs": .., "ScratchSize": .., "VGPRs Spill": .., ...}} from the
    compiler's kernel-resource-usage remarks (device pass only; host remarks do not occur)."""
    out: dict[str, dict[str, str]] = {}
    current = None
    for key, value in _REMARK.findall(stderr):
        if key == "Function Name":
            current = out.setdefault(value, {})
        elif current is not None:
            current[key.strip()] = value
    return out


def _build_torchcall(verbose: bool) -> None:
    """_trktorch: PreparedTRKernel's per-call path in C++ (g++ against torch's headers)."""
    import torch

    root = Path(torch.__file__).resolve().parent
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch.compiled_with_cxx11_abi())}",
           f"-I{root / 'include'}", f"-I{root / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
           f"-I{rocm}/include", f"-I{sysconfig.get_paths()['include']}", f"-I{INCLUDE}",
           str(CSRC / "trk_torchcall.cpp"), "-o", str(TORCHCALL.with_suffix(".tmp")),
           f"-L{root / 'lib'}", "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip",
           "-ltorch_python",
           f"-L{PACKAGE}", "-l:libtrk.so", "-Wl,-rpath,$ORIGIN"]
    if verbose:
        print(" ".join(cmd), flush=True)
    done = subprocess.run(cmd, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"g++ failed on trk_torchcall.cpp:\n{done.stderr}")
    os.replace(TORCHCALL.with_suffix(".tmp"), TORCHCALL)


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv[1:], incremental="--incremental" in sys.argv[1:]))

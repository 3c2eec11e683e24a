"""Variant modules built at prepare time for shapes the library has no MFMA tables for.

libtrk.so carries MFMA kernels for the declared shapes only (tilegen.DECLARED); a plan for
any other shape would run the generic VALU kernel. For fp16, bf16 and fp32 plans,
PreparedTRKernel asks this module for a variant module instead:

  1. the kernel rank: the cores' rank if it is a power of two >= 8, else the next such power
     (up to 32). A padded plan (trk_plan_create_padded) packs zeros into the extra ring
     entries, so its kernels compute exactly the rank-R operator;
  2. the variant table of (shape, kernel rank, dtype), written by tilegen.emit_module: the
     generator's rule-based tiles for that shape (untuned token ranges);
  3. hipcc compiles it into a shared library next to the package (kernel-task_amd/_jit/,
     or $TRK_JIT_DIR), named by a hash of the table, the kernel headers and the compiler
     flags, so a changed header or table builds a new module and an unchanged one is reused
     across processes;
  4. trk_plan_load_module checks the module's ABI and plan layout and adds its variants. The
     module names libtrk.so as a dependency without a path; the copy the process has loaded
     (SONAME libtrk.so) satisfies it, so a tree copied elsewhere works unchanged.

This is the role of the reference's first-use build of its extension (tr_kernel.py:31-57,
torch.utils.cpp_extension.load: about a minute the first time, then cached). A module build
takes tens of seconds once per shape; TRK_JIT=0 turns it off (such shapes then run the
generic kernel).
"""
from __future__ import annotations

import fcntl
import hashlib
import os
import subprocess
from pathlib import Path

from . import build_ext, tilegen

PACKAGE = Path(__file__).resolve().parent
CACHE = Path(os.environ.get("TRK_JIT_DIR", PACKAGE.parent / "_jit"))
HEADERS = ("trk_mfma_kernel.h", "trk_internal.h", "trk_types.h")
MAX_KERNEL_RANK = 32
# how a module links (hashed with the source): libtrk.so by name only, no run path
LINK_FLAGS = ("-shared", "-fvisibility=hidden", "-l:libtrk.so")


def enabled() -> bool:
    return os.environ.get("TRK_JIT", "1") != "0"


def kernel_rank(rank: int) -> int | None:
    """The rank the MFMA kernels run for cores of `rank`: the smallest power of two that is
    at least max(8, rank), or None above MAX_KERNEL_RANK."""
    k = 8
    while k < rank:
        k *= 2
    return k if k <= MAX_KERNEL_RANK else None


def module_source(shape: tilegen.ShapeDecl) -> str | None:
    """The module's source, or None when the generator finds no tile for the shape. Only the
    tiles with a token range are compiled (the rule's picks)."""
    src = tilegen.emit_module(shape)
    lines = [ln for ln in src.splitlines()
             if "TRK_ENTRY(" not in ln or not ln.rstrip().split("//")[0].rstrip().endswith(", 0, 0)")]
    if not any("TRK_ENTRY(" in ln for ln in lines):
        return None
    return "\n".join(lines) + "\n"


def _fingerprint(src: str) -> str:
    h = hashlib.sha256(src.encode())
    for name in HEADERS:
        h.update((build_ext.CSRC / name).read_bytes())
    h.update((build_ext.INCLUDE / "trk.h").read_bytes())
    # the flags without the include directories: those are absolute paths of this checkout,
    # and the headers they point to are hashed above, so a copy of the tree elsewhere (a
    # GPU box) reuses the modules built here
    h.update(" ".join(f for f in build_ext.HIPCC_FLAGS if not f.startswith("-I")).encode())
    h.update(" ".join(LINK_FLAGS).encode())
    return h.hexdigest()[:16]


def module_path(shape: tilegen.ShapeDecl) -> Path | None:
    """Where the module of `shape` lives (built or not), or None when it has no tiles."""
    src = module_source(shape)
    if src is None:
        return None
    return CACHE / f"trk_mod_{shape.key}_{_fingerprint(src)}.so"


def build_module(shape: tilegen.ShapeDecl, verbose: bool = False) -> Path | None:
    """The path of the compiled module of `shape`, compiling it if needed (one process at a
    time per module; others wait and reuse it). None when the shape has no tiles."""
    src = module_source(shape)
    if src is None:
        return None
    path = CACHE / f"trk_mod_{shape.key}_{_fingerprint(src)}.so"
    if path.exists():
        return path
    CACHE.mkdir(parents=True, exist_ok=True)
    with open(path.with_suffix(".lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        if path.exists():
            return path
        source = path.with_suffix(".hip")
        source.write_text(src)
        tmp = path.with_name(path.name + f".tmp{os.getpid()}")
        # no run path: the module is only ever loaded into a process that has loaded
        # libtrk.so (trk_plan_load_module), whose SONAME satisfies the dependency, so a copy
        # of the tree at another path binds to its own library and never to this checkout's
        cmd = [build_ext._hipcc(), *build_ext.HIPCC_FLAGS, "-x", "hip", str(source), "-o",
               str(tmp), f"-L{PACKAGE}", *LINK_FLAGS]
        if verbose:
            print(" ".join(cmd), flush=True)
        done = subprocess.run(cmd, capture_output=True, text=True)
        if done.returncode != 0:
            tmp.unlink(missing_ok=True)
            raise RuntimeError(f"hipcc failed on the variant module of {shape.key}:\n"
                               f"{done.stderr[-4000:]}")
        os.replace(tmp, path)
    return path

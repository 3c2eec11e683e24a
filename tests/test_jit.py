"""Prepare-time variant modules (factorized_inference/jit.py) and padded plans, host side:
the kernel-rank rule, the generated module source, building and caching, loading into a plan
through trk_plan_load_module, and the work a padded plan reports. No GPU needed (hipcc
cross-compiles; dlopen of a HIP module works without a device)."""
from __future__ import annotations

import pytest
import torch

from factorized_inference import TRSpec, _lib, jit, tilegen
from factorized_inference.tr_kernel import make_plan
from jit_shapes import JIT_SHAPES


def test_kernel_rank_rule():
    assert [jit.kernel_rank(r) for r in (1, 4, 7, 8)] == [8] * 4
    assert [jit.kernel_rank(r) for r in (9, 12, 16)] == [16] * 3
    assert [jit.kernel_rank(r) for r in (17, 24, 32)] == [32] * 3
    assert jit.kernel_rank(33) is None


def test_module_source_keeps_only_ranged_tiles():
    shape = tilegen.ShapeDecl("t", (4, 6, 8), (6, 4, 8), 16, "f16")
    src = jit.module_source(shape)
    entries = [ln for ln in src.splitlines() if "TRK_ENTRY(" in ln]
    assert entries and not any(ln.split("//")[0].rstrip().endswith(", 0, 0)") for ln in entries)
    for symbol in ("trk_module_register", "trk_module_plan_size", "trk_module_abi"):
        assert symbol in src
    # no tile fits this shape (12 inputs, no contiguous first-core order): no module
    assert jit.module_source(tilegen.ShapeDecl("t", (2, 3, 2), (2, 4, 3), 8, "f16")) is None


def test_module_is_built_once_and_reused():
    shape = tilegen.ShapeDecl("t", (4, 6, 8), (6, 4, 8), 8, "f16")
    path = jit.build_module(shape)
    assert path is not None and path.exists() and path == jit.module_path(shape)
    stamp = path.stat().st_mtime_ns
    assert jit.build_module(shape) == path and path.stat().st_mtime_ns == stamp


@pytest.mark.parametrize("ins,outs,rank,dtype", JIT_SHAPES)
def test_undeclared_shapes_get_mfma_variants(ins, outs, rank, dtype):
    spec = TRSpec(ins, outs, rank)
    dt = getattr(torch, dtype)
    plan = make_plan(spec, dt)
    assert plan.has_mfma
    assert plan.kernel_rank == jit.kernel_rank(rank)
    for tokens in (1, 8, 64, 1000):
        assert plan.describe(-1, tokens)["kind"] == "mfma", tokens
    # the work reported is the rank-`rank` operator's, whatever rank the kernels run at
    code = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16,
            torch.float32: _lib.DTYPE_F32}[dt]
    unpadded = _lib.Plan(ins, outs, rank, code)
    for tokens in (1, 7):
        assert plan.describe(-1, tokens)["bytes"] == unpadded.describe(0, tokens)["bytes"]
    params = sum(rank * rank * i * o for i, o in zip(ins, outs))
    elem = dt.itemsize
    assert plan.describe(-1, 1)["bytes"] == elem * (params + spec.in_features + spec.out_features)


def test_module_names_do_not_depend_on_the_checkout_path(monkeypatch):
    # the tree is copied to other paths (a GPU box): modules built here must keep their names
    from factorized_inference import build_ext
    shape = tilegen.ShapeDecl("prepared", (4, 6, 8), (6, 4, 8), 8, "f16")
    here = jit.module_path(shape)
    moved = [f"-I/elsewhere/{f[2:].lstrip('/')}" if f.startswith("-I") else f
             for f in build_ext.HIPCC_FLAGS]
    monkeypatch.setattr(build_ext, "HIPCC_FLAGS", moved)
    assert jit.module_path(shape) == here
    monkeypatch.setattr(build_ext, "HIPCC_FLAGS", moved + ["-O2"])
    assert jit.module_path(shape) != here


def test_disabled_jit_keeps_the_generic_kernel(monkeypatch):
    spec = TRSpec((4, 6, 8), (6, 4, 8), 8)
    monkeypatch.setenv("TRK_JIT", "0")
    for dtype in (torch.float16, torch.float32):
        assert not make_plan(spec, dtype).has_mfma


def test_loader_rejects_other_libraries():
    from factorized_inference import _trkcall

    plan = _lib.Plan((4, 6, 8), (6, 4, 8), 8, _lib.DTYPE_F16)
    with pytest.raises(_lib.TrkError, match="not a variant module"):
        plan.load_module(_trkcall.__file__)
    with pytest.raises(_lib.TrkError):
        plan.load_module("/nonexistent/trk_mod.so")


def test_module_binds_to_the_library_of_a_relocated_tree(tmp_path):
    # A copy of the tree at another path (a GPU box) loads its modules against its own
    # libtrk.so: the module carries no path to the library, and the SONAME of the copy the
    # process loaded satisfies its dependency. Checked in a fresh process that loads only
    # the copy, with the maps listing exactly one libtrk.so.
    import shutil
    import subprocess
    import sys

    from factorized_inference import build_ext

    shape = tilegen.ShapeDecl("prepared", (4, 6, 8), (6, 4, 8), 8, "f16")
    built = jit.build_module(shape)
    pkg = tmp_path / "moved" / "factorized_inference"
    shutil.copytree(build_ext.PACKAGE, pkg, ignore=shutil.ignore_patterns("__pycache__"))
    module = tmp_path / "moved" / "_jit" / built.name
    module.parent.mkdir()
    shutil.copy(built, module)
    script = (
        "import sys\n"
        f"sys.path.insert(0, {str(pkg.parent)!r})\n"
        "from factorized_inference import _lib\n"
        "plan = _lib.Plan((4, 6, 8), (6, 4, 8), 8, _lib.DTYPE_F16)\n"
        f"added = plan.load_module({str(module)!r})\n"
        "maps = sorted({l.split()[-1] for l in open('/proc/self/maps') if 'libtrk.so' in l})\n"
        "print(added, plan.has_mfma, *maps)\n")
    done = subprocess.run([sys.executable, "-c", script], capture_output=True, text=True,
                          timeout=300)
    assert done.returncode == 0, done.stderr[-2000:]
    added, has_mfma, *maps = done.stdout.split()
    assert int(added) > 0 and has_mfma == "True"
    assert maps == [str(pkg / "libtrk.so")]

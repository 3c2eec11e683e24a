"""CPU tests of the host side: the reference API mirror and the C ABI's host logic.

No GPU work runs here. The library is loaded and its plan logic (host-only) is exercised;
every kernel launch is covered by the gpu-marked tests.
"""
from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest
import torch

from factorized_inference import (
    TRSpec, dense_forward, make_cores, materialize_dense_weight, prepare_optimized,
    tr_forward_optimized, tr_forward_reference,
)
from factorized_inference import _lib
from oracle import ring_oracle as orc

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = Path(__file__).parent / "golden"


def oracle64(x, cores):
    return torch.from_numpy(orc.tr_forward(x.double().numpy(), [c.double().numpy() for c in cores]))


# ---- TRSpec (reference.py:15-50; tests/test_benchmark.py:18, :26-27) ------------------------
def test_spec_known_answers():
    spec = TRSpec((2, 2, 2), (2, 3, 2), 2)
    assert spec.dense_parameters == 96
    assert spec.factor_parameters == 56
    default = TRSpec()
    assert (default.in_features, default.out_features) == (1920, 2880)
    assert default.factor_parameters == 44_544
    assert TRSpec(rank=16).factor_parameters == 178_176
    assert TRSpec((16, 16, 16), (16, 28, 32), 8).factor_parameters == 77_824
    assert TRSpec((16, 28, 32), (16, 16, 16), 16).factor_parameters == 311_296


@pytest.mark.parametrize("args", [((2, 2), (2, 2, 2), 2), ((2, 2, 2), (2, 2, 2, 2), 2),
                                  ((2, 0, 2), (2, 2, 2), 2), ((2, 2, 2), (2, 2, 2), 0)])
def test_spec_rejects_bad_shapes(args):
    with pytest.raises(ValueError):
        TRSpec(*args)


# ---- make_cores (reference.py:53-77) --------------------------------------------------------
def test_make_cores_matches_reference_values():
    golden = np.load(GOLDEN / "reference_cores.npz")
    specs = {
        "s232_243_r2_seed0": (TRSpec((2, 3, 2), (2, 4, 3), 2), 0, torch.float32),
        "s444_444_r8_seed19": (TRSpec((4, 4, 4), (4, 4, 4), 8), 19, torch.float32),
        "s222_232_r2_seed0": (TRSpec((2, 2, 2), (2, 3, 2), 2), 0, torch.float32),
        "s232_243_r3_seed1_f16": (TRSpec((2, 3, 2), (2, 4, 3), 3), 1, torch.float16),
        "s232_243_r3_seed2_bf16": (TRSpec((2, 3, 2), (2, 4, 3), 3), 2, torch.bfloat16),
    }
    for name, (spec, seed, dtype) in specs.items():
        cores = make_cores(spec, seed=seed, dtype=dtype)
        for k, core in enumerate(cores):
            assert core.dtype == dtype
            assert core.shape == (spec.rank, spec.output_modes[k], spec.input_modes[k], spec.rank)
            np.testing.assert_array_equal(core.float().numpy(), golden[f"{name}/g{k + 1}"])


def test_make_cores_scales_and_uniform_init():
    spec = TRSpec((16, 16, 16), (16, 28, 32), 8)
    per_core = make_cores(spec, seed=0)
    uniform = make_cores(spec, seed=0, init="uniform")
    sigma = (spec.in_features * spec.rank ** 3) ** (-1 / 6)
    for k, (a, b) in enumerate(zip(per_core, uniform)):
        # every i_k = 16 here, so the two inits coincide up to rounding of the scale factor
        torch.testing.assert_close(a, b, rtol=1e-6, atol=0)
        assert abs(b.std().item() / sigma - 1) < 0.05
    with pytest.raises(ValueError):
        make_cores(spec, init="xavier")


# ---- the reference path on CPU (reference.py:99-149; tests/test_correctness.py:26-46) -------
@pytest.mark.parametrize("seed", [0, 19])
@pytest.mark.parametrize("spec", [TRSpec((2, 3, 2), (2, 4, 3), 2), TRSpec((4, 4, 4), (4, 4, 4), 8),
                                  TRSpec((4, 4, 4), (4, 4, 4), 16)])
def test_cpu_reference_numerics_and_changing_inputs(spec, seed):
    cores = make_cores(spec, seed=seed)
    original = tuple(c.clone() for c in cores)
    generator = torch.Generator().manual_seed(seed + 37)
    for tokens, scale in [(1, 1.0), (5, 0.0), (3, 0.1), (1, 2.0)]:
        x = torch.randn(tokens, spec.in_features, generator=generator) * scale
        x0 = x.clone()
        y = tr_forward_reference(x, cores, spec)
        assert y.shape == (tokens, spec.out_features) and y.dtype == torch.float32
        torch.testing.assert_close(y.double(), oracle64(x0, original), rtol=1e-4, atol=1e-4)
        torch.testing.assert_close(x, x0, rtol=0, atol=0)
        for c, c0 in zip(cores, original):
            torch.testing.assert_close(c, c0, rtol=0, atol=0)


def test_dense_weight_and_forward_match_oracle():
    spec = TRSpec((3, 2, 5), (4, 3, 6), 3)
    cores = make_cores(spec, seed=5, dtype=torch.float64)
    w = materialize_dense_weight(cores, spec)
    np.testing.assert_allclose(w.numpy(), orc.dense_weight([c.numpy() for c in cores]), atol=1e-12)
    x = torch.randn(4, spec.in_features, dtype=torch.float64)
    np.testing.assert_allclose(dense_forward(x, w).numpy(),
                               orc.tr_forward(x.numpy(), [c.numpy() for c in cores]), atol=1e-12)


def test_reference_validates_shapes():
    spec = TRSpec((2, 3, 2), (2, 4, 3), 2)
    cores = make_cores(spec)
    with pytest.raises(ValueError):
        tr_forward_reference(torch.zeros(2, spec.in_features + 1), cores, spec)
    with pytest.raises(ValueError):
        tr_forward_reference(torch.zeros(spec.in_features), cores, spec)
    with pytest.raises(ValueError):
        tr_forward_reference(torch.zeros(1, spec.in_features), cores[:2], spec)
    with pytest.raises(ValueError):
        tr_forward_reference(torch.zeros(1, spec.in_features), (cores[0], cores[2], cores[1]), spec)


def test_optimized_path_never_runs_on_the_cpu():
    spec = TRSpec((2, 3, 2), (2, 4, 3), 2)
    cores = make_cores(spec)
    with pytest.raises(RuntimeError, match="ROCm device"):
        prepare_optimized(cores, spec)
    with pytest.raises(RuntimeError, match="ROCm device"):
        tr_forward_optimized(torch.zeros(1, spec.in_features), cores, spec)


# ---- the C ABI: symbols and host-only plan logic ---------------------------------------------
def declared_symbols():
    text = (ROOT / "include" / "trk.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(trk_[a-z_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = declared_symbols()
    assert len(declared) >= 14
    assert set(declared) == set(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.trk_abi_version() == _lib.ABI_VERSION
    assert lib.trk_empty_call() == 0


def test_c_program_uses_the_abi(tmp_path):
    """A C host program compiled against include/trk.h and linked to libtrk.so: the boundary
    as another language's binding sees it (host-side entry points, no GPU needed)."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc is not available")
    lib_dir = _lib.LIBRARY.parent
    exe = tmp_path / "c_abi_check"
    subprocess.run([gcc, "-std=c11", "-Wall", "-Werror", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "c_abi_check.c"), "-o", str(exe), f"-L{lib_dir}",
                    "-l:libtrk.so", f"-Wl,-rpath,{lib_dir}"], check=True)
    done = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert done.returncode == 0, done.stdout + done.stderr
    assert "all checks passed" in done.stdout


def test_call_bindings_load_and_check_their_arguments():
    from factorized_inference import _trkcall, _trktorch

    assert callable(_trkcall.forward) and callable(_trkcall.forward_variant)
    plan = _lib.Plan((2, 3, 2), (2, 4, 3), 2, _lib.DTYPE_F16)
    with pytest.raises(ValueError, match="null plan"):
        _trktorch.bind(0, 0, 12, 24, _lib.DTYPE_F16, 0)
    with pytest.raises(ValueError, match="unknown dtype"):
        _trktorch.bind(plan.handle, 256, 12, 24, 7, 0)
    bound = _trktorch.bind(plan.handle, 256, 12, 24, _lib.DTYPE_F16, 0)
    # inputs the C++ path does not take come back as None (no launch happens for them)
    assert _trktorch.forward(bound, torch.zeros(1, 12, dtype=torch.float16)) is None
    assert _trktorch.forward(bound, "not a tensor") is None
    with pytest.raises(TypeError):
        _trktorch.forward(bound)


def test_call_slot_takes_the_native_path_or_the_checked_one():
    # _trktorch.Op, the base of PreparedTRKernel: a call with one argument that the C++ path
    # takes runs there; every other call (unbound object, x it declines, more arguments)
    # goes to the instance's _checked_call with the same arguments
    from factorized_inference import _trktorch
    from factorized_inference.tr_kernel import PreparedTRKernel

    assert issubclass(PreparedTRKernel, _trktorch.Op)
    assert "__call__" not in vars(PreparedTRKernel)  # the call is the base's C++ slot

    class Probe(_trktorch.Op):
        def _checked_call(self, *args, **kwargs):
            return "checked", args, kwargs

    p = Probe()
    assert p("x") == ("checked", ("x",), {})           # not bound yet
    plan = _lib.Plan((2, 3, 2), (2, 4, 3), 2, _lib.DTYPE_F16)
    with pytest.raises(ValueError, match="null plan"):
        p._bind_native(0, 0, 12, 24, _lib.DTYPE_F16, 0)
    p._bind_native(plan.handle, 256, 12, 24, _lib.DTYPE_F16, 0)
    x = torch.zeros(1, 12, dtype=torch.float16)         # on the CPU: the C++ path declines
    assert p(x)[0] == "checked" and p(x)[1][0] is x
    assert p(x, 1) == ("checked", (x, 1), {})
    assert p(x, epilogue=1)[2] == {"epilogue": 1}


@pytest.mark.parametrize("ins,outs,R,dtype", [
    ((8, 12, 20), (12, 10, 24), 8, _lib.DTYPE_F16),
    ((8, 12, 20), (12, 10, 24), 16, _lib.DTYPE_F16),
    ((16, 16, 16), (16, 28, 32), 8, _lib.DTYPE_BF16),
    ((16, 28, 32), (16, 16, 16), 16, _lib.DTYPE_BF16),
    ((2, 3, 2), (2, 4, 3), 2, _lib.DTYPE_F32),
    ((3, 2, 5), (4, 3, 6), 3, _lib.DTYPE_F16),
])
def test_plan_host_logic(ins, outs, R, dtype):
    plan = _lib.Plan(ins, outs, R, dtype)
    elem = 4 if dtype == _lib.DTYPE_F32 else 2
    factors = sum(R * o * i * R for o, i in zip(outs, ins))
    assert plan.packed_bytes >= elem * factors          # packing never drops a value
    assert plan.packed_bytes <= elem * factors * 4 + 6 * 3 * 256  # ...and expands by padding only
    assert plan.variant_count >= 1
    generic = plan.describe(0, 1)
    assert generic["kind"] == "generic"
    # the generic variant runs the order with the fewest flops
    counts = {o: orc.flops_per_token(ins, outs, R, o) for o in orc.CHAIN_ORDERS}
    assert abs(generic["flops"] - min(counts.values())) <= 1e-6 * generic["flops"]
    for tokens in (1, 8, 32, 256):
        index = plan.select(tokens)
        info = plan.describe(-1, tokens)
        assert info == plan.describe(index, tokens)
        assert info["flops"] == pytest.approx(counts[tuple(info["order"])] * tokens)
        in_f, out_f = int(np.prod(ins)), int(np.prod(outs))
        assert info["bytes"] == pytest.approx(elem * (factors + tokens * (in_f + out_f)))
        assert info["lds_bytes"] <= 160 * 1024
        assert min(info["grid"]) >= 1


def test_plan_errors_and_variant_routing():
    with pytest.raises(_lib.TrkError, match="modes must be positive"):
        _lib.Plan((2, 0, 2), (2, 2, 2), 2, _lib.DTYPE_F16)
    with pytest.raises(_lib.TrkError, match="unknown dtype"):
        _lib.Plan((2, 2, 2), (2, 2, 2), 2, 7)
    with pytest.raises(_lib.TrkError, match="rank"):
        _lib.Plan((2, 2, 2), (2, 2, 2), 0, _lib.DTYPE_F16)
    plan = _lib.Plan((8, 12, 20), (12, 10, 24), 8, _lib.DTYPE_F16)
    with pytest.raises(_lib.TrkError):
        plan.set_variant(1, 4, plan.variant_count)
    with pytest.raises(_lib.TrkError):
        plan.describe(plan.variant_count, 1)
    last = plan.variant_count - 1
    plan.set_variant(3, 5, last)
    assert [plan.select(t) for t in (3, 4, 5)] == [last] * 3
    plan.set_variant(1, 1 << 20, 0)
    assert all(plan.select(t) == 0 for t in (1, 2, 7, 64, 1000))
    lib = _lib.load()
    # forward argument checks happen before any device work
    assert lib.trk_forward(plan.handle, None, None, None, 0, None) == _lib.OK   # T = 0: no launch
    assert lib.trk_forward(plan.handle, None, None, None, -1, None) == _lib.ERR_INVALID
    assert lib.trk_forward(plan.handle, None, None, None, 1, None) == _lib.ERR_INVALID
    assert b"null buffer" in lib.trk_last_error()
    assert lib.trk_forward_variant(plan.handle, 99, 1, 1, 1, 1, None) == _lib.ERR_INVALID


def test_forward_swiglu_argument_checks():
    """trk_forward_swiglu checks its plans before any device work: they must agree in shape,
    dtype and rank; a selected variant without a fused gate/up kernel is TRK_ERR_UNSUPPORTED
    (the caller's cue to run the two-launch chain); tokens = 0 launches nothing."""
    lib = _lib.load()
    call = lib.trk_forward_swiglu
    a = _lib.Plan((8, 12, 20), (12, 10, 24), 8, _lib.DTYPE_F16)
    b = _lib.Plan((8, 12, 20), (12, 10, 24), 8, _lib.DTYPE_F16)
    for other in (_lib.Plan((8, 12, 20), (12, 10, 24), 16, _lib.DTYPE_F16),
                  _lib.Plan((8, 12, 20), (12, 10, 24), 8, _lib.DTYPE_BF16),
                  _lib.Plan((8, 12, 20), (10, 12, 24), 8, _lib.DTYPE_F16)):
        assert call(a.handle, None, other.handle, None, None, None, 1, None) == _lib.ERR_INVALID
        assert b"differ" in lib.trk_last_error()
    assert call(None, None, b.handle, None, None, None, 1, None) == _lib.ERR_INVALID
    assert call(a.handle, None, b.handle, None, None, None, -1, None) == _lib.ERR_INVALID
    assert call(a.handle, None, b.handle, None, None, None, 0, None) == _lib.OK
    assert call(a.handle, None, b.handle, None, None, None, 1, None) == _lib.ERR_UNSUPPORTED
    # the Llama-3-8B up projection has fused kernels in every tuned token range: past the
    # variant check, the buffers are checked
    g = _lib.Plan((16, 16, 16), (16, 28, 32), 8, _lib.DTYPE_BF16)
    u = _lib.Plan((16, 16, 16), (16, 28, 32), 8, _lib.DTYPE_BF16)
    for tokens in (1, 2, 5, 33, 200, 4096):
        assert call(g.handle, None, u.handle, None, None, None, tokens, None) == _lib.ERR_INVALID
        assert b"null buffer" in lib.trk_last_error()

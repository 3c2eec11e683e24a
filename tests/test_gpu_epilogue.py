"""GPU parity of the output epilogues (through the C ABI) against the CPU oracle.

The reference's fp32-output path and its consumers (PreparedTRKernel.accumulate,
tr_kernel.py:230-243; consume_silu_mul / consume_add, csrc/v3g/bind.cu:96-149; the MLP
block of tools/v3g_fp32out.py) restated as kernel epilogues:
  - accumulate(x) is the kernel's fp32 accumulator: within tolerance of the oracle, and
    the 16-bit forward is exactly its rounding;
  - forward_add / forward_silu_mul equal the fp32 add or SiLU gate applied to that
    accumulator and rounded once (bitwise for the add, within one rounding for the gate);
  - consume_silu_mul / consume_add against torch and the oracle, odd sizes and misaligned
    views included;
  - a Llama-3-8B-shaped SwiGLU MLP block (gate, up, down, residual) against the oracle.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from factorized_inference import TRSpec, make_cores, prepare_optimized
from factorized_inference import _lib
from factorized_inference.tr_kernel import consume_add, consume_silu_mul, forward_swiglu
from gpu_util import TOLERANCE, check_result, oracle_y
from oracle import ring_oracle as orc

pytestmark = pytest.mark.gpu

DEFAULT = dict(input_modes=(8, 12, 20), output_modes=(12, 10, 24))
LLAMA_UP = dict(input_modes=(16, 16, 16), output_modes=(16, 28, 32))
LLAMA_DOWN = dict(input_modes=(16, 28, 32), output_modes=(16, 16, 16))
ODD = dict(input_modes=(3, 2, 5), output_modes=(4, 3, 6))
QWEN_GATE_UP = dict(input_modes=(20, 16, 16), output_modes=(16, 34, 32))


def gpu_randn(shape, seed, dtype):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(*shape, generator=g, device="cuda", dtype=dtype)


def announce(**case):
    print("case:", ", ".join(f"{k}={v}" for k, v in case.items()), flush=True)


def check_epilogue(actual: torch.Tensor, y_ref: np.ndarray, kind: str, aux: torch.Tensor,
                   dtype: torch.dtype) -> None:
    """An epilogue output against the oracle: the operator's error allowance (the reference's
    |err| <= tol + tol*|y|) carried through the epilogue, which scales it by |silu(a)| for
    the gate (1 for the add), plus one rounding of the output.

        |actual - e(y)| <= |s| * (tol + tol*|y|) + eps(dtype) * |e(y)|"""
    tol = TOLERANCE[dtype]
    a = aux.double().cpu().numpy()
    expected = orc.epilogue(kind, y_ref, a)
    scale = np.abs(orc.silu(a)) if kind == "silu_mul" else 1.0
    bound = scale * (tol + tol * np.abs(y_ref)) + torch.finfo(dtype).eps * np.abs(expected)
    got = actual.double().cpu().numpy()
    assert actual.dtype == dtype and got.shape == expected.shape and np.isfinite(got).all()
    excess = np.abs(got - expected) - bound
    assert (excess <= 0).all(), (kind, float(excess.max()), int(np.argmax(excess)))


def check_activation(act: torch.Tensor, g64: np.ndarray, u64: np.ndarray,
                     dtype: torch.dtype) -> None:
    """silu(G x) * (U x) against the oracle's gate and up outputs: both errors (each within
    the operator's tol + tol*|.|) carried through silu(g) * u (|silu'| <= 1.1), plus one
    rounding of the output."""
    tol = TOLERANCE[dtype]
    a64 = orc.epilogue("silu_mul", u64, g64)
    got = act.double().cpu().numpy()
    assert act.dtype == dtype and got.shape == a64.shape and np.isfinite(got).all()
    bound = (1.1 * np.abs(u64) * (tol + tol * np.abs(g64))
             + np.abs(orc.silu(g64)) * (tol + tol * np.abs(u64))
             + torch.finfo(dtype).eps * np.abs(a64))
    excess = np.abs(got - a64) - bound
    assert (excess <= 0).all(), (float(excess.max()), int(np.argmax(excess)))


CASES = [
    (DEFAULT, 8, torch.float16, (1, 8, 32)),
    (DEFAULT, 16, torch.float16, (1, 32)),
    (LLAMA_UP, 8, torch.bfloat16, (1, 32)),
    (LLAMA_DOWN, 16, torch.bfloat16, (1, 32)),
    (ODD, 3, torch.float16, (1, 5)),      # generic kernel
    (ODD, 3, torch.float32, (1, 5)),      # generic kernel, fp32 plan
]


def _prepare(shape, rank, dtype, seed):
    spec = TRSpec(rank=rank, **shape)
    init = "uniform" if dtype == torch.bfloat16 else "per_core"
    cores = make_cores(spec, device="cuda", dtype=dtype, seed=seed, init=init)
    return spec, cores, prepare_optimized(cores, spec)


@pytest.mark.parametrize("shape,rank,dtype,tokens", CASES)
def test_accumulate_add_and_silu_mul(shape, rank, dtype, tokens):
    spec, cores, run = _prepare(shape, rank, dtype, seed=11)
    tol = TOLERANCE[dtype]
    for T in tokens:
        announce(test="epilogues", shape=shape, rank=rank, dtype=dtype, tokens=T)
        x = gpu_randn((T, spec.in_features), 200 + T, dtype)
        expected = oracle_y(x, cores, spec)
        y32 = run.accumulate(x)
        y = run(x)
        torch.cuda.synchronize()
        assert y32.dtype == torch.float32 and y32.shape == (T, spec.out_features)
        # the fp32 accumulator: at least as close to the oracle as the rounded output
        check_result(y32.to(dtype), expected, dtype)
        err32 = np.abs(y32.double().cpu().numpy() - expected).max()
        assert err32 <= tol * (1.0 + np.abs(expected).max())
        # the default store is exactly the rounding of that accumulator
        assert torch.equal(y, y32.to(dtype))
        # residual add, residual in the plan's dtype and in fp32: the fp32 sum rounded once
        for h in (gpu_randn((T, spec.out_features), 300 + T, dtype),
                  gpu_randn((T, spec.out_features), 400 + T, torch.float32)):
            y_add = run.forward_add(x, h)
            assert y_add.dtype == dtype
            assert torch.equal(y_add, (h.float() + y32).to(dtype))
            check_epilogue(y_add, expected, "add", h, dtype)
        # SwiGLU gate: silu(g) * y in fp32, rounded once; g fp32 (an accumulate() output) or
        # in the plan's dtype
        for g in (gpu_randn((T, spec.out_features), 500 + T, torch.float32) * 3.0,
                  gpu_randn((T, spec.out_features), 600 + T, dtype)):
            y_gate = run.forward_silu_mul(x, g)
            assert y_gate.dtype == dtype
            ref32 = F.silu(g.float()) * y32
            # the kernel's exp and torch's differ by a few fp32 ulps, so the results are at
            # most one output rounding apart (relative 2 eps; 1e-5 for fp32 outputs, 1e-6
            # absolute below the fp16 normal range)
            torch.testing.assert_close(y_gate.float(), ref32.to(dtype).float(),
                                       rtol=max(2 * torch.finfo(dtype).eps, 1e-5), atol=1e-6)
            check_epilogue(y_gate, expected, "silu_mul", g, dtype)


def test_every_variant_takes_every_epilogue():
    spec, cores, run = _prepare(DEFAULT, 8, torch.float16, seed=12)
    x = gpu_randn((7, spec.in_features), 7, torch.float16)
    h = gpu_randn((7, spec.out_features), 8, torch.float16)
    for variant, info in enumerate(run.variants()):
        announce(test="variant epilogues", variant=info["name"])
        y32 = run.run_variant(x, variant, _lib.EPI_F32)
        assert torch.equal(run.run_variant(x, variant), y32.to(torch.float16))
        assert torch.equal(run.run_variant(x, variant, _lib.EPI_ADD, h),
                           (h.float() + y32).to(torch.float16))
        y_gate = run.run_variant(x, variant, _lib.EPI_SILU_MUL, h)
        torch.testing.assert_close(y_gate.float(), (F.silu(h.float()) * y32).half().float(),
                                   rtol=2e-3, atol=1e-6)


def test_in_place_epilogue_through_the_c_abi():
    """aux may be y itself: each element is read before its own store."""
    spec, cores, run = _prepare(DEFAULT, 8, torch.float16, seed=13)
    x = gpu_randn((4, spec.in_features), 9, torch.float16)
    y32 = run.accumulate(x)
    h = gpu_randn((4, spec.out_features), 10, torch.float16)
    buf = h.clone()
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(run._forward_epilogue(run._plan_handle, -1, run._packed_ptr, x.data_ptr(),
                                     buf.data_ptr(), 4, _lib.EPI_ADD, buf.data_ptr(),
                                     _lib.DTYPE_F16, stream))
    torch.cuda.synchronize()
    assert torch.equal(buf, (h.float() + y32).half())


def test_epilogue_argument_errors():
    spec, cores, run = _prepare(DEFAULT, 8, torch.float16, seed=14)
    x = gpu_randn((2, spec.in_features), 11, torch.float16)
    with pytest.raises(ValueError, match="shape"):
        run.forward_add(x, torch.zeros(3, spec.out_features, device="cuda", dtype=torch.float16))
    with pytest.raises(ValueError, match="float16 or float32"):
        run.forward_silu_mul(x, torch.zeros(2, spec.out_features, device="cuda",
                                            dtype=torch.bfloat16))
    with pytest.raises(ValueError):
        run.forward_add(x, torch.zeros(2, spec.out_features, dtype=torch.float16))  # on the CPU
    lib = _lib.load()
    y = torch.empty(2, spec.out_features, device="cuda", dtype=torch.float16)
    args = (run._plan_handle, -1, run._packed_ptr, x.data_ptr(), y.data_ptr(), 2)
    assert lib.trk_forward_epilogue(*args, 7, None, 0, None) == _lib.ERR_INVALID
    assert lib.trk_forward_epilogue(*args, _lib.EPI_ADD, None, 0, None) == _lib.ERR_INVALID
    assert lib.trk_forward_epilogue(*args, _lib.EPI_ADD, y.data_ptr(), _lib.DTYPE_BF16,
                                    None) == _lib.ERR_INVALID
    # a non-contiguous residual goes through the checked path, which copies it
    h = gpu_randn((spec.out_features, 2), 12, torch.float16).t()
    assert torch.equal(run.forward_add(x, h), (h.float() + run.accumulate(x)).half())


@pytest.mark.parametrize("n", [0, 1, 3, 4, 1000, 14336 * 5 + 3])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_consumers(n, dtype):
    announce(test="consumers", n=n, dtype=dtype)
    g = gpu_randn((n,), 1, torch.float32) * 4.0
    u = gpu_randn((n,), 2, torch.float32)
    h = gpu_randn((n,), 3, dtype)
    out = consume_silu_mul(g, u, dtype)
    assert out.dtype == dtype and out.shape == g.shape
    ref = torch.from_numpy(orc.silu(g.double().cpu().numpy()) * u.double().cpu().numpy())
    eps = max(torch.finfo(dtype).eps, 1e-5)  # one output rounding; fp32: the exp's error
    torch.testing.assert_close(out.double().cpu(), ref, rtol=eps, atol=1e-6)
    added = consume_add(h, u)
    assert torch.equal(added, (h.float() + u).to(dtype))
    g0, u0 = g.clone(), u.clone()
    torch.cuda.synchronize()
    assert torch.equal(g, g0) and torch.equal(u, u0)   # inputs only read
    if n > 8:  # misaligned views take the scalar kernels
        gs, us, hs = g[1:], u[1:], h[1:]
        torch.testing.assert_close(consume_silu_mul(gs, us, dtype).double().cpu(), ref[1:],
                                   rtol=eps, atol=1e-6)
        assert torch.equal(consume_add(hs, us), (hs.float() + us).to(dtype))


def test_consumer_argument_errors():
    g = torch.zeros(8, device="cuda")
    with pytest.raises(ValueError):
        consume_silu_mul(g, torch.zeros(7, device="cuda"))
    with pytest.raises(ValueError):
        consume_silu_mul(g.half(), g.half())
    with pytest.raises(ValueError):
        consume_add(g.half(), g.half())


def test_llama_swiglu_mlp_block():
    """h + down(silu(gate(x)) * up(x)) with the Llama-3-8B shapes (gate/up 4096 -> 14336 at
    rank 8, down 14336 -> 4096 at rank 16, bf16): the fused three-launch chain against the
    oracle, and against the unfused torch chain."""
    dtype = torch.bfloat16
    spec_up = TRSpec(rank=8, **LLAMA_UP)
    spec_down = TRSpec(rank=16, **LLAMA_DOWN)
    cg = make_cores(spec_up, device="cuda", dtype=dtype, seed=1, init="uniform")
    cu = make_cores(spec_up, device="cuda", dtype=dtype, seed=2, init="uniform")
    cd = make_cores(spec_down, device="cuda", dtype=dtype, seed=3, init="uniform")
    gate, up, down = (prepare_optimized(c, s) for c, s in
                      ((cg, spec_up), (cu, spec_up), (cd, spec_down)))
    for T in (1, 4, 32):
        announce(test="mlp block", tokens=T)
        x = gpu_randn((T, 4096), 20 + T, dtype)
        h = gpu_randn((T, 4096), 40 + T, dtype)
        act = up.forward_silu_mul(x, gate.accumulate(x))
        fused = down.forward_add(act, h)
        unfused = h + down(F.silu(gate(x)) * up(x))
        torch.cuda.synchronize()
        # each launch against the oracle on the inputs it actually received
        g64 = oracle_y(x, cg, spec_up)
        u64 = oracle_y(x, cu, spec_up)
        a64 = orc.epilogue("silu_mul", u64, g64)
        check_activation(act, g64, u64, dtype)
        assert torch.equal(forward_swiglu(gate, up, x), act)
        check_epilogue(fused, oracle_y(act, cd, spec_down), "add", h, dtype)
        h64 = h.double().cpu().numpy()
        # end to end against the float64 chain without intermediate rounding: the fused
        # chain (fp32 gate, one rounding of the activation) is no worse than torch's
        ref = orc.epilogue("add", oracle_y(torch.from_numpy(a64), cd, spec_down), h64)
        err_fused = orc.errors(fused.double().cpu().numpy(), ref)["relative_l2_error"]
        err_unfused = orc.errors(unfused.double().cpu().numpy(), ref)["relative_l2_error"]
        assert err_fused <= max(1.5 * err_unfused, 5e-3), (err_fused, err_unfused)


@pytest.mark.parametrize("shape,rank,tokens", [
    (LLAMA_UP, 8, None),            # the first token count of every tuned range
    (QWEN_GATE_UP, 8, (1, 3, 16)),
    (QWEN_GATE_UP, 16, (1, 3, 16)),
])
def test_forward_swiglu(shape, rank, tokens):
    """The fused gate/up launch (trk_forward_swiglu) against the two-launch chain
    up.forward_silu_mul(x, gate.accumulate(x)), which runs the same variant, the same stage
    code and the same fp32 gate: equal bit for bit. And against the oracle."""
    dtype = torch.bfloat16
    spec = TRSpec(rank=rank, **shape)
    cg = make_cores(spec, device="cuda", dtype=dtype, seed=31, init="uniform")
    cu = make_cores(spec, device="cuda", dtype=dtype, seed=32, init="uniform")
    gate, up = prepare_optimized(cg, spec), prepare_optimized(cu, spec)
    if tokens is None:
        tokens = sorted({v["t_min"] for v in gate.variants()
                         if v["kind"] == "mfma" and 0 < v["t_min"] <= 256})
        assert len(tokens) >= 4  # single-token, mid-size and register-resident tiles
    for T in tokens:
        announce(test="fused gate/up", shape=shape, rank=rank, tokens=T,
                 variant=gate.selected(T)["name"])
        x = gpu_randn((T, spec.in_features), 70 + T, dtype)
        fused = forward_swiglu(gate, up, x)
        two = up.forward_silu_mul(x, gate.accumulate(x))
        torch.cuda.synchronize()
        assert fused.shape == (T, spec.out_features)
        assert torch.equal(fused, two)
        check_activation(fused, oracle_y(x, cg, spec, chunk=64), oracle_y(x, cu, spec, chunk=64),
                         dtype)
    assert forward_swiglu(gate, up, x[:0]).shape == (0, spec.out_features)


def test_forward_swiglu_without_a_fused_kernel():
    """Shapes without a fused kernel give the same result from the two-launch chain; operands
    that do not pair are refused."""
    spec, cores, gate = _prepare(DEFAULT, 8, torch.float16, seed=33)
    up = prepare_optimized(make_cores(spec, device="cuda", dtype=torch.float16, seed=34), spec)
    x = gpu_randn((5, spec.in_features), 13, torch.float16)
    assert torch.equal(forward_swiglu(gate, up, x), up.forward_silu_mul(x, gate.accumulate(x)))
    _, _, other = _prepare(DEFAULT, 16, torch.float16, seed=35)
    with pytest.raises(ValueError, match="one shape"):
        forward_swiglu(gate, other, x)
    with pytest.raises(ValueError):
        forward_swiglu(gate, up, x.float())

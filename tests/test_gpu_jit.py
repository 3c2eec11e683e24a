"""GPU parity of the MFMA variants that shapes without compiled tables get at prepare time
(factorized_inference/jit.py): variant modules for new shapes, and zero-padded ring links for
ranks without kernels (4 and 12 here), against the float64 oracle, through prepare_optimized
and the C ABI (every variant of each plan)."""
from __future__ import annotations

import pytest
import torch

from factorized_inference import TRSpec, _lib, make_cores, prepare_optimized
from gpu_util import check_result, oracle_y
from jit_shapes import JIT_SHAPES

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("ins,outs,rank,dtype", JIT_SHAPES)
def test_prepared_mfma_variants_match_the_oracle(ins, outs, rank, dtype):
    dt = getattr(torch, dtype)
    spec = TRSpec(ins, outs, rank)
    cores = make_cores(spec, device="cuda", dtype=dt, seed=31, init="uniform")
    run = prepare_optimized(cores, spec)
    assert run.plan.has_mfma, "the shape should run MFMA variants"
    g = torch.Generator(device="cuda").manual_seed(rank)
    for tokens in (1, 5, 33, 70):
        print(f"case: jit {ins}->{outs} R{rank} {dtype} T={tokens} "
              f"{run.selected(tokens)['name']}", flush=True)
        x = torch.randn(tokens, spec.in_features, generator=g, device="cuda", dtype=dt)
        y = run(x)
        y32 = run.accumulate(x)
        torch.cuda.synchronize()
        assert run.selected(tokens)["kind"] == "mfma"
        expected = oracle_y(x, cores, spec)
        check_result(y, expected, dt)
        assert torch.equal(y, y32.to(dt)), "the fp32 epilogue must round to the plain store"
    x = torch.randn(3, spec.in_features, generator=g, device="cuda", dtype=dt)
    expected = oracle_y(x, cores, spec)
    for variant, info in enumerate(run.variants(3)):
        print(f"case: jit variant {info['name']}", flush=True)
        check_result(run.run_variant(x, variant), expected, dt)

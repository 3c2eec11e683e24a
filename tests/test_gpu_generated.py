"""GPU parity of the generated MFMA variant tables (factorized_inference/tilegen.py).

Every variant compiled for a declared shape (the BASELINE configs, and the reference's
Qwen3.8-27B layer shapes, tools/qwen_shapes.py:20-27, at ranks 8 and 16 in bf16, as
tools/qwen_bench.py runs them) is checked against the oracle at 1, 5 and 33 tokens, on a
subset of the token rows (rows are independent, so a full-size launch is checked row-exactly
on the rows sampled), with bitwise-identical repeated calls; the plan's default selection
is checked at every token count the autotuner measures.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from factorized_inference import TRSpec, make_cores, prepare_optimized
from factorized_inference import tilegen
from gpu_util import check_result, oracle_y

pytestmark = pytest.mark.gpu

ROWS = {1: [0], 5: [0, 4], 33: [0, 17, 32]}


def announce(**case):
    print("case:", ", ".join(f"{k}={v}" for k, v in case.items()), flush=True)


@pytest.mark.parametrize("shape", tilegen.DECLARED, ids=lambda s: s.key)
def test_every_generated_variant(shape):
    dtype = torch.bfloat16 if shape.dtype == "bf16" else torch.float16
    spec = TRSpec(shape.ins, shape.outs, shape.rank)
    cores = make_cores(spec, device="cuda", dtype=dtype, seed=5, init="uniform")
    run = prepare_optimized(cores, spec)
    variants = [(i, v) for i, v in enumerate(run.variants()) if v["kind"] == "mfma"]
    assert variants, "declared shapes have MFMA variants"
    g = torch.Generator(device="cuda").manual_seed(77)
    for T, rows in ROWS.items():
        x = torch.randn(T, spec.in_features, generator=g, device="cuda", dtype=dtype)
        idx = torch.tensor(rows, device="cuda")
        expected = oracle_y(x[idx], cores, spec)
        for i, info in variants:
            announce(test="generated", shape=shape.key, variant=info["name"], tokens=T)
            y = run.run_variant(x, i)
            y2 = run.run_variant(x, i)
            torch.cuda.synchronize()
            assert torch.equal(y, y2), "repeated calls must be bitwise identical"
            check_result(y[idx], expected, dtype)
        # the default selection takes an MFMA variant at every token count
        assert run.selected(T)["kind"] == "mfma"
        check_result(run(x)[idx], expected, dtype)


def test_generated_selection_covers_all_token_counts():
    for shape in tilegen.DECLARED:
        spec = TRSpec(shape.ins, shape.outs, shape.rank)
        dtype = torch.bfloat16 if shape.dtype == "bf16" else torch.float16
        cores = make_cores(spec, device="cuda", dtype=dtype, seed=1)
        run = prepare_optimized(cores, spec)
        for T in (1, 2, 3, 8, 16, 17, 64, 65, 128, 1000):
            assert run.selected(T)["kind"] == "mfma", (shape.key, T)

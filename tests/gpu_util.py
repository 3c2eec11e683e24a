"""Shared helpers of the GPU parity tests: the oracle call and the acceptance rule."""
from __future__ import annotations

import numpy as np
import torch

from oracle import ring_oracle as orc

# Acceptance (IMPLEMENTATION.md:30-36; benchmarks/benchmark.py:182): elementwise
# |y - y_ref| <= tol + tol*|y_ref| with tol = 0.02 for fp16/bf16 and 1e-4 for fp32, and, for
# 16-bit types, max|y - y_ref| <= 1e-2 * max|y_ref|.
TOLERANCE = {torch.float16: 2e-2, torch.bfloat16: 2e-2, torch.float32: 1e-4}
MAX_ABS_FRACTION = 1e-2


def oracle_y(x: torch.Tensor, cores, spec, chunk: int = 0) -> np.ndarray:
    """float64 oracle output for the exact (already rounded) x and cores, on the CPU.

    Contracts in the cheapest order; every order equals the reference's to ~1e-14
    (tests/test_oracle.py). chunk > 0 runs `chunk` token rows at a time (token rows are
    independent), which bounds the float64 intermediates at large token counts."""
    xs = x.detach().double().cpu().numpy()
    cs = [c.detach().double().cpu().numpy() for c in cores]
    order = min(orc.CHAIN_ORDERS,
                key=lambda o: orc.flops_per_token(spec.input_modes, spec.output_modes, spec.rank, o))
    if chunk <= 0 or xs.shape[0] <= chunk:
        return orc.chain_forward(xs, cs, order)
    return np.concatenate([orc.chain_forward(xs[t:t + chunk], cs, order)
                           for t in range(0, xs.shape[0], chunk)])


def check_result(actual: torch.Tensor, expected: np.ndarray, dtype: torch.dtype) -> dict:
    tol = TOLERANCE[dtype]
    assert actual.dtype == dtype
    assert tuple(actual.shape) == expected.shape
    a = actual.detach().double().cpu()
    assert torch.isfinite(a).all()
    e = torch.from_numpy(np.ascontiguousarray(expected))
    torch.testing.assert_close(a, e, rtol=tol, atol=tol)
    stats = orc.errors(a.numpy(), expected)
    if dtype != torch.float32 and expected.size:
        assert stats["max_absolute_error"] <= MAX_ABS_FRACTION * float(np.abs(expected).max()), stats
    return stats

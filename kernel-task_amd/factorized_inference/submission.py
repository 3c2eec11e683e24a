"""The drop-in boundary: prepare_optimized(cores, spec) -> fn(x).

Mirrors src/factorized_inference/submission.py:10-48 of the reference (same names, argument
meaning and shape errors). One deliberate difference: the reference falls back to its torch
path for CPU cores and for dtype mismatches; here the operator always runs the HIP library,
and anything it cannot run raises instead of taking another path.
"""
from __future__ import annotations

from typing import Callable, Sequence

import torch

from .reference import TRSpec, _validate


def prepare_optimized(
    cores: Sequence[torch.Tensor],
    spec: TRSpec,
) -> Callable[[torch.Tensor], torch.Tensor]:
    """One-time preparation; returns a callable taking x [T, in_features] -> y [T, out_features].

    Packs the cores on their device (fp16, bf16 or fp32 on a ROCm GPU) and returns the HIP
    operator. The cores and x are never modified, the dense weight is never built, one
    prepared callable accepts any token count and values, and callables for different
    weights are independent. Raises RuntimeError for CPU cores or a missing HIP library.
    """
    if not all(isinstance(c, torch.Tensor) and c.device.type == "cuda" for c in cores):
        raise RuntimeError(
            "prepare_optimized runs the HIP kernel and needs the cores on a ROCm device; "
            "tr_forward_reference computes the operator on the CPU")
    from .tr_kernel import PreparedTRKernel

    return PreparedTRKernel(cores, spec)


def tr_forward_optimized(
    x: torch.Tensor,
    cores: Sequence[torch.Tensor],
    spec: TRSpec,
) -> torch.Tensor:
    """One-shot form of prepare_optimized(cores, spec)(x) (reference submission.py:10-23).

    Packs the cores on every call; keep the prepared callable when calling repeatedly.
    """
    _validate(x, cores, spec)
    return prepare_optimized(cores, spec)(x)

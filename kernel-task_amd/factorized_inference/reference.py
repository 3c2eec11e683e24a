"""The operator's harness API: spec, seeded cores, the factorized reference path, the dense
baseline.

Mirrors src/factorized_inference/reference.py of the reference (names, argument meaning,
errors), so that code written against it runs unchanged. These functions are the API's
comparators (the "factorized_reference" and "dense" methods of the harness) and its fp32/
fp64 oracle helpers; the accelerated path is `prepare_optimized` (submission.py), which runs
the HIP library.

Indices: x[t,i,j,k], G1[a,p,i,b], G2[b,q,j,c], G3[c,r,k,a], y[t,p,q,r]; the ring links a, b,
c close the cycle (IMPLEMENTATION.md:7-10).
"""
from __future__ import annotations

from dataclasses import dataclass
from math import prod
from typing import Sequence

import torch


@dataclass(frozen=True)
class TRSpec:
    """Shape of a three-core tensor-ring linear layer (reference.py:15-50).

    Core k has shape [rank, output_modes[k], input_modes[k], rank]; the dense weight it
    represents is [out_features, in_features].
    """

    input_modes: tuple[int, int, int] = (8, 12, 20)
    output_modes: tuple[int, int, int] = (12, 10, 24)
    rank: int = 8

    def __post_init__(self) -> None:
        if len(self.input_modes) != 3 or len(self.output_modes) != 3:
            raise ValueError("Exactly three input and output modes are required")
        if min(*self.input_modes, *self.output_modes, self.rank) <= 0:
            raise ValueError("All modes and the rank must be positive")

    @property
    def in_features(self) -> int:
        return prod(self.input_modes)

    @property
    def out_features(self) -> int:
        return prod(self.output_modes)

    @property
    def factor_parameters(self) -> int:
        return sum(self.rank * o * i * self.rank
                   for o, i in zip(self.output_modes, self.input_modes))

    @property
    def dense_parameters(self) -> int:
        return self.in_features * self.out_features


def make_cores(
    spec: TRSpec,
    *,
    device: torch.device | str = "cpu",
    dtype: torch.dtype = torch.float32,
    seed: int = 0,
    init: str = "per_core",
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Seeded cores G_k ~ N(0, sigma_k^2) of shape [R, o_k, i_k, R] (reference.py:53-77).

    init="per_core" (the reference's, and the default): sigma_k = (R * i_k)^(-1/2). The
    draws are the same calls on one generator seeded with `seed`, in core order, in the
    target dtype on the target device, so the values match the reference's bit for bit.
    init="uniform": every core uses sigma = (in_features * R^3)^(-1/6), the wording of the
    benchmark configs. Both give Var(W) = 1/in_features.
    """
    if init not in ("per_core", "uniform"):
        raise ValueError("init must be 'per_core' or 'uniform'")
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    R = spec.rank
    cores = []
    for o, i in zip(spec.output_modes, spec.input_modes):
        draw = torch.randn(R, o, i, R, generator=generator, device=device, dtype=dtype)
        if init == "per_core":
            scale = 1.0 / (R * i) ** 0.5
        else:
            scale = (spec.in_features * R ** 3) ** (-1.0 / 6.0)
        cores.append(draw * scale)
    return tuple(cores)  # type: ignore[return-value]


def _validate(x: torch.Tensor, cores: Sequence[torch.Tensor], spec: TRSpec) -> None:
    """Shape checks of reference.py:80-96: ValueError on a mismatch."""
    if x.ndim != 2 or x.shape[1] != spec.in_features:
        raise ValueError(
            f"Expected x with shape [tokens, {spec.in_features}], got {tuple(x.shape)}")
    _validate_cores(cores, spec)


def _validate_cores(cores: Sequence[torch.Tensor], spec: TRSpec) -> None:
    if len(cores) != 3:
        raise ValueError(f"Expected three cores, got {len(cores)}")
    for index, (core, o, i) in enumerate(zip(cores, spec.output_modes, spec.input_modes)):
        expected = (spec.rank, o, i, spec.rank)
        if tuple(core.shape) != expected:
            raise ValueError(f"Core {index} should have shape {expected}, got {tuple(core.shape)}")


def tr_forward_reference(
    x: torch.Tensor,
    cores: Sequence[torch.Tensor],
    spec: TRSpec,
) -> torch.Tensor:
    """Direct factorized execution, never forming W (reference.py:99-125).

    Three pairwise contractions in the reference's fixed order, each one permute plus one
    matrix product in the input dtype:
      stage 1  I1[t,j,k,a,p,b] = sum_i       x[t,i,j,k]      G1[a,p,i,b]
      stage 2  I2[t,k,a,p,q,c] = sum_{j,b}   I1[t,j,k,a,p,b] G2[b,q,j,c]
      stage 3  y[t,p,q,r]      = sum_{k,c,a} I2[t,k,a,p,q,c] G3[c,r,k,a]
    """
    _validate(x, cores, spec)
    g1, g2, g3 = cores
    R = spec.rank
    ni, nj, nk = spec.input_modes
    P, Q, Rr = spec.output_modes
    T = x.shape[0]
    xm = x.reshape(T, ni, nj, nk)
    lhs = xm.permute(0, 2, 3, 1).reshape(T * nj * nk, ni)
    i1 = (lhs @ g1.permute(2, 0, 1, 3).reshape(ni, R * P * R)).reshape(T, nj, nk, R, P, R)
    lhs = i1.permute(0, 2, 3, 4, 1, 5).reshape(T * nk * R * P, nj * R)
    i2 = (lhs @ g2.permute(2, 0, 1, 3).reshape(nj * R, Q * R)).reshape(T, nk, R, P, Q, R)
    lhs = i2.permute(0, 3, 4, 1, 5, 2).reshape(T * P * Q, nk * R * R)
    y = lhs @ g3.permute(2, 0, 3, 1).reshape(nk * R * R, Rr)
    return y.reshape(T, spec.out_features)


def materialize_dense_weight(cores: Sequence[torch.Tensor], spec: TRSpec) -> torch.Tensor:
    """The equivalent dense [out_features, in_features] weight (reference.py:128-143).

    For validation and the dense baseline only; the accelerated path never builds it.
    """
    if len(cores) != 3:
        raise ValueError(f"Expected three cores, got {len(cores)}")
    g1, g2, g3 = cores
    R = spec.rank
    ni, nj, nk = spec.input_modes
    P, Q, Rr = spec.output_modes
    ab = (g1.reshape(R * P * ni, R) @ g2.reshape(R, Q * nj * R)).reshape(R, P, ni, Q, nj, R)
    lhs = ab.permute(1, 2, 3, 4, 5, 0).reshape(P * ni * Q * nj, R * R)
    w = (lhs @ g3.permute(0, 3, 1, 2).reshape(R * R, Rr * nk)).reshape(P, ni, Q, nj, Rr, nk)
    return w.permute(0, 2, 4, 1, 3, 5).reshape(spec.out_features, spec.in_features)


def dense_forward(x: torch.Tensor, dense_weight: torch.Tensor) -> torch.Tensor:
    """Dense baseline y = x W^T with a materialised weight (reference.py:146-149)."""
    return torch.nn.functional.linear(x, dense_weight)

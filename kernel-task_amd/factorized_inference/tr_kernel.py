"""Host side of the HIP tensor-ring operator: prepare once, call per input.

Mirrors src/factorized_inference/tr_kernel.py of the reference (PreparedTRKernel, packing at
prepare time, a tiling/variant choice per token count) with its own mechanics:

  prepare  trk_plan_create picks the contraction order(s) and kernel variants for the shape;
           trk_pack packs the cores into one device buffer (no dense W, padding only)
  call     one C++ call per input (_trktorch.forward): check x, allocate the output with
           torch's caching allocator, trk_forward on the caller's current stream. No
           workspace, counters or other state survives a call, so one prepared object may
           be used from several streams. Inputs that need checking or copying go through
           the Python path below, which raises or copies first.

Environment switch (read at prepare time, for sweeps): TRK_VARIANT=<index> routes every
token count to that variant of the plan (indices from `PreparedTRKernel.variants()`).
"""
from __future__ import annotations

import os
from typing import Sequence

import torch

from . import _lib
from .reference import TRSpec, _validate_cores

_DTYPES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16,
           torch.float32: _lib.DTYPE_F32}

_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
if _raw_stream is None:
    _raw_stream = lambda device_index: torch.cuda.current_stream(device_index).cuda_stream  # noqa: E731


def _fast_forward():
    """The CPython fast-call binding of trk_forward (built next to libtrk.so), else ctypes."""
    _lib.load()  # binds and version-checks libtrk.so first
    try:
        from . import _trkcall
    except ImportError:
        lib = _lib.load()
        return lib.trk_forward, lib.trk_forward_variant
    return _trkcall.forward, _trkcall.forward_variant


def _torch_call():
    """_trktorch (built next to libtrk.so): PreparedTRKernel's per-call path in C++."""
    _lib.load()
    try:
        from . import _trktorch
    except ImportError as exc:
        raise RuntimeError(
            f"the _trktorch extension is not built or does not load ({exc}); run "
            "python -m factorized_inference.build_ext") from exc
    return _trktorch


def current_stream_handle(device_index: int) -> int:
    """hipStream_t of torch's current stream on `device_index`, as an integer."""
    return _raw_stream(device_index)


class PreparedTRKernel:
    """Callable returned by prepare_optimized for cores on a ROCm device.

    fp16, bf16 and fp32 cores are supported; x must have the cores' dtype and device. The
    output is a new [T, out_features] tensor written on the caller's current stream.
    """

    def __init__(self, cores: Sequence[torch.Tensor], spec: TRSpec):
        _validate_cores(cores, spec)
        dtype, device = cores[0].dtype, cores[0].device
        if device.type != "cuda":
            raise RuntimeError("PreparedTRKernel needs the cores on a ROCm (cuda) device")
        if any(c.dtype != dtype or c.device != device for c in cores):
            raise ValueError("All three cores must share one dtype and device")
        if dtype not in _DTYPES:
            raise ValueError(f"Unsupported dtype {dtype}; use float16, bfloat16 or float32")
        self.spec = spec
        self.dtype = dtype
        self.device = device
        self.device_index = device.index if device.index is not None else torch.cuda.current_device()
        self.in_features = spec.in_features
        self.out_features = spec.out_features
        self.plan = _lib.Plan(spec.input_modes, spec.output_modes, spec.rank, _DTYPES[dtype])
        forced = os.environ.get("TRK_VARIANT")
        if forced is not None:
            self.plan.set_variant(1, 1 << 30, int(forced))
        with torch.cuda.device(self.device_index):
            self.packed = torch.empty(self.plan.packed_bytes, dtype=torch.uint8, device=device)
            g = [c.contiguous() for c in cores]
            _lib.check(_lib.load().trk_pack(self.plan.handle, g[0].data_ptr(), g[1].data_ptr(),
                                            g[2].data_ptr(), self.packed.data_ptr(),
                                            current_stream_handle(self.device_index)))
            del g  # packing is stream-ordered before any later call on this stream
        self._forward, self._forward_variant = _fast_forward()
        self._plan_handle = self.plan.handle
        self._packed_ptr = self.packed.data_ptr()
        torch_call = _torch_call()
        self._bound = torch_call.bind(self._plan_handle, self._packed_ptr, self.in_features,
                                      self.out_features, _DTYPES[dtype], self.device_index)
        self._call = torch_call.forward

    # ---- queries -------------------------------------------------------------------------
    @property
    def packed_bytes(self) -> int:
        return self.plan.packed_bytes

    def variants(self, tokens: int = 1) -> list[dict]:
        return self.plan.variants(tokens)

    def selected(self, tokens: int) -> dict:
        return self.plan.describe(-1, tokens)

    # ---- calls ---------------------------------------------------------------------------
    def _check(self, x: torch.Tensor) -> torch.Tensor:
        """x as the kernels read it: same dtype/device, [T, in], contiguous, 16-byte aligned."""
        if x.dtype is not self.dtype or x.get_device() != self.device_index:
            raise ValueError(f"x must be {self.dtype} on {self.device}, got {x.dtype} on {x.device}")
        if x.ndim != 2 or x.shape[1] != self.in_features:
            raise ValueError(
                f"Expected x with shape [tokens, {self.in_features}], got {tuple(x.shape)}")
        if x.shape[0] > 2**31 - 1:
            raise ValueError(f"At most 2**31 - 1 tokens per call, got {x.shape[0]}")
        if not x.is_contiguous() or x.data_ptr() & 15:
            x = x.clone(memory_format=torch.contiguous_format)
        return x

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        y = self._call(self._bound, x)
        return y if y is not None else self._checked_call(x)

    def _checked_call(self, x: torch.Tensor) -> torch.Tensor:
        x = self._check(x)
        tokens = x.shape[0]
        y = x.new_empty((tokens, self.out_features))
        if tokens:
            status = self._forward(self._plan_handle, self._packed_ptr, x.data_ptr(),
                                   y.data_ptr(), tokens, _raw_stream(self.device_index))
            if status:
                _lib.check(status)
        return y

    def run_variant(self, x: torch.Tensor, variant: int) -> torch.Tensor:
        """Forward through one explicit variant (tests and sweeps)."""
        x = self._check(x)
        tokens = x.shape[0]
        y = x.new_empty((tokens, self.out_features))
        if tokens:
            _lib.check(self._forward_variant(self._plan_handle, int(variant), self._packed_ptr,
                                             x.data_ptr(), y.data_ptr(), tokens,
                                             _raw_stream(self.device_index)))
        return y

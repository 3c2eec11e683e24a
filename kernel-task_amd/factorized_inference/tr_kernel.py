"""Host side of the HIP tensor-ring operator: prepare once, call per input.

Mirrors src/factorized_inference/tr_kernel.py of the reference (PreparedTRKernel, packing at
prepare time, a tiling/variant choice per token count) with its own mechanics:

  prepare  trk_plan_create picks the contraction order(s) and kernel variants for the shape;
           a shape without compiled MFMA tables gets a variant module built for it
           (jit.py: the generator's table compiled once, cached), at the next power-of-two
           kernel rank when the cores' rank has none (zero-padded ring links, exact);
           trk_pack packs the cores into one device buffer (no dense W, padding only)
  call     one C++ call per input (the call slot of _trktorch.Op, PreparedTRKernel's base):
           check x, allocate the output with torch's caching allocator, trk_forward on the
           caller's current stream. No workspace, counters or other state survives a call,
           so one prepared object may be used from several streams. Inputs that need
           checking or copying go through the Python path below (_checked_call), which
           raises or copies first.

  epilogues accumulate(x) stores y in fp32; forward_add(x, h) and forward_silu_mul(x, g)
           fuse a residual add or a SwiGLU gate into the kernel's output store
           (trk_forward_epilogue). consume_silu_mul / consume_add are the standalone
           elementwise forms of the reference's fp32-output consumers.

Environment switches (read at prepare time): TRK_VARIANT=<index> routes every token count to
that variant of the plan (indices from `PreparedTRKernel.variants()`, for sweeps);
TRK_XCD_LOCAL=1 calls `use_xcd_local()`.
"""
from __future__ import annotations

import os
import warnings
from typing import Sequence

import torch

from . import _lib, jit, tilegen
from .reference import TRSpec, _validate_cores

_DTYPES = {torch.float16: _lib.DTYPE_F16, torch.bfloat16: _lib.DTYPE_BF16,
           torch.float32: _lib.DTYPE_F32}
_TILEGEN_DTYPES = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}

_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)
if _raw_stream is None:
    _raw_stream = lambda device_index: torch.cuda.current_stream(device_index).cuda_stream  # noqa: E731


def _fast_forward():
    """The CPython fast-call bindings of trk_forward, trk_forward_variant and
    trk_forward_epilogue (built next to libtrk.so), else their ctypes bindings."""
    _lib.load()  # binds and version-checks libtrk.so first
    try:
        from . import _trkcall
    except ImportError:
        lib = _lib.load()
        return lib.trk_forward, lib.trk_forward_variant, lib.trk_forward_epilogue
    return _trkcall.forward, _trkcall.forward_variant, _trkcall.forward_epilogue


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


def make_plan(spec: TRSpec, dtype: torch.dtype) -> _lib.Plan:
    """The plan of one operator: the library's own variant tables; for shapes without MFMA
    variants, a plan at the MFMA kernel rank (trk_plan_create_padded when the cores' rank is
    not a power of two >= 8) with a variant module built for the shape (jit.build_module).
    Shapes the generator has no tile for and TRK_JIT=0 keep the generic HIP kernel."""
    code = _DTYPES[dtype]
    plan = _lib.Plan(spec.input_modes, spec.output_modes, spec.rank, code)
    if plan.has_mfma or not jit.enabled():
        return plan
    krank = jit.kernel_rank(spec.rank)
    if krank is None:
        return plan
    padded = plan if krank == spec.rank else _lib.Plan(
        spec.input_modes, spec.output_modes, spec.rank, code, kernel_rank=krank)
    if not padded.has_mfma:
        shape = tilegen.ShapeDecl("prepared", tuple(spec.input_modes), tuple(spec.output_modes),
                                  krank, _TILEGEN_DTYPES[dtype])
        try:
            path = jit.build_module(shape)
            if path is None:
                return plan
            padded.load_module(path)
        except (OSError, RuntimeError) as exc:
            warnings.warn(f"no MFMA variant module for {shape.key} ({exc}); the generic "
                          "kernel serves this shape", RuntimeWarning)
            return plan
    return padded if padded.has_mfma else plan


try:  # the base whose C++ call slot runs a prepared operator's calls (built with libtrk.so)
    from . import _trktorch as _native_call
    _CallBase = _native_call.Op
except ImportError:  # not built: PreparedTRKernel() raises in _torch_call()
    _CallBase = object


def current_stream_handle(device_index: int) -> int:
    """hipStream_t of torch's current stream on `device_index`, as an integer."""
    return _raw_stream(device_index)


class PreparedTRKernel(_CallBase):
    """Callable returned by prepare_optimized for cores on a ROCm device.

    fp16, bf16 and fp32 cores are supported; x must have the cores' dtype and device.
    `run(x)` returns a new [T, out_features] tensor written on the caller's current stream
    (reference: PreparedTRKernel.__call__, tr_kernel.py:264-319). The call is the C++ slot of
    the base class _trktorch.Op; x it does not take goes to _checked_call, which raises or
    copies it first.
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
        self.plan = make_plan(spec, dtype)
        forced = os.environ.get("TRK_VARIANT")
        if forced is not None:
            self.plan.set_variant(1, 1 << 30, int(forced))
        elif os.environ.get("TRK_XCD_LOCAL") == "1":
            self.use_xcd_local()
        with torch.cuda.device(self.device_index):
            self.packed = torch.empty(self.plan.packed_bytes, dtype=torch.uint8, device=device)
            g = [c.contiguous() for c in cores]
            _lib.check(_lib.load().trk_pack(self.plan.handle, g[0].data_ptr(), g[1].data_ptr(),
                                            g[2].data_ptr(), self.packed.data_ptr(),
                                            current_stream_handle(self.device_index)))
            # the packed cores are complete before prepare returns, so a first call on any
            # stream (not only the one that packed) reads them whole
            torch.cuda.current_stream(self.device_index).synchronize()
            del g
        self._forward, self._forward_variant, self._forward_epilogue = _fast_forward()
        self._plan_handle = self.plan.handle
        self._packed_ptr = self.packed.data_ptr()
        torch_call = _torch_call()
        bind = (self._plan_handle, self._packed_ptr, self.in_features, self.out_features,
                _DTYPES[dtype], self.device_index)
        self._bound = torch_call.bind(*bind)   # the epilogue methods' path (forward())
        self._call = torch_call.forward
        self._bind_native(*bind)               # what a call of the object runs

    # ---- queries -------------------------------------------------------------------------
    @property
    def packed_bytes(self) -> int:
        return self.plan.packed_bytes

    def variants(self, tokens: int = 1) -> list[dict]:
        return self.plan.variants(tokens)

    def selected(self, tokens: int) -> dict:
        return self.plan.describe(-1, tokens)

    def use_xcd_local(self, max_tokens: int = 1) -> bool:
        """Route token counts 1..max_tokens to the plan's XCD-local variant, if it has one
        (a name with `_xl`: the launch's work runs on one XCD, so one L2 fetches each core
        slice once and writes every line of y once, and the other seven XCDs stay free for
        concurrent work). It trades latency for HBM traffic: on MI355X the tokens=1 launch of
        1920->2880 at rank 8 moves about 175 KB instead of the default's 280 KB (itself on 4
        XCDs) and takes about 5 % longer.
        Returns False, changing nothing, when the plan has no such variant."""
        for index, v in enumerate(self.variants()):
            if "_xl<" in v["name"]:
                self.plan.set_variant(1, max_tokens, index)
                return True
        return False

    # ---- calls (run(x) is the call slot of the base class) ---------------------------------
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

    def accumulate(self, x: torch.Tensor) -> torch.Tensor:
        """y = TR(cores) x in fp32, [T, out_features]: the kernel's accumulator stored without
        rounding to 16 bits (reference: PreparedTRKernel.accumulate, tr_kernel.py:230-243,
        which returns a view of its persistent workspace that the consumer must clear; this
        returns an ordinary new tensor)."""
        y = self._call(self._bound, x, _lib.EPI_F32, None)
        return y if y is not None else self._checked_call(x, _lib.EPI_F32)

    def forward_add(self, x: torch.Tensor, residual: torch.Tensor) -> torch.Tensor:
        """residual + TR(cores) x in the cores' dtype, the add fused into the kernel's output
        store and rounded once. residual: [T, out_features], the cores' dtype or fp32
        (the reference's consume_add(h, accumulate(x)), csrc/v3g/bind.cu:112-122, as one
        launch)."""
        y = self._call(self._bound, x, _lib.EPI_ADD, residual)
        return y if y is not None else self._checked_call(x, _lib.EPI_ADD, residual)

    def forward_silu_mul(self, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        """silu(gate) * TR(cores) x in the cores' dtype, fused into the kernel's output
        store: the up projection of a SwiGLU MLP consuming the gate projection's output
        (fp32 from accumulate(), or the cores' dtype). The reference's
        consume_silu_mul(g, u), csrc/v3g/bind.cu:96-110, folded into the u launch."""
        y = self._call(self._bound, x, _lib.EPI_SILU_MUL, gate)
        return y if y is not None else self._checked_call(x, _lib.EPI_SILU_MUL, gate)

    def _check_aux(self, aux: torch.Tensor, tokens: int) -> tuple[torch.Tensor, int]:
        if not isinstance(aux, torch.Tensor):
            raise ValueError("the epilogue input must be a tensor")
        if aux.dtype is not self.dtype and aux.dtype is not torch.float32:
            raise ValueError(f"the epilogue input must be {self.dtype} or float32, got {aux.dtype}")
        if aux.get_device() != self.device_index:
            raise ValueError(f"the epilogue input must be on {self.device}, got {aux.device}")
        if tuple(aux.shape) != (tokens, self.out_features):
            raise ValueError(f"Expected the epilogue input with shape [{tokens}, "
                             f"{self.out_features}], got {tuple(aux.shape)}")
        return aux.contiguous(), _DTYPES[aux.dtype]

    def _checked_call(self, x: torch.Tensor, epilogue: int = _lib.EPI_STORE,
                      aux: torch.Tensor | None = None) -> torch.Tensor:
        x = self._check(x)
        tokens = x.shape[0]
        aux_ptr, aux_dtype = 0, _DTYPES[self.dtype]
        if epilogue in (_lib.EPI_ADD, _lib.EPI_SILU_MUL):
            aux, aux_dtype = self._check_aux(aux, tokens)
            aux_ptr = aux.data_ptr()
        y_dtype = torch.float32 if epilogue == _lib.EPI_F32 else self.dtype
        y = x.new_empty((tokens, self.out_features), dtype=y_dtype)
        if tokens:
            stream = _raw_stream(self.device_index)
            if epilogue == _lib.EPI_STORE:
                status = self._forward(self._plan_handle, self._packed_ptr, x.data_ptr(),
                                       y.data_ptr(), tokens, stream)
            else:
                status = self._forward_epilogue(self._plan_handle, -1, self._packed_ptr,
                                                x.data_ptr(), y.data_ptr(), tokens, epilogue,
                                                aux_ptr, aux_dtype, stream)
            if status:
                _lib.check(status)
        return y

    def run_variant(self, x: torch.Tensor, variant: int, epilogue: int = _lib.EPI_STORE,
                    aux: torch.Tensor | None = None) -> torch.Tensor:
        """Forward through one explicit variant, optionally with an epilogue (tests, sweeps)."""
        x = self._check(x)
        tokens = x.shape[0]
        aux_ptr, aux_dtype = 0, _DTYPES[self.dtype]
        if epilogue in (_lib.EPI_ADD, _lib.EPI_SILU_MUL):
            aux, aux_dtype = self._check_aux(aux, tokens)
            aux_ptr = aux.data_ptr()
        y_dtype = torch.float32 if epilogue == _lib.EPI_F32 else self.dtype
        y = x.new_empty((tokens, self.out_features), dtype=y_dtype)
        if tokens:
            _lib.check(self._forward_epilogue(self._plan_handle, int(variant), self._packed_ptr,
                                              x.data_ptr(), y.data_ptr(), tokens, int(epilogue),
                                              aux_ptr, aux_dtype, _raw_stream(self.device_index)))
        return y


def _check_consumer_operand(name: str, t: torch.Tensor, dtype: torch.dtype | None,
                            like: torch.Tensor) -> torch.Tensor:
    if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
        raise ValueError(f"{name} must be a tensor on a ROCm (cuda) device")
    if dtype is not None and t.dtype is not dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if t.shape != like.shape or t.device != like.device:
        raise ValueError(f"{name} must match {tuple(like.shape)} on {like.device}, got "
                         f"{tuple(t.shape)} on {t.device}")
    return t.contiguous()


def forward_swiglu(gate: PreparedTRKernel, up: PreparedTRKernel, x: torch.Tensor) -> torch.Tensor:
    """silu(gate(x)) * up(x), the gate and up projections of a SwiGLU block, in the cores'
    dtype from one launch (trk_forward_swiglu): each workgroup computes its tile of gate(x),
    keeps it in fp32 registers, computes the same tile of up(x) and stores the product,
    rounded once. Where the plan's selected variant has no fused kernel (shapes other than
    the declared gate/up ones), the same result comes from two launches:
    up.forward_silu_mul(x, gate.accumulate(x)). Reference: the accumulate / accumulate /
    consume_silu_mul chain of csrc/v3g/bind.cu:84-136, which takes three launches."""
    if not isinstance(gate, PreparedTRKernel) or not isinstance(up, PreparedTRKernel):
        raise ValueError("gate and up must be prepared operators (prepare_optimized)")
    if (gate.spec != up.spec or gate.dtype is not up.dtype or gate.device != up.device):
        raise ValueError("gate and up must have one shape, dtype and device")
    x = gate._check(x)
    y = torch.empty(x.shape[0], gate.out_features, dtype=gate.dtype, device=gate.device)
    lib = _lib.load()
    status = lib.trk_forward_swiglu(gate.plan.handle, gate.packed.data_ptr(), up.plan.handle,
                                    up.packed.data_ptr(), x.data_ptr(), y.data_ptr(), x.shape[0],
                                    current_stream_handle(gate.device_index))
    if status == _lib.ERR_UNSUPPORTED:
        return up.forward_silu_mul(x, gate.accumulate(x))
    _lib.check(status)
    return y


def consume_silu_mul(g: torch.Tensor, u: torch.Tensor,
                     out_dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """silu(g) * u for fp32 g and u of one shape, rounded once to out_dtype (default bf16).

    Reference: consume_silu_mul (csrc/v3g/bind.cu:96-110, :126-136), which also zeroes g and
    u because they are its persistent workspace; here g and u are only read. For the
    operator's own outputs, PreparedTRKernel.forward_silu_mul fuses this into the kernel."""
    g = _check_consumer_operand("g", g, torch.float32, g)
    u = _check_consumer_operand("u", u, torch.float32, g)
    if out_dtype not in _DTYPES:
        raise ValueError(f"Unsupported output dtype {out_dtype}")
    out = torch.empty(g.shape, dtype=out_dtype, device=g.device)
    with torch.cuda.device(g.device):
        _lib.check(_lib.load().trk_consume_silu_mul(
            g.data_ptr(), u.data_ptr(), out.data_ptr(), _DTYPES[out_dtype], g.numel(),
            current_stream_handle(g.device.index)))
    return out


def consume_add(h: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """h + y for h in fp16/bf16/fp32 and fp32 y of one shape, rounded once to h's dtype.

    Reference: consume_add (csrc/v3g/bind.cu:112-122, :138-149), which also zeroes y (its
    persistent workspace); here y is only read. PreparedTRKernel.forward_add fuses this
    into the kernel for the operator's own outputs."""
    if not isinstance(h, torch.Tensor) or h.dtype not in _DTYPES:
        raise ValueError("h must be a float16, bfloat16 or float32 tensor")
    h = _check_consumer_operand("h", h, None, h)
    y = _check_consumer_operand("y", y, torch.float32, h)
    out = torch.empty_like(h)
    with torch.cuda.device(h.device):
        _lib.check(_lib.load().trk_consume_add(
            h.data_ptr(), y.data_ptr(), out.data_ptr(), _DTYPES[h.dtype], h.numel(),
            current_stream_handle(h.device.index)))
    return out


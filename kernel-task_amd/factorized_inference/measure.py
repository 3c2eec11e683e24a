"""Timing helpers shared by bench.py and the harness (benchmarks/benchmark.py).

Definitions follow the reference's harness (benchmarks/benchmark.py:138-174) and
tools/measure_kernels.py:36-103:
  stream latency   HIP events bracketing a block of back-to-back calls on the current
                   stream, divided by the block length (not a sum of kernel durations).
                   The events are created without the system-scope fence at record
                   (hipEventDisableSystemFence): a default event's record ends with a release
                   to system scope, the L2s written back for the host, which the block's end
                   marker would add to the block (measured at the headline, 20 calls: 3.16 ->
                   3.08 us per call). Every call keeps its own end-of-kernel release
  host latency     wall clock around one call including the trailing synchronize
  kernel time      not measured in process. The reference reads profiler kernel events
                   (tools/measure_kernels.py:69-82); on ROCm torch.profiler adds ~2.5-3.5 us
                   and HIP events bound to the dispatch (hipExtLaunchKernel) ~1 us to kernels
                   of a few microseconds, so both read above the stream period there. Kernel
                   durations come from rocprofv3 kernel traces instead
  floors           an empty C call, and one empty kernel launch without and with the forward
                   kernels' arguments (host and stream time)
  work             algorithmic flops of the chain order the kernel runs, the reference's
                   flop count (its fixed order, tools/measure_kernels.py:36-44), and
                   compulsory bytes = element size x (factor parameters + T*in + T*out)
"""
from __future__ import annotations

import ctypes
import os
import statistics
import time
from typing import Callable

import torch

# MI355X (gfx950) peaks: HBM3E 8 TB/s; dense MFMA fp16/bf16 2.5 PFLOP/s, fp32 157.3 TFLOP/s.
PEAK_HBM_GBS = 8000.0
PEAK_TFLOPS = {torch.float16: 2500.0, torch.bfloat16: 2500.0, torch.float32: 157.3}


def synchronize() -> None:
    torch.cuda.synchronize()


HIP_EVENT_DISABLE_SYSTEM_FENCE = 0x20000000  # hip_runtime_api.h
_events = None


def _hip_runtime() -> ctypes.CDLL:
    """The HIP runtime torch has loaded (the copy whose streams torch hands out; a second copy
    of the runtime would not know them), found among the process's mappings."""
    torch.cuda.init()
    with open("/proc/self/maps") as maps:
        paths = {line.split(None, 5)[5].strip() for line in maps
                 if "libamdhip64.so" in line}
    if len(paths) != 1:
        raise RuntimeError(f"expected one HIP runtime in the process, found {sorted(paths)}")
    hip = ctypes.CDLL(paths.pop(), mode=os.RTLD_NOLOAD)
    vp = ctypes.c_void_p
    hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(vp), ctypes.c_uint]
    hip.hipEventRecord.argtypes = [vp, vp]
    hip.hipEventSynchronize.argtypes = [vp]
    hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
    hip.hipGetErrorString.restype = ctypes.c_char_p
    return hip


class _Events:
    """A start and an end HIP event without the system-scope fence, reused by every block."""

    def __init__(self):
        self.hip = _hip_runtime()
        self.start, self.end = ctypes.c_void_p(), ctypes.c_void_p()
        for e in (self.start, self.end):
            self.check(self.hip.hipEventCreateWithFlags(ctypes.byref(e),
                                                        HIP_EVENT_DISABLE_SYSTEM_FENCE))

    def check(self, status: int) -> None:
        if status != 0:
            raise RuntimeError(f"HIP error {status}: {self.hip.hipGetErrorString(status).decode()}")

    def record(self, event: ctypes.c_void_p) -> None:
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        self.check(self.hip.hipEventRecord(event, stream))

    def elapsed_ms(self) -> float:
        self.check(self.hip.hipEventSynchronize(self.end))
        ms = ctypes.c_float()
        self.check(self.hip.hipEventElapsedTime(ctypes.byref(ms), self.start, self.end))
        return ms.value


def stream_us(fn: Callable[[], object], calls: int, blocks: int = 1) -> list[float]:
    """Per-call stream latency (us) of `blocks` event-bracketed blocks of `calls` calls."""
    global _events
    if _events is None:
        _events = _Events()
    ev = _events
    out = []
    for _ in range(blocks):
        synchronize()
        ev.record(ev.start)
        for _ in range(calls):
            fn()
        ev.record(ev.end)
        out.append(ev.elapsed_ms() * 1000.0 / calls)
    return out


def host_us(fn: Callable[[], object], samples: int,
            sync: Callable[[], None] = synchronize) -> list[float]:
    """Host-synchronized latency (us) of single calls (`sync` waits for the device; a no-op
    for work on the CPU)."""
    out = []
    for _ in range(samples):
        sync()
        t0 = time.perf_counter_ns()
        fn()
        sync()
        out.append((time.perf_counter_ns() - t0) / 1000.0)
    return out


def host_submit_us(fn: Callable[[], object], calls: int) -> float:
    """Host time per call without synchronizing (what the host needs to submit one call)."""
    synchronize()
    t0 = time.perf_counter_ns()
    for _ in range(calls):
        fn()
    t1 = time.perf_counter_ns()
    synchronize()
    return (t1 - t0) / 1000.0 / calls


def reference_flops(spec, tokens: int) -> float:
    """Flops of the reference's fixed contraction order (G1, G2, G3) for `tokens` tokens
    (tools/measure_kernels.py:36-44): the count its "% FP16 TC peak" column uses."""
    ni, nj, nk = spec.input_modes
    P, Q, Rr = spec.output_modes
    R = spec.rank
    per_token = ni * nj * nk * P * R * R + nj * nk * P * Q * R ** 3 + nk * P * Q * Rr * R * R
    return 2.0 * tokens * per_token


def floors(lib, calls: int = 2000) -> dict:
    """Host cost of an empty C call and of an empty launch; stream time of empty launches
    (the reference's floors, tools/measure_kernels.py:97-103, without its profiler kernel
    time of the empty kernel)."""
    from .tr_kernel import current_stream_handle

    dev = torch.cuda.current_device()
    stream = current_stream_handle(dev)
    t0 = time.perf_counter_ns()
    for _ in range(calls):
        lib.trk_empty_call()
    empty_call = (time.perf_counter_ns() - t0) / 1000.0 / calls
    launch = lambda: lib.trk_empty_launch(current_stream_handle(dev))  # noqa: E731
    # an empty kernel with the forward kernels' argument list: fetching a launch's kernel
    # arguments is part of every forward call's stream time
    launch_args = lambda: lib.trk_empty_launch_args(current_stream_handle(dev))  # noqa: E731
    for _ in range(50):
        launch()
        launch_args()
    out = {
        "host_empty_c_call_us": empty_call,
        "host_empty_launch_us": host_submit_us(launch, calls),
        "stream_empty_launch_us": statistics.median(stream_us(launch, 200, blocks=5)),
        "host_empty_launch_args_us": host_submit_us(launch_args, calls),
        "stream_empty_launch_args_us": statistics.median(stream_us(launch_args, 200, blocks=5)),
        "stream_handle": bool(stream is not None),
    }
    return out


def roofline(flops: float, nbytes: float, us: float, dtype: torch.dtype) -> dict:
    seconds = us * 1e-6
    gbs = nbytes / seconds / 1e9
    tflops = flops / seconds / 1e12
    return {
        "achieved_GBps": gbs, "frac_hbm": gbs / PEAK_HBM_GBS,
        "achieved_TFLOPs": tflops, "frac_mfma": tflops / PEAK_TFLOPS[dtype],
    }

"""GPU checks of the stream timer (factorized_inference.measure.stream_us).

The timer records HIP events created without the system-scope fence on torch's current
stream, through the HIP runtime torch has loaded. On a block long enough that the markers'
own cost vanishes it must read what torch's default events read, on the default stream and
on a side stream.
"""
from __future__ import annotations

import statistics

import pytest
import torch

from factorized_inference import measure

pytestmark = pytest.mark.gpu


def torch_event_us(fn, calls):
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(calls):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) * 1000.0 / calls


def test_stream_timer_agrees_with_torch_events_on_long_blocks():
    print("case: stream timer vs torch events, 2048^2 fp16 matmul blocks", flush=True)
    measure._hip_runtime()  # exactly one HIP runtime in the process, or it raises
    a = torch.randn(2048, 2048, device="cuda", dtype=torch.float16)
    fn = lambda: a @ a  # noqa: E731
    for _ in range(50):
        fn()
    ours, theirs = [], []
    for _ in range(5):  # alternating blocks, so that clock drift hits both timers alike
        ours += measure.stream_us(fn, 20)
        theirs.append(torch_event_us(fn, 20))
    ratio = statistics.median(ours) / statistics.median(theirs)
    assert 0.95 < ratio < 1.05, (ours, theirs)


def test_stream_timer_follows_the_current_stream():
    print("case: stream timer on a side stream", flush=True)
    a = torch.randn(1024, 1024, device="cuda", dtype=torch.float16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())  # `a` is written on the default stream
    with torch.cuda.stream(side):
        fn = lambda: a @ a  # noqa: E731
        fn()
        t = measure.stream_us(fn, 10, blocks=2)
    torch.cuda.synchronize()
    assert len(t) == 2 and all(v > 0 for v in t)

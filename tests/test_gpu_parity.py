"""GPU parity of the HIP operator (through the C ABI) against the CPU oracle.

Ports the reference's GPU tests (tests/test_correctness.py:49-77) and its manual sweeps
(tools/check_kernel.py, check_v3.py, check_v3t.py, check_bf16.py): the required fp16
workloads, the bf16 Llama-shaped configs, changing token counts on one prepared object
(ragged, up and down), independent prepared weights, unmodified inputs, every compiled
variant, odd shapes, fp32, T = 0, repeated calls and side streams.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from factorized_inference import TRSpec, make_cores, prepare_optimized
from gpu_util import check_result, oracle_y

pytestmark = pytest.mark.gpu

DEFAULT = dict(input_modes=(8, 12, 20), output_modes=(12, 10, 24))
LLAMA_UP = dict(input_modes=(16, 16, 16), output_modes=(16, 28, 32))
LLAMA_DOWN = dict(input_modes=(16, 28, 32), output_modes=(16, 16, 16))


def gpu_x(spec, tokens, seed, dtype):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(tokens, spec.in_features, generator=g, device="cuda", dtype=dtype)


def announce(**case):
    print("case:", ", ".join(f"{k}={v}" for k, v in case.items()), flush=True)


# ---- the reference's acceptance workloads (tests/test_correctness.py:68-77) ----------------
@pytest.mark.parametrize("rank,tokens", [(8, 1), (8, 8), (8, 32), (16, 1), (16, 32), (16, 8)])
def test_required_workloads_fp16(rank, tokens):
    announce(test="required", rank=rank, tokens=tokens)
    spec = TRSpec(rank=rank)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=23)
    x = gpu_x(spec, tokens, 41 + tokens, torch.float16)
    y = prepare_optimized(cores, spec)(x)
    torch.cuda.synchronize()
    check_result(y, oracle_y(x, cores, spec), torch.float16)


# ---- Llama-3-8B-shaped configs, bf16, uniform sigma (BASELINE configs 4 and 5) --------------
@pytest.mark.parametrize("shape,rank,tokens", [
    (LLAMA_UP, 8, 1), (LLAMA_UP, 8, 8), (LLAMA_UP, 8, 32), (LLAMA_UP, 8, 128),
    (LLAMA_DOWN, 16, 1), (LLAMA_DOWN, 16, 32), (LLAMA_DOWN, 16, 256),
])
def test_llama_shapes_bf16(shape, rank, tokens):
    announce(test="llama", shape=shape, rank=rank, tokens=tokens)
    spec = TRSpec(rank=rank, **shape)
    cores = make_cores(spec, device="cuda", dtype=torch.bfloat16, seed=0, init="uniform")
    x = gpu_x(spec, tokens, tokens, torch.bfloat16)
    y = prepare_optimized(cores, spec)(x)
    torch.cuda.synchronize()
    # every row of the full-size launch, so every token tile (blockIdx.y) of the grid is
    # checked; the oracle runs in token chunks to bound its float64 intermediates
    check_result(y, oracle_y(x, cores, spec, chunk=32), torch.bfloat16)


# ---- BASELINE configs[0] through the HIP path: fp32, 1920 -> 2880, rank 8 -------------------
@pytest.mark.parametrize("init", ["per_core", "uniform"])
@pytest.mark.parametrize("tokens", [1, 8, 32])
def test_config0_fp32(tokens, init):
    """The reference's CPU-runnable case in float32 on the GPU (the generic kernel), with
    the harness's seeds (cores seed 0, x seed 0 + T: benchmarks/benchmark.py:107-108) and
    the float32 acceptance rule |y - y_ref| <= 1e-4 + 1e-4 |y_ref|
    (tests/test_correctness.py:17-23)."""
    announce(test="config0 fp32", tokens=tokens, init=init)
    spec = TRSpec(rank=8)
    cores = make_cores(spec, device="cuda", dtype=torch.float32, seed=0, init=init)
    x = gpu_x(spec, tokens, 0 + tokens, torch.float32)
    run = prepare_optimized(cores, spec)
    y = run(x)
    torch.cuda.synchronize()
    check_result(y, oracle_y(x, cores, spec), torch.float32)
    for variant, info in enumerate(run.variants(tokens)):  # both generic splits
        check_result(run.run_variant(x, variant), oracle_y(x, cores, spec), torch.float32)


# ---- one prepared object, changing values and token counts ---------------------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rank", [8, 16])
def test_changing_token_counts_on_one_object(rank, dtype):
    announce(test="changing", rank=rank, dtype=dtype)
    spec = TRSpec(rank=rank)
    cores = make_cores(spec, device="cuda", dtype=dtype, seed=3)
    original = tuple(c.clone() for c in cores)
    run = prepare_optimized(cores, spec)
    g = torch.Generator(device="cuda").manual_seed(5)
    for tokens in (2, 3, 8, 5, 12, 9, 32, 17, 33, 8, 1, 64, 4):
        x = torch.randn(tokens, spec.in_features, generator=g, device="cuda", dtype=dtype)
        x0 = x.clone()
        y = run(x)
        torch.cuda.synchronize()
        check_result(y, oracle_y(x0, original, spec), dtype)
        assert torch.equal(x, x0)
    for c, c0 in zip(cores, original):
        assert torch.equal(c, c0)


def test_zero_and_scaled_inputs():
    spec = TRSpec(rank=8)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=9)
    run = prepare_optimized(cores, spec)
    assert torch.count_nonzero(run(torch.zeros(5, spec.in_features, device="cuda",
                                               dtype=torch.float16))) == 0
    x = gpu_x(spec, 3, 10, torch.float16)
    for scale in (0.1, 2.0):
        xs = (x * scale).to(torch.float16)
        check_result(run(xs), oracle_y(xs, cores, spec), torch.float16)


def test_token_counts_beyond_one_launch():
    """More tokens than one launch's grid holds (65535 token tiles) split into consecutive
    launches; rows on both sides of each split are checked, with and without an epilogue."""
    from factorized_inference import _lib

    spec = TRSpec(rank=8)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=12)
    run = prepare_optimized(cores, spec)
    tokens = 70_000
    # a one-token tile: 65535 tokens per launch, so 70,000 tokens take two launches
    variant = next(i for i, v in enumerate(run.variants()) if v["kind"] == "mfma" and v["tile"][0] == 1)
    x = gpu_x(spec, tokens, 3, torch.float16)
    announce(test="beyond one launch", tokens=tokens, variant=run.variants()[variant]["name"])
    y = run.run_variant(x, variant)
    y32 = run.run_variant(x, variant, _lib.EPI_F32)
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 65534, 65535, 65536, tokens - 1], device="cuda")
    check_result(y[rows], oracle_y(x[rows], cores, spec), torch.float16)
    assert torch.equal(y, y32.half())


def test_empty_input():
    spec = TRSpec(rank=8)
    run = prepare_optimized(make_cores(spec, device="cuda", dtype=torch.float16), spec)
    y = run(torch.empty(0, spec.in_features, device="cuda", dtype=torch.float16))
    assert y.shape == (0, spec.out_features) and y.dtype == torch.float16


# ---- interface (tests/test_correctness.py:49-65) --------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_prepared_weights_are_independent(dtype):
    spec = TRSpec((2, 3, 2), (2, 4, 3), 3)
    a = make_cores(spec, device="cuda", dtype=dtype, seed=1)
    b = make_cores(spec, device="cuda", dtype=dtype, seed=2)
    run_a, run_b = prepare_optimized(a, spec), prepare_optimized(b, spec)
    x = gpu_x(spec, 3, 7, dtype)
    for run, weights in [(run_a, a), (run_b, b), (run_a, a)]:
        check_result(run(x), oracle_y(x, weights, spec), dtype)


def test_rejects_mismatched_inputs():
    spec = TRSpec(rank=8)
    run = prepare_optimized(make_cores(spec, device="cuda", dtype=torch.float16), spec)
    with pytest.raises(ValueError):
        run(torch.zeros(1, spec.in_features, device="cuda", dtype=torch.float32))
    with pytest.raises(ValueError):
        run(torch.zeros(1, spec.in_features, dtype=torch.float16))
    with pytest.raises(ValueError):
        run(torch.zeros(1, spec.in_features + 1, device="cuda", dtype=torch.float16))
    with pytest.raises(ValueError):
        prepare_optimized(make_cores(TRSpec(rank=4), device="cuda", dtype=torch.float16), spec)


def test_non_contiguous_input_and_side_stream():
    spec = TRSpec(rank=8)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=4)
    run = prepare_optimized(cores, spec)
    base = gpu_x(spec, 6, 12, torch.float16)
    x = base[::2]                      # non-contiguous rows
    expected = oracle_y(x, cores, spec)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        y = run(x)
    stream.synchronize()
    check_result(y, expected, torch.float16)


def test_first_call_on_a_stream_that_never_waited_for_the_packing():
    """prepare_optimized returns with the packed cores complete, so a first call on a stream
    that never waited for the packing stream reads them whole."""
    spec = TRSpec(rank=16)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=6)
    x = gpu_x(spec, 4, 14, torch.float16)
    expected = oracle_y(x, cores, spec)
    torch.cuda.synchronize()  # the cores and x are ready; nothing waits for the packing below
    run = prepare_optimized(cores, spec)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        y = run(x)
    stream.synchronize()
    check_result(y, expected, torch.float16)


def test_one_object_on_concurrent_streams_and_threads():
    """No state survives a call, so one prepared object serves several streams and host threads
    at once (the reference's design B must not: tr_kernel.py:185-187). Results are bitwise
    equal to the same calls made one at a time on the default stream."""
    import threading

    spec = TRSpec(rank=16)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=14)
    run = prepare_optimized(cores, spec)
    xs = [gpu_x(spec, T, 60 + T, torch.float16) for T in (1, 3, 8, 32, 1, 5)]
    expected = [run(x) for x in xs]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    outs = [None] * len(xs)
    for rep in range(3):                    # interleaved launches on two streams
        for i, x in enumerate(xs):
            with torch.cuda.stream(streams[i % 2]):
                outs[i] = run(x)
    torch.cuda.synchronize()
    for y, e in zip(outs, expected):
        assert torch.equal(y, e)
    results = {}

    def worker(k):                          # two host threads, each with its own stream
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.default_stream())
        with torch.cuda.stream(stream):
            ys = [run(x) for x in xs for _ in range(2)]
        stream.synchronize()
        results[k] = ys

    threads = [threading.Thread(target=worker, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    for k in range(2):
        ys = results[k]
        for j, y in enumerate(ys):
            assert torch.equal(y, expected[j // 2]), (k, j)
    check_result(expected[3], oracle_y(xs[3], cores, spec), torch.float16)


# ---- every variant the plan holds (tools/check_v3.py / check_v3t.py) ------------------------
@pytest.mark.parametrize("shape,rank,dtype", [
    (DEFAULT, 8, torch.float16), (DEFAULT, 16, torch.float16),
    (LLAMA_UP, 8, torch.bfloat16), (LLAMA_DOWN, 16, torch.bfloat16),
])
def test_every_variant(shape, rank, dtype):
    spec = TRSpec(rank=rank, **shape)
    cores = make_cores(spec, device="cuda", dtype=dtype, seed=17)
    run = prepare_optimized(cores, spec)
    for variant, info in enumerate(run.variants()):
        for tokens in (1, 7, 32):
            announce(test="variant", shape=shape, rank=rank, variant=info["name"], tokens=tokens)
            x = gpu_x(spec, tokens, 100 + tokens, dtype)
            y = run.run_variant(x, variant)
            y2 = run.run_variant(x, variant)
            torch.cuda.synchronize()
            assert torch.equal(y, y2), "repeated calls must be bitwise identical"
            check_result(y, oracle_y(x, cores, spec), dtype)


# ---- the XCD-local route (PreparedTRKernel.use_xcd_local) ------------------------------------
def test_xcd_local_route():
    announce(test="xcd_local", rank=8)
    spec = TRSpec(rank=8, **DEFAULT)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=5)
    run = prepare_optimized(cores, spec)
    default = run.selected(1)
    assert run.use_xcd_local()
    info = run.selected(1)
    assert "_xl<" in info["name"] and "_xl<" not in default["name"]
    # every workgroup of an XCD-local grid that is not dealt to XCD 0 exits: 8x the columns
    tile = info["tile"]
    assert info["grid"][0] == 8 * (24 // tile[1]) * (10 // tile[2]) * (12 // tile[3])
    assert "_xl<" not in run.selected(2)["name"]
    for tokens in (1, 2, 1):
        x = gpu_x(spec, tokens, 60 + tokens, torch.float16)
        y = run(x)
        torch.cuda.synchronize()
        check_result(y, oracle_y(x, cores, spec), torch.float16)
    # a plan without an XCD-local variant keeps its routing
    spec16 = TRSpec(rank=16, **DEFAULT)
    run16 = prepare_optimized(make_cores(spec16, device="cuda", dtype=torch.float16, seed=5), spec16)
    before = run16.selected(1)["name"]
    assert not run16.use_xcd_local() and run16.selected(1)["name"] == before


# ---- odd shapes and fp32 (tools/check_kernel.py:63-101, check_bf16.py) ---------------------
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("ins,outs,rank", [
    ((2, 3, 2), (2, 4, 3), 2), ((4, 4, 4), (4, 4, 4), 8), ((4, 4, 4), (4, 4, 4), 16),
    ((3, 2, 5), (4, 3, 6), 3), ((5, 7, 3), (3, 5, 7), 5), ((1, 1, 1), (1, 1, 1), 1),
    ((8, 12, 20), (12, 10, 24), 4),
    ((4, 4, 4), (4, 4, 4), 12),  # generic kernel on K orders grouped by 4 at a rank that is
                                 # not a power of two
])
def test_odd_shapes(ins, outs, rank, dtype):
    announce(test="odd", ins=ins, outs=outs, rank=rank, dtype=dtype)
    spec = TRSpec(ins, outs, rank)
    cores = make_cores(spec, device="cuda", dtype=dtype, seed=2)
    run = prepare_optimized(cores, spec)
    for tokens in (1, 3):
        x = gpu_x(spec, tokens, 50 + tokens, dtype)
        expected = oracle_y(x, cores, spec)
        check_result(run(x), expected, dtype)
        for variant, info in enumerate(run.variants(tokens)):  # e.g. both generic splits
            check_result(run.run_variant(x, variant), expected, dtype)


# ---- the committed golden vectors (tests/golden/oracle_vectors.npz) -------------------------
def test_golden_vectors_fp32():
    from pathlib import Path

    golden = np.load(Path(__file__).parent / "golden" / "oracle_vectors.npz")
    names = sorted({k.split("/")[0] for k in golden.files})
    for name in names:
        x = torch.from_numpy(golden[f"{name}/x"]).float().cuda()
        cores = [torch.from_numpy(golden[f"{name}/g{k}"]).float().cuda() for k in (1, 2, 3)]
        R = cores[0].shape[0]
        spec = TRSpec(tuple(c.shape[2] for c in cores), tuple(c.shape[1] for c in cores), R)
        announce(test="golden", name=name)
        y = prepare_optimized(cores, spec)(x)
        # the fixture was computed from the float64 values; the fp32 inputs differ from them by
        # one rounding, so compare with the fp32 tolerance scaled to the output magnitude
        expected = golden[f"{name}/y"]
        err = np.abs(y.double().cpu().numpy() - expected).max()
        assert err <= 1e-4 * max(1.0, np.abs(expected).max()), (name, err)


# ---- the per-call path and graph capture ----------------------------------------------------
def test_calls_take_the_native_path_and_fall_back_for_misaligned_x():
    spec = TRSpec(rank=8)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=6)
    run = prepare_optimized(cores, spec)
    x = gpu_x(spec, 3, 21, torch.float16)
    y_native = run._call(run._bound, x)          # the C++ path of __call__ (allocate + launch)
    assert y_native is not None and y_native.shape == (3, spec.out_features)
    check_result(y_native, oracle_y(x, cores, spec), torch.float16)
    flat = torch.empty(3 * spec.in_features + 1, device="cuda", dtype=torch.float16)
    shifted = flat[1:].view(3, spec.in_features)  # 2-byte offset: not 16-byte aligned
    shifted.copy_(x)
    assert run._call(run._bound, shifted) is None  # left to the checked path, which copies
    assert torch.equal(run(shifted), y_native)


def test_graph_capture_replays_match_eager_calls():
    spec = TRSpec(rank=8)
    cores = make_cores(spec, device="cuda", dtype=torch.float16, seed=8)
    run = prepare_optimized(cores, spec)
    static_x = gpu_x(spec, 4, 30, torch.float16)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(static_x)                             # warm up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_y = run(static_x)
    for replay in range(4):
        announce(test="graph", replay=replay)
        static_x.copy_(gpu_x(spec, 4, 31 + replay, torch.float16))
        graph.replay()
        eager = run(static_x.clone())             # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(static_y, eager), replay
        check_result(static_y, oracle_y(static_x, cores, spec), torch.float16)

"""Property tests of the host-side plan logic (no GPU): for random operator shapes, ranks and
dtypes, every plan the C ABI creates must describe itself consistently.

- the generic variant runs the chain order with the fewest flops, and every variant's flops
  are the oracle's count for the order it reports (tools/measure_kernels.py:36-44 form);
- compulsory bytes = element size x (factor parameters + T*in + T*out);
- LDS within 160 KB, grids of at least one workgroup, packed bytes between the factors and
  their padding;
- every token count selects a variant whose range holds it (or the generic fallback), and
  set_variant then routes a range to the chosen variant without touching counts outside it.
"""
from __future__ import annotations

import numpy as np
from hypothesis import given, settings
from hypothesis import strategies as st

from factorized_inference import _lib
from oracle import ring_oracle as orc

modes = st.tuples(st.integers(1, 24), st.integers(1, 24), st.integers(1, 24))
DTYPES = [_lib.DTYPE_F16, _lib.DTYPE_BF16, _lib.DTYPE_F32]


@settings(max_examples=80, deadline=None)
@given(ins=modes, outs=modes, rank=st.integers(1, 20), dtype=st.sampled_from(DTYPES),
       tokens=st.lists(st.integers(0, 5000), min_size=1, max_size=4))
def test_plans_describe_themselves_consistently(ins, outs, rank, dtype, tokens):
    plan = _lib.Plan(ins, outs, rank, dtype)
    elem = 4 if dtype == _lib.DTYPE_F32 else 2
    factors = sum(rank * o * i * rank for o, i in zip(outs, ins))
    in_f, out_f = int(np.prod(ins)), int(np.prod(outs))
    assert elem * factors <= plan.packed_bytes <= elem * factors * 16 + 6 * 3 * 256 * 4
    counts = {o: orc.flops_per_token(ins, outs, rank, o) for o in orc.CHAIN_ORDERS}
    generic = plan.describe(0, 1)
    assert generic["kind"] == "generic"
    assert abs(generic["flops"] - min(counts.values())) <= 1e-9 * generic["flops"]
    for T in tokens:
        index = plan.select(T)
        info = plan.describe(-1, T)
        assert info == plan.describe(index, T)
        assert info["flops"] == counts[tuple(info["order"])] * T
        assert info["bytes"] == elem * (factors + T * (in_f + out_f))
        assert 0 < info["lds_bytes"] <= 160 * 1024
        assert min(info["grid"]) >= 1
        if index > 0:
            assert info["t_min"] <= T <= info["t_max"]


@settings(max_examples=40, deadline=None)
@given(lo=st.integers(1, 300), width=st.integers(0, 300), data=st.data())
def test_set_variant_routes_exactly_its_range(lo, width, data):
    plan = _lib.Plan((8, 12, 20), (12, 10, 24), 8, _lib.DTYPE_F16)
    n = plan.variant_count
    variant = data.draw(st.integers(1, n - 1))
    before = {T: plan.select(T) for T in range(1, 700)}
    hi = lo + width
    plan.set_variant(lo, hi, variant)
    for T in range(1, 700):
        if lo <= T <= hi:
            assert plan.select(T) == variant
        elif before[T] == variant:
            # the variant's old range outside [lo, hi] is given up (it serves [lo, hi] now)
            assert plan.select(T) != variant
        else:
            assert plan.select(T) in (before[T], 0)

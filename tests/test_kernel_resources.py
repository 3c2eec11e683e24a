"""CPU checks of the compiler's per-kernel resource report (written by build_ext).

A ring3 MFMA kernel keeps its core slices, prefetched loads and accumulators in registers.
Scratch memory in one that reports no register spills means a register array fell into
memory (a helper left as a call took it by reference); that cost one tile 3.5x its time.
Spilled registers of deliberately over-budget tiles are allowed (the autotuner decides).
"""
from __future__ import annotations

import json

import pytest

from factorized_inference import build_ext


@pytest.fixture(scope="module")
def resources() -> dict:
    assert build_ext.RESOURCES.exists(), "build first: python -m factorized_inference.build_ext"
    return json.loads(build_ext.RESOURCES.read_text())


def test_report_covers_the_kernels(resources):
    names = list(resources)
    assert any("ring3_mfma_kernel" in n for n in names)
    assert any("ring3_generic" in n for n in names)
    for n, r in resources.items():
        assert {"VGPRs", "ScratchSize", "LDS Size"} <= set(r), n


def test_no_stack_objects_in_mfma_kernels(resources):
    bad = [n for n, r in resources.items() if "ring3_mfma_kernel" in n
           and int(r["ScratchSize"]) > 0 and int(r.get("VGPRs Spill", "0")) == 0]
    assert not bad, f"{len(bad)} MFMA kernels hold register arrays in scratch, e.g. {bad[:2]}"


def test_lds_within_160_kb(resources):
    for n, r in resources.items():
        assert int(r["LDS Size"]) <= 160 * 1024, n

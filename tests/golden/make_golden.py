"""Write the golden fixtures under tests/golden/ (run from the repository root).

    python tests/golden/make_golden.py

oracle_vectors.npz
    Inputs and float64 outputs of the oracle (oracle/ring_oracle.py, reference order) for
    small specs, plus the dense weight. Produced by the oracle after it passes the
    definition checks of tests/test_oracle.py; committed so that a later change to the
    oracle, or a GPU run without the oracle's sources, is checked against fixed numbers.
    The specs are the reference's own test specs (tests/test_correctness.py:26-31, :80-91;
    tests/test_benchmark.py:12-16) and one odd spec with every mode different.

reference_cores.npz
    make_cores values as written by the reference's own make_cores
    (src/factorized_inference/reference.py:53-77), CPU generator. make_cores is the one
    function on the path that no mathematical check pins (its values come from torch's RNG
    stream), so its output is recorded from the reference itself: this script loads
    reference.py from /root/reference by file path, calls make_cores, and stores the
    values. Only this container has /root/reference; the fixture is data.
"""
from __future__ import annotations

import importlib.util
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from oracle import ring_oracle  # noqa: E402

ORACLE_SPECS = [  # (name, input modes, output modes, rank, tokens, seed)
    ("s232_243_r2", (2, 3, 2), (2, 4, 3), 2, 3, 0),
    ("s444_444_r8", (4, 4, 4), (4, 4, 4), 8, 2, 19),
    ("s444_444_r16", (4, 4, 4), (4, 4, 4), 16, 2, 19),
    ("s222_222_r2", (2, 2, 2), (2, 2, 2), 2, 2, 11),
    ("s222_232_r2", (2, 2, 2), (2, 3, 2), 2, 1, 0),
    ("s325_436_r3", (3, 2, 5), (4, 3, 6), 3, 5, 7),
]

CORE_SPECS = [  # (name, input modes, output modes, rank, seed, dtype)
    ("s232_243_r2_seed0", (2, 3, 2), (2, 4, 3), 2, 0, "float32"),
    ("s444_444_r8_seed19", (4, 4, 4), (4, 4, 4), 8, 19, "float32"),
    ("s222_232_r2_seed0", (2, 2, 2), (2, 3, 2), 2, 0, "float32"),
    ("s232_243_r3_seed1_f16", (2, 3, 2), (2, 4, 3), 3, 1, "float16"),
    ("s232_243_r3_seed2_bf16", (2, 3, 2), (2, 4, 3), 3, 2, "bfloat16"),
]


def oracle_vectors() -> dict:
    out = {}
    for name, ins, outs, R, T, seed in ORACLE_SPECS:
        rng = np.random.default_rng(seed)
        cores = tuple(rng.standard_normal((R, o, i, R)) / np.sqrt(R * i) for o, i in zip(outs, ins))
        x = rng.standard_normal((T, int(np.prod(ins))))
        out[f"{name}/x"] = x
        for k, c in enumerate(cores):
            out[f"{name}/g{k + 1}"] = c
        out[f"{name}/y"] = ring_oracle.tr_forward(x, cores)
        out[f"{name}/w"] = ring_oracle.dense_weight(cores)
    return out


def reference_cores() -> dict:
    path = Path("/root/reference/src/factorized_inference/reference.py")
    spec = importlib.util.spec_from_file_location("reference_reference", path)
    module = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = module  # dataclasses look their module up here
    spec.loader.exec_module(module)
    import torch

    out = {}
    for name, ins, outs, R, seed, dtype in CORE_SPECS:
        cores = module.make_cores(module.TRSpec(ins, outs, R), dtype=getattr(torch, dtype), seed=seed)
        for k, c in enumerate(cores):
            # 16-bit values are stored widened to float32 (exact)
            out[f"{name}/g{k + 1}"] = c.float().numpy()
    return out


if __name__ == "__main__":
    np.savez_compressed(HERE / "oracle_vectors.npz", **oracle_vectors())
    print("wrote", HERE / "oracle_vectors.npz")
    if "--oracle-only" not in sys.argv:
        np.savez_compressed(HERE / "reference_cores.npz", **reference_cores())
        print("wrote", HERE / "reference_cores.npz")

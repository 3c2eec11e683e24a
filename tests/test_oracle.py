"""Pin the CPU oracle (oracle/) before trusting it as the parity checker.

Every oracle function is checked against something that does not restate its own formula:
  - the trace definition W = trace(G1[:,p,i,:] G2[:,q,j,:] G3[:,r,k,:]) by explicit sums
    (the reference's known-answer test, tests/test_correctness.py:80-91);
  - numpy.kron at rank 1 (the ring collapses to a Kronecker product);
  - invariants: linearity in x, trilinearity in the cores, one-hot columns, gauge
    invariance of each ring link, cyclic rotation of the cores;
  - the independent C restatement (oracle/ring_oracle.c);
  - the committed golden vectors (tests/golden/oracle_vectors.npz).
Planted mistakes (a wrong ring orientation, swapped modes, a dropped ring term) are made in a
copy of the oracle and must fail these checks.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import c_oracle
from oracle import ring_oracle as orc

GOLDEN = np.load(__import__("pathlib").Path(__file__).parent / "golden" / "oracle_vectors.npz")

SPECS = [
    ((2, 3, 2), (2, 4, 3), 2),
    ((2, 2, 2), (2, 2, 2), 2),
    ((3, 2, 5), (4, 3, 6), 3),
    ((4, 4, 4), (4, 4, 4), 8),
    ((2, 3, 4), (5, 2, 3), 4),
]


def make(spec, seed=0, tokens=3):
    ins, outs, R = spec
    rng = np.random.default_rng(seed)
    cores = tuple(rng.standard_normal((R, o, i, R)) for o, i in zip(outs, ins))
    x = rng.standard_normal((tokens, int(np.prod(ins))))
    return x, cores


def trace_weight(cores):
    R, ins, outs = orc._dims(cores)
    n_out, n_in = int(np.prod(outs)), int(np.prod(ins))
    return np.array([[orc.trace_entry(cores, o, i) for i in range(n_in)] for o in range(n_out)])


def close(a, b, tol=1e-11):
    scale = max(1.0, float(np.abs(b).max()))
    return float(np.abs(a - b).max()) <= tol * scale


# ---- the definition -------------------------------------------------------------------------
def test_known_answer_trace_definition():
    # the reference's KAT: spec (2,2,2)->(2,2,2) rank 2; the trace over 2x2 products
    _, cores = make(((2, 2, 2), (2, 2, 2), 2), seed=11)
    w = orc.dense_weight(cores)
    for o in range(8):
        p, q, r = o // 4, o // 2 % 2, o % 2
        for n in range(8):
            i, j, k = n // 4, n // 2 % 2, n % 2
            expected = np.trace(cores[0][:, p, i, :] @ cores[1][:, q, j, :] @ cores[2][:, r, k, :])
            assert abs(w[o, n] - expected) <= 1e-12
            assert abs(orc.trace_entry(cores, o, n) - expected) <= 1e-12


@pytest.mark.parametrize("spec", SPECS[:3] + [SPECS[4]])
def test_dense_weight_matches_trace_definition(spec):
    _, cores = make(spec, seed=3)
    assert close(orc.dense_weight(cores), trace_weight(cores))


@pytest.mark.parametrize("spec", SPECS)
def test_forward_forms_agree_with_dense_oracle(spec):
    x, cores = make(spec, seed=5)
    expected = orc.dense_forward(x, orc.dense_weight(cores))
    assert close(orc.tr_forward(x, cores), expected)
    assert close(orc.forward_pieces(x, cores), expected)
    for order in orc.CHAIN_ORDERS:
        assert close(orc.chain_forward(x, cores, order), expected), order


def test_rank_one_is_a_kronecker_product():
    _, cores = make(((2, 3, 4), (3, 2, 2), 1), seed=2)
    assert close(orc.dense_weight(cores), orc.kron_weight(cores))
    assert close(trace_weight(cores), orc.kron_weight(cores))


# ---- invariants -------------------------------------------------------------------------------
@pytest.mark.parametrize("spec", SPECS[:3])
def test_linearity_and_zero(spec):
    x, cores = make(spec, seed=8, tokens=4)
    x2 = np.random.default_rng(9).standard_normal(x.shape)
    y, y2 = orc.tr_forward(x, cores), orc.tr_forward(x2, cores)
    assert close(orc.tr_forward(2.5 * x - 0.75 * x2, cores), 2.5 * y - 0.75 * y2)
    assert np.all(orc.tr_forward(np.zeros_like(x), cores) == 0.0)


def test_trilinearity_in_the_cores():
    x, cores = make(SPECS[2], seed=4)
    y = orc.tr_forward(x, cores)
    for k, alpha in zip(range(3), (2.0, -0.5, 3.0)):
        scaled = tuple(c * alpha if m == k else c for m, c in enumerate(cores))
        assert close(orc.tr_forward(x, scaled), alpha * y)


def test_one_hot_inputs_give_columns_of_w():
    _, cores = make(SPECS[2], seed=6)
    w = orc.dense_weight(cores)
    eye = np.eye(w.shape[1])
    assert close(orc.tr_forward(eye, cores), w.T)


def test_gauge_invariance_of_each_ring_link():
    x, cores = make(SPECS[2], seed=12)
    g1, g2, g3 = cores
    R = g1.shape[0]
    rng = np.random.default_rng(13)
    m = rng.standard_normal((R, R)) + R * np.eye(R)
    mi = np.linalg.inv(m)
    # link b (G1 -> G2), link c (G2 -> G3), link a (G3 -> G1)
    gauged = [
        (np.einsum("apib,bd->apid", g1, m), np.einsum("db,bqjc->dqjc", mi, g2), g3),
        (g1, np.einsum("bqjc,cd->bqjd", g2, m), np.einsum("dc,crka->drka", mi, g3)),
        (np.einsum("da,apib->dpib", mi, g1), g2, np.einsum("crka,ad->crkd", g3, m)),
    ]
    y = orc.tr_forward(x, cores)
    for g in gauged:
        assert close(orc.tr_forward(x, g), y, tol=1e-9)


def test_cyclic_rotation_permutes_w():
    _, cores = make(((2, 3, 4), (3, 2, 5), 3), seed=14)
    w = orc.dense_weight(cores).reshape(3, 2, 5, 2, 3, 4)          # p q r i j k
    rotated = orc.dense_weight((cores[1], cores[2], cores[0])).reshape(2, 5, 3, 3, 4, 2)  # q r p j k i
    assert close(rotated, w.transpose(1, 2, 0, 4, 5, 3))


# ---- independent restatement and fixtures ----------------------------------------------------
@pytest.mark.parametrize("spec", SPECS)
def test_c_restatement_agrees(spec):
    x, cores = make(spec, seed=21)
    assert close(c_oracle.tr_forward(x, cores), orc.tr_forward(x, cores))
    if int(np.prod(spec[0])) * int(np.prod(spec[1])) <= 4096:
        assert close(c_oracle.dense_weight(cores), orc.dense_weight(cores))


def golden_names():
    return sorted({k.split("/")[0] for k in GOLDEN.files})


@pytest.mark.parametrize("name", golden_names())
def test_golden_vectors(name):
    x = GOLDEN[f"{name}/x"]
    cores = tuple(GOLDEN[f"{name}/g{k}"] for k in (1, 2, 3))
    assert close(orc.tr_forward(x, cores), GOLDEN[f"{name}/y"], tol=1e-13)
    assert close(orc.dense_weight(cores), GOLDEN[f"{name}/w"], tol=1e-13)
    assert close(c_oracle.tr_forward(x, cores), GOLDEN[f"{name}/y"], tol=1e-12)
    assert close(orc.dense_forward(x, GOLDEN[f"{name}/w"]), GOLDEN[f"{name}/y"], tol=1e-12)


# ---- planted mistakes must be caught ---------------------------------------------------------
def _wrong_ring_orientation(x, cores):
    g1, g2, g3 = cores
    return orc.tr_forward(x, (g1, g2.transpose(3, 1, 2, 0), g3))


def _swapped_input_modes(x, cores):
    T = x.shape[0]
    g1, g2, g3 = cores
    ni, nj, nk = g1.shape[2], g2.shape[2], g3.shape[2]
    xs = x.reshape(T, ni, nj, nk).transpose(0, 1, 3, 2).reshape(T, -1)  # j and k exchanged
    return orc.chain_forward(xs, (g1, g2, g3), (0, 1, 2)) if nj == nk else orc.tr_forward(xs, cores)


def _dropped_ring_term(x, cores):
    g1, g2, g3 = cores
    g3b = g3.copy()
    g3b[:, :, :, -1] = 0.0  # loses the a = R-1 term of the trace
    return orc.tr_forward(x, (g1, g2, g3b))


@pytest.mark.parametrize("mistake", [_wrong_ring_orientation, _swapped_input_modes, _dropped_ring_term])
def test_planted_mistakes_fail_the_checks(mistake):
    spec = ((2, 3, 3), (2, 3, 2), 3)
    x, cores = make(spec, seed=31, tokens=4)
    w = trace_weight(cores)
    assert not close(mistake(x, cores), orc.dense_forward(x, w))
    # the invariant checks catch them as well: one-hot inputs must return the columns of W
    eye = np.eye(w.shape[1])
    assert not close(mistake(eye, cores), w.T)


# ---- work counts --------------------------------------------------------------------------
def test_flop_count_matches_reference_formula_and_baseline():
    # reference order: 2*(ni nj nk P R^2 + nj nk P Q R^3 + nk P Q Rr R^2) per token
    (ni, nj, nk), (P, Q, Rr), R = (8, 12, 20), (12, 10, 24), 8
    ref = 2 * (ni * nj * nk * P * R**2 + nj * nk * P * Q * R**3 + nk * P * Q * Rr * R**2)
    assert orc.flops_per_token((8, 12, 20), (12, 10, 24), 8) == ref
    assert abs(ref - 39.8e6) < 0.05e6                      # 39.8 MFLOP per token at R8
    assert abs(orc.flops_per_token((8, 12, 20), (12, 10, 24), 16) - 277.2e6) < 0.1e6
    assert abs(orc.flops_per_token((16, 28, 32), (16, 16, 16), 16) - 2063.6e6) < 0.1e6
    # the chain order changes the count; (2,1,0) is the cheapest for the Llama down shape
    counts = {o: orc.flops_per_token((16, 28, 32), (16, 16, 16), 16, o) for o in orc.CHAIN_ORDERS}
    assert min(counts, key=counts.get) == (2, 1, 0)


def test_error_metrics():
    e = orc.errors(np.array([[1.0, 2.0]]), np.array([[1.0, 1.5]]))
    assert e["max_absolute_error"] == 0.5
    assert e["mean_absolute_error"] == 0.25
    assert abs(e["relative_l2_error"] - 0.5 / np.sqrt(1.0 + 2.25)) < 1e-15


# ---- epilogues: silu and the fused consumers -----------------------------------------------
def test_silu_matches_an_independent_logistic_and_its_identities():
    from scipy.special import expit

    a = np.concatenate([np.linspace(-30.0, 30.0, 2001), [-800.0, -1e-30, 0.0, 1e-30, 800.0]])
    s = orc.silu(a)
    assert np.all(np.isfinite(s))
    np.testing.assert_allclose(s, a * expit(a), rtol=1e-14, atol=1e-300)
    assert orc.silu(0.0) == 0.0
    np.testing.assert_allclose(s - orc.silu(-a), a, rtol=1e-13, atol=1e-13)  # silu(a)-silu(-a)=a
    assert orc.silu(800.0) == 800.0 and abs(orc.silu(-800.0)) < 1e-300
    assert abs(orc.silu(1.0) - 1.0 / (1.0 + np.exp(-1.0))) < 1e-16      # sigmoid(1) by hand


def test_epilogues_compose_with_the_operator():
    x, cores = make(SPECS[2], seed=5, tokens=4)
    y = orc.tr_forward(x, cores)
    rng = np.random.default_rng(6)
    aux = rng.standard_normal(y.shape)
    assert np.array_equal(orc.epilogue("store", y), y)
    assert np.array_equal(orc.epilogue("f32", y), y)
    assert np.array_equal(orc.epilogue("add", y, aux), aux + y)
    # a SwiGLU block: silu(gate) * up, elementwise, equals silu(gate) scaled per element
    from scipy.special import expit
    np.testing.assert_allclose(orc.epilogue("silu_mul", y, aux), aux * expit(aux) * y,
                               rtol=1e-13, atol=1e-13)
    # linearity of the operator carries through: silu_mul(g, y1 + y2) = silu_mul(g,y1)+(g,y2)
    x2 = rng.standard_normal(x.shape)
    y2 = orc.tr_forward(x2, cores)
    lhs = orc.epilogue("silu_mul", orc.tr_forward(x + x2, cores), aux)
    np.testing.assert_allclose(lhs, orc.epilogue("silu_mul", y, aux) + orc.epilogue("silu_mul", y2, aux),
                               rtol=1e-11, atol=1e-11)
    with pytest.raises(ValueError):
        orc.epilogue("add", y, aux[:1])
    with pytest.raises(ValueError):
        orc.epilogue("relu", y, aux)


@pytest.mark.parametrize("mistake", [
    lambda a: a / (1.0 + np.exp(a)),            # flipped sign in the exponent
    lambda a: 1.0 / (1.0 + np.exp(-a)),         # sigmoid without the factor a
    lambda a: a * (1.0 / (1.0 + np.exp(-2 * a))),  # wrong slope
])
def test_planted_silu_mistakes_fail_the_identities(mistake):
    a = np.linspace(-6.0, 6.0, 121)
    with np.errstate(over="ignore"):
        s = mistake(a)
    ok_pair = np.allclose(s - mistake(-a), a, rtol=1e-12, atol=1e-12)
    from scipy.special import expit
    ok_ref = np.allclose(s, a * expit(a), rtol=1e-12, atol=1e-12)
    assert not (ok_pair and ok_ref)


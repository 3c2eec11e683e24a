"""CPU oracle for the three-core tensor-ring linear operator.

TEST INFRASTRUCTURE ONLY. Nothing in the product imports this module: only `tests/`,
`__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` use it, and only as the
checker (or, for `cpu_baseline`, as the timed CPU port of the reference path). The product
path (`factorized_inference.prepare_optimized`) runs the HIP library and raises when it is
missing.

Operator (reference: IMPLEMENTATION.md:7-10):

    W[(p,q,r), (i,j,k)] = sum_{a,b,c} G1[a,p,i,b] * G2[b,q,j,c] * G3[c,r,k,a]
    y[t, (p,q,r)]       = sum_{(i,j,k)} x[t, (i,j,k)] * W[(p,q,r), (i,j,k)]

Core k has shape (rank, output_mode[k], input_mode[k], rank) (reference.py:19-20).
x is row-major [T, in] with in = (i*nj + j)*nk + k; y is row-major [T, out] with
out = (p*Q + q)*Rr + r (reference.py:119, :125).

Functions and the reference lines they restate:
  tr_forward        three pairwise contractions in the reference's fixed order
                    (src/factorized_inference/reference.py:99-125)
  dense_weight      the dense oracle W (reference.py:128-143)
  dense_forward     y = x @ W^T (reference.py:146-149)
  trace_entry       one W entry by the trace definition (tests/test_correctness.py:80-91)
  forward_pieces    y as the sum over (a, k) of independent pieces
                    (kernel_work/pieces_cpu.py:15-33)
  kron_weight       the rank-1 special case W = G1_0 (x) G2_0 (x) G3_0 (textbook Kronecker)
  chain_forward     the same operator contracted in any core order (F, S, L); the HIP
                    kernels use such orders, this is their CPU statement
  errors            max-abs / mean-abs / rel-L2 (benchmarks/benchmark.py:66-75)
  silu              silu(a) = a * sigmoid(a), the gate of the reference's fp32-output
                    consumer consume_silu_mul (src/factorized_inference/csrc/v3g/bind.cu:96-110)
  epilogue          what an output store writes for an accumulated y: y itself, silu(a)*y
                    (consume_silu_mul, bind.cu:96-110) or a + y (consume_add, bind.cu:112-122)

Pinning (what makes each function trustworthy, see tests/test_oracle.py):
  tr_forward, dense_weight, dense_forward, forward_pieces, chain_forward: agree with the
  brute-force trace definition on small specs in float64 (1e-12), with numpy.kron at
  rank 1, and with the invariants (linearity, trilinearity, one-hot columns, gauge
  invariance of the ring, cyclic rotation); a planted index mistake must fail these.
  trace_entry: the reference's own known-answer test (tests/test_correctness.py:80-91) and
  numpy.kron at rank 1. Also checked against the independent C restatement
  (oracle/ring_oracle.c) and the committed golden vectors (tests/golden/).
  silu, epilogue: scipy.special.expit (an independent logistic function), the closed-form
  identities silu(0) = 0, silu(a) - silu(-a) = a, silu(a) -> a and -> 0 at the far ends,
  and planted mistakes (a flipped sign, a dropped factor) that must fail them.
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "tr_forward", "dense_weight", "dense_forward", "trace_entry", "forward_pieces",
    "kron_weight", "chain_forward", "errors", "flops_per_token", "CHAIN_ORDERS", "silu",
    "epilogue", "EPILOGUES",
]

# Output epilogues, named as the kernels' (include/trk.h: enum trk_epilogue).
EPILOGUES = ("store", "f32", "add", "silu_mul")


def _dims(cores):
    g1, g2, g3 = cores
    R = g1.shape[0]
    (_, P, ni, _), (_, Q, nj, _), (_, Rr, nk, _) = g1.shape, g2.shape, g3.shape
    return R, (ni, nj, nk), (P, Q, Rr)


def tr_forward(x, cores):
    """y = TR(G1,G2,G3) x by the reference's three pairwise contractions, in its order.

    reference.py:119-125:
      stage 1  I1[t,j,k,a,p,b] = sum_i     x[t,i,j,k]   G1[a,p,i,b]
      stage 2  I2[t,k,a,p,q,c] = sum_{j,b} I1[t,j,k,a,p,b] G2[b,q,j,c]
      stage 3  y[t,p,q,r]      = sum_{k,c,a} I2[t,k,a,p,q,c] G3[c,r,k,a]
    Each stage is one matrix product over the contracted indices (what torch's einsum does
    on the CPU: permute, then a BLAS product), in the dtype of the inputs.
    """
    g1, g2, g3 = cores
    R, (ni, nj, nk), (P, Q, Rr) = _dims(cores)
    T = x.shape[0]
    xm = x.reshape(T, ni, nj, nk)
    # stage 1: rows (t,j,k), contracted i, columns (a,p,b)
    lhs = xm.transpose(0, 2, 3, 1).reshape(T * nj * nk, ni)
    rhs = g1.transpose(2, 0, 1, 3).reshape(ni, R * P * R)
    i1 = (lhs @ rhs).reshape(T, nj, nk, R, P, R)                 # t j k a p b
    # stage 2: rows (t,k,a,p), contracted (j,b), columns (q,c)
    lhs = i1.transpose(0, 2, 3, 4, 1, 5).reshape(T * nk * R * P, nj * R)
    rhs = g2.transpose(2, 0, 1, 3).reshape(nj * R, Q * R)
    i2 = (lhs @ rhs).reshape(T, nk, R, P, Q, R)                  # t k a p q c
    # stage 3: rows (t,p,q), contracted (k,c,a), columns r
    lhs = i2.transpose(0, 3, 4, 1, 5, 2).reshape(T * P * Q, nk * R * R)
    rhs = g3.transpose(2, 0, 3, 1).reshape(nk * R * R, Rr)
    y = lhs @ rhs                                                # (t p q) r
    return y.reshape(T, P * Q * Rr)


def dense_weight(cores):
    """W[(p,q,r),(i,j,k)] (reference.py:128-143): first G1.G2 over b, then with G3 over
    (c, a). Oracle and baseline use only."""
    g1, g2, g3 = cores
    R, (ni, nj, nk), (P, Q, Rr) = _dims(cores)
    # G1G2[a,p,i,q,j,c] = sum_b G1[a,p,i,b] G2[b,q,j,c]
    ab = g1.reshape(R * P * ni, R) @ g2.reshape(R, Q * nj * R)
    ab = ab.reshape(R, P, ni, Q, nj, R)
    # W[p,q,r,i,j,k] = sum_{c,a} G1G2[a,p,i,q,j,c] G3[c,r,k,a]
    lhs = ab.transpose(1, 2, 3, 4, 5, 0).reshape(P * ni * Q * nj, R * R)   # (p i q j) (c a)
    rhs = g3.transpose(0, 3, 1, 2).reshape(R * R, Rr * nk)                 # (c a) (r k)
    w = (lhs @ rhs).reshape(P, ni, Q, nj, Rr, nk)
    return w.transpose(0, 2, 4, 1, 3, 5).reshape(P * Q * Rr, ni * nj * nk)


def dense_forward(x, w):
    """y = x @ W^T (reference.py:146-149)."""
    return x @ w.T


def trace_entry(cores, out_index, in_index):
    """W[(p,q,r),(i,j,k)] = trace(G1[:,p,i,:] @ G2[:,q,j,:] @ G3[:,r,k,:]), by explicit
    sums over the three ring links (the definition, tests/test_correctness.py:80-91)."""
    g1, g2, g3 = cores
    R, (ni, nj, nk), (P, Q, Rr) = _dims(cores)
    p, rem = divmod(out_index, Q * Rr)
    q, r = divmod(rem, Rr)
    i, rem = divmod(in_index, nj * nk)
    j, k = divmod(rem, nk)
    total = 0.0
    for a in range(R):
        for b in range(R):
            for c in range(R):
                total += float(g1[a, p, i, b]) * float(g2[b, q, j, c]) * float(g3[c, r, k, a])
    return total


def forward_pieces(x, cores):
    """y as the sum of R*nk independent pieces piece(a, k) (kernel_work/pieces_cpu.py:15-33):
    piece(a,k)[t,p,q,r] = sum_c (sum_{j,b} (sum_i x[t,i,j,k] G1[a,p,i,b]) G2[b,q,j,c]) G3[c,r,k,a]."""
    g1, g2, g3 = cores
    R, (ni, nj, nk), (P, Q, Rr) = _dims(cores)
    T = x.shape[0]
    xm = x.reshape(T, ni, nj, nk)
    y = np.zeros((T, P, Q, Rr), dtype=np.result_type(x, g1))
    for a in range(R):
        for k in range(nk):
            s1 = np.einsum("tij,pib->tpjb", xm[:, :, :, k], g1[a])
            s2 = np.einsum("tpjb,bqjc->tpqc", s1, g2)
            y += np.einsum("tpqc,cr->tpqr", s2, g3[:, :, k, a])
    return y.reshape(T, P * Q * Rr)


def kron_weight(cores):
    """Rank 1: W = G1[0,:,:,0] (x) G2[0,:,:,0] (x) G3[0,:,:,0] (Kronecker product)."""
    g1, g2, g3 = cores
    if g1.shape[0] != 1:
        raise ValueError("kron_weight needs rank 1")
    return np.kron(g1[0, :, :, 0], np.kron(g2[0, :, :, 0], g3[0, :, :, 0]))


# The six orders in which the three cores can be contracted with x, as (first, second, last)
# core indices. (0,1,2), (1,2,0), (2,0,1) follow the ring forward, the others backward.
CHAIN_ORDERS = ((0, 1, 2), (1, 2, 0), (2, 0, 1), (0, 2, 1), (1, 0, 2), (2, 1, 0))


def chain_forward(x, cores, order):
    """The same operator, contracted core by core in `order` = (F, S, L).

    With the cores re-indexed as chain cores Fc[r1,f,iF,r2], Sc[r2,s,iS,r3], Lc[r3,l,iL,r1]
    (r1 = link L-F, r2 = link F-S, r3 = link S-L; a backward order transposes the two ring
    indices of every core):
      stage 1  U[t,iS,iL,r1,f,r2] = sum_iF        x[t,iF,iS,iL] Fc[r1,f,iF,r2]
      stage 2  V[t,iL,r1,f,s,r3]  = sum_{iS,r2}   U Sc[r2,s,iS,r3]
      stage 3  y[t,f,s,l]         = sum_{iL,r1,r3} V Lc[r3,l,iL,r1]
    then y is permuted back to (p,q,r). order=(0,1,2) is exactly tr_forward.
    """
    F, S, L = order
    forward = (S - F) % 3 == 1
    if sorted(order) != [0, 1, 2]:
        raise ValueError("order must be a permutation of (0, 1, 2)")
    g = [c if forward else c.transpose(3, 1, 2, 0) for c in cores]
    R, in_modes, out_modes = _dims(cores)
    T = x.shape[0]
    xm = x.reshape(T, *in_modes).transpose(0, 1 + F, 1 + S, 1 + L)  # t iF iS iL
    nF, nS, nL = in_modes[F], in_modes[S], in_modes[L]
    oF, oS, oL = out_modes[F], out_modes[S], out_modes[L]
    fc, sc, lc = g[F], g[S], g[L]
    lhs = xm.transpose(0, 2, 3, 1).reshape(T * nS * nL, nF)
    rhs = fc.transpose(2, 0, 1, 3).reshape(nF, R * oF * R)
    u = (lhs @ rhs).reshape(T, nS, nL, R, oF, R)                 # t iS iL r1 f r2
    lhs = u.transpose(0, 2, 3, 4, 1, 5).reshape(T * nL * R * oF, nS * R)
    rhs = sc.transpose(2, 0, 1, 3).reshape(nS * R, oS * R)
    v = (lhs @ rhs).reshape(T, nL, R, oF, oS, R)                 # t iL r1 f s r3
    lhs = v.transpose(0, 3, 4, 1, 2, 5).reshape(T * oF * oS, nL * R * R)
    rhs = lc.transpose(2, 3, 0, 1).reshape(nL * R * R, oL)       # (iL r1 r3) l
    y = (lhs @ rhs).reshape(T, oF, oS, oL)                       # t f s l
    inverse = np.argsort((F, S, L))
    y = y.transpose(0, *(1 + inverse))                           # t p q r
    return y.reshape(T, -1)


def flops_per_token(in_modes, out_modes, rank, order=(0, 1, 2)):
    """Multiply-adds x 2 per token of the chain contraction in `order` (no padding).

    For order (0,1,2) this is the reference's count (tools/measure_kernels.py:36-44):
    2*(ni*nj*nk*P*R^2 + nj*nk*P*Q*R^3 + nk*P*Q*Rr*R^2)."""
    F, S, L = order
    n, o, R = in_modes, out_modes, rank
    total_in = n[0] * n[1] * n[2]
    total_out = o[0] * o[1] * o[2]
    s1 = total_in * o[F] * R * R
    s2 = n[S] * n[L] * o[F] * o[S] * R ** 3
    s3 = n[L] * total_out * R * R
    return 2 * (s1 + s2 + s3)


def errors(actual, expected):
    """max-abs, mean-abs and relative-L2 error (benchmarks/benchmark.py:66-75)."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    d = np.abs(a - e)
    return {
        "max_absolute_error": float(d.max()) if d.size else 0.0,
        "mean_absolute_error": float(d.mean()) if d.size else 0.0,
        "relative_l2_error": float(np.linalg.norm(d) / max(np.linalg.norm(e), 1e-12)),
    }


def silu(a):
    """silu(a) = a * sigmoid(a) = a / (1 + exp(-a)), float64, overflow-safe at both ends.

    The gate of the SwiGLU MLP that the reference's consume_silu_mul applies to its fp32
    gate output (src/factorized_inference/csrc/v3g/bind.cu:96-110: g / (1 + exp(-g)) * u)."""
    a = np.asarray(a, dtype=np.float64)
    e = np.exp(-np.abs(a))               # in (0, 1]: never overflows
    sig = np.where(a >= 0, 1.0 / (1.0 + e), e / (1.0 + e))
    return a * sig


def epilogue(kind, y, aux=None):
    """What an output store writes for accumulated values y (float64):
      "store", "f32": y;  "add": aux + y (consume_add, bind.cu:112-122);
      "silu_mul": silu(aux) * y (consume_silu_mul with u = y, bind.cu:96-110)."""
    y = np.asarray(y, dtype=np.float64)
    if kind in ("store", "f32"):
        return y
    aux = np.asarray(aux, dtype=np.float64)
    if aux.shape != y.shape:
        raise ValueError(f"aux {aux.shape} does not match y {y.shape}")
    if kind == "add":
        return aux + y
    if kind == "silu_mul":
        return silu(aux) * y
    raise ValueError(f"unknown epilogue {kind!r}")


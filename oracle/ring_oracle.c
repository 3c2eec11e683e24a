/*
 * CPU oracle for the three-core tensor-ring linear operator, in plain C (float64).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (through ctypes) as a second, independent
 * restatement next to oracle/ring_oracle.py. The product never links or calls it.
 *
 * oracle_tr_forward_f64 restates src/factorized_inference/reference.py:99-125: the three
 * pairwise contractions in the reference's fixed order, with explicit loops
 *   stage 1  I1[t,j,k,a,p,b] = sum_i       x[t,i,j,k]      G1[a,p,i,b]
 *   stage 2  I2[t,k,a,p,q,c] = sum_{j,b}   I1[t,j,k,a,p,b] G2[b,q,j,c]
 *   stage 3  y[t,p,q,r]      = sum_{k,c,a} I2[t,k,a,p,q,c] G3[c,r,k,a]
 * oracle_dense_weight_f64 restates reference.py:128-143 entry by entry through the trace
 * definition W[(p,q,r),(i,j,k)] = trace(G1[:,p,i,:] G2[:,q,j,:] G3[:,r,k,:])
 * (tests/test_correctness.py:80-91).
 *
 * Layouts: core k is [R][o_k][i_k][R] row-major; x is [T][ni*nj*nk]; y is [T][P*Q*Rr].
 * Pinned by tests/test_oracle.py against the numpy oracle, the trace definition and the
 * Kronecker product at rank 1.
 */
#include <stdlib.h>
#include <string.h>

#define IDX4(a, b, c, d, B, C, D) ((((size_t)(a) * (B) + (b)) * (C) + (c)) * (D) + (d))

int oracle_tr_forward_f64(const double *x, int T, const double *g1, const double *g2,
                          const double *g3, const int *in_modes, const int *out_modes, int R,
                          double *y)
{
    const int ni = in_modes[0], nj = in_modes[1], nk = in_modes[2];
    const int P = out_modes[0], Q = out_modes[1], Rr = out_modes[2];
    if (T < 0 || R <= 0 || ni <= 0 || nj <= 0 || nk <= 0 || P <= 0 || Q <= 0 || Rr <= 0)
        return 1;
    const size_t in = (size_t)ni * nj * nk, out = (size_t)P * Q * Rr;
    /* per token: I1[j][k][a][p][b], I2[k][a][p][q][c] */
    double *i1 = (double *)malloc(sizeof(double) * (size_t)nj * nk * R * P * R);
    double *i2 = (double *)malloc(sizeof(double) * (size_t)nk * R * P * Q * R);
    if (!i1 || !i2) {
        free(i1);
        free(i2);
        return 2;
    }
    for (int t = 0; t < T; ++t) {
        const double *xt = x + (size_t)t * in;
        double *yt = y + (size_t)t * out;
        for (int j = 0; j < nj; ++j)
            for (int k = 0; k < nk; ++k)
                for (int a = 0; a < R; ++a)
                    for (int p = 0; p < P; ++p)
                        for (int b = 0; b < R; ++b) {
                            double s = 0.0;
                            for (int i = 0; i < ni; ++i)
                                s += xt[((size_t)i * nj + j) * nk + k] *
                                     g1[IDX4(a, p, i, b, P, ni, R)];
                            i1[((((size_t)j * nk + k) * R + a) * P + p) * R + b] = s;
                        }
        for (int k = 0; k < nk; ++k)
            for (int a = 0; a < R; ++a)
                for (int p = 0; p < P; ++p)
                    for (int q = 0; q < Q; ++q)
                        for (int c = 0; c < R; ++c) {
                            double s = 0.0;
                            for (int j = 0; j < nj; ++j)
                                for (int b = 0; b < R; ++b)
                                    s += i1[((((size_t)j * nk + k) * R + a) * P + p) * R + b] *
                                         g2[IDX4(b, q, j, c, Q, nj, R)];
                            i2[((((size_t)k * R + a) * P + p) * Q + q) * R + c] = s;
                        }
        for (int p = 0; p < P; ++p)
            for (int q = 0; q < Q; ++q)
                for (int r = 0; r < Rr; ++r) {
                    double s = 0.0;
                    for (int k = 0; k < nk; ++k)
                        for (int c = 0; c < R; ++c)
                            for (int a = 0; a < R; ++a)
                                s += i2[((((size_t)k * R + a) * P + p) * Q + q) * R + c] *
                                     g3[IDX4(c, r, k, a, Rr, nk, R)];
                    yt[((size_t)p * Q + q) * Rr + r] = s;
                }
    }
    free(i1);
    free(i2);
    return 0;
}

int oracle_dense_weight_f64(const double *g1, const double *g2, const double *g3,
                            const int *in_modes, const int *out_modes, int R, double *w)
{
    const int ni = in_modes[0], nj = in_modes[1], nk = in_modes[2];
    const int P = out_modes[0], Q = out_modes[1], Rr = out_modes[2];
    if (R <= 0 || ni <= 0 || nj <= 0 || nk <= 0 || P <= 0 || Q <= 0 || Rr <= 0)
        return 1;
    const size_t in = (size_t)ni * nj * nk;
    for (int p = 0; p < P; ++p)
        for (int q = 0; q < Q; ++q)
            for (int r = 0; r < Rr; ++r)
                for (int i = 0; i < ni; ++i)
                    for (int j = 0; j < nj; ++j)
                        for (int k = 0; k < nk; ++k) {
                            double s = 0.0;
                            for (int a = 0; a < R; ++a)
                                for (int b = 0; b < R; ++b)
                                    for (int c = 0; c < R; ++c)
                                        s += g1[IDX4(a, p, i, b, P, ni, R)] *
                                             g2[IDX4(b, q, j, c, Q, nj, R)] *
                                             g3[IDX4(c, r, k, a, Rr, nk, R)];
                            w[(((size_t)p * Q + q) * Rr + r) * in + ((size_t)i * nj + j) * nk + k] = s;
                        }
    return 0;
}

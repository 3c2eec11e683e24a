// Generic fused tensor-ring kernel: any modes, any rank, fp16 / bf16 / fp32, fp32 accumulation.
//
// Role of the reference's generic WMMA kernel (tr_ring.cu:104-338), own design: instead of
// splitting the ring into pieces over workgroups and reducing them through an fp32
// workspace with atomics and a last-block finish, one workgroup owns one token and one
// output digit f of the first core in the contraction chain, and loops over every piece
// (iL, r1) itself. No workspace, counter or second pass exists, the result is
// deterministic, and calls share no state.
//
// Per workgroup (f, t), for every last-core input digit iL and ring-link chunk r1:
//   stage 1  U[r1][iS][r2] = sum_iF      x[t, iF, iS, iL] * Fc[r1][f][iF][r2]
//   stage 2  V[r1][s][r3]  = sum_{iS,r2} U[r1][iS][r2]     * Sc[r2][s][iS][r3]
//   stage 3  Y[s][l]      += sum_{r1,r3} V[r1][s][r3]      * Lc[r3][l][iL][r1]
// with U, V and Y in LDS (fp32) and the cores read from the packed buffer (L2-resident).
// This is the fallback for shapes without a compiled MFMA variant; it runs on VALU FMAs.
#include <algorithm>

#include "trk_internal.h"
#include "trk_types.h"

namespace trk {
namespace {

constexpr int kThreads = 256;
constexpr int kLdsBudget = 64 * 1024;

struct GenericArgs {
    int T, in_features, out_features;
    int R, RC, SG, nSG;
    int nF, nS, nL, oF, oS, oL, KF, K2;
    int sxF, sxS, sxL, syF, syS, syL;
};

// Workgroup (f, sg) of token t owns y[t, f, s, :] for the SG second-core digits
// s in [sg*SG, sg*SG + SG). Stage 1 (the cheapest stage) is recomputed by every sg of an f;
// stage 2, the rank^3 stage, is split over them without overlap.
template <int DT>
__global__ void __launch_bounds__(kThreads) ring3_generic_kernel(
    const typename Elem<DT>::T *__restrict__ x, const typename Elem<DT>::T *__restrict__ Fk,
    const typename Elem<DT>::T *__restrict__ Sk, const typename Elem<DT>::T *__restrict__ Lk,
    void *y, GenericArgs a, const void *aux, int epi_mode) {  // aux may equal y
    using E = Elem<DT>;
    extern __shared__ float lds[];
    const int R = a.R, RC = a.RC, SG = a.SG;
    float *U = lds;                       // [RC][nS][R]
    float *V = U + RC * a.nS * R;         // [RC][SG][R]
    float *Y = V + RC * SG * R;           // [SG][oL]
    const int f = blockIdx.x / a.nSG;
    const int s0 = (blockIdx.x % a.nSG) * SG;
    const int SGv = min(SG, a.oS - s0);
    const int tid = threadIdx.x;
    const int nU = a.nS * R, nV = SGv * R, nY = SGv * a.oL;

    for (int t = blockIdx.y; t < a.T; t += gridDim.y) {
        const typename E::T *xt = x + size_t(t) * a.in_features;
        for (int i = tid; i < nY; i += kThreads) Y[i] = 0.0f;
        for (int iL = 0; iL < a.nL; ++iL) {
            for (int r1c = 0; r1c < R; r1c += RC) {
                const int rc = min(RC, R - r1c);
                // stage 1 (U was last read by stage 2 of the previous step, before a barrier)
                for (int idx = tid; idx < rc * nU; idx += kThreads) {
                    const int r1 = r1c + idx / nU;
                    const int iS = (idx % nU) / R, r2 = idx % R;
                    const typename E::T *fk = Fk + ((size_t(f) * R + r1) * R + r2) * a.KF;
                    const typename E::T *xs = xt + iS * a.sxS + iL * a.sxL;
                    float acc = 0.0f;
                    for (int iF = 0; iF < a.nF; ++iF)
                        acc += E::to_f32(xs[iF * a.sxF]) * E::to_f32(fk[iF]);
                    U[idx] = acc;
                }
                __syncthreads();
                // stage 2 (V was last read by stage 3 of the previous step, before the barrier above)
                for (int idx = tid; idx < rc * nV; idx += kThreads) {
                    const int r1 = idx / nV;
                    const int s = (idx % nV) / R, r3 = idx % R;
                    const float *u = U + r1 * nU;
                    const typename E::T *sk = Sk + (size_t(s0 + s) * R + r3) * a.K2;
                    float acc = 0.0f;
                    for (int k = 0; k < nU; ++k) acc += u[k] * E::to_f32(sk[k]);
                    V[(r1 * SG + s) * R + r3] = acc;
                }
                __syncthreads();
                // stage 3: each thread owns its Y entries, so no barrier follows
                for (int idx = tid; idx < nY; idx += kThreads) {
                    const int s = idx / a.oL, l = idx % a.oL;
                    const typename E::T *lk = Lk + ((size_t(iL) * a.oL + l) * R + r1c) * R;
                    float acc = Y[idx];
                    for (int r1 = 0; r1 < rc; ++r1) {
                        const float *v = V + (r1 * SG + s) * R;
                        for (int r3 = 0; r3 < R; ++r3) acc += v[r3] * E::to_f32(lk[r1 * R + r3]);
                    }
                    Y[idx] = acc;
                }
            }
        }
        const size_t yt = size_t(t) * a.out_features + size_t(f) * a.syF;
        for (int idx = tid; idx < nY; idx += kThreads) {
            const int s = idx / a.oL, l = idx % a.oL;
            const size_t o = yt + (s0 + s) * a.syS + l * a.syL;
            epi_put<DT>(y, epi_mode, o, Y[idx], epi_aux<DT>(aux, epi_mode, o));
        }
        __syncthreads();  // U of the next token is written after every thread left stage 2
    }
}

__global__ void ring3_empty_kernel() {}

int lds_bytes(const Chain &c, int rc, int sg) {
    return 4 * (rc * c.R * (c.nS + sg) + sg * c.oL);
}

}  // namespace

int generic_configure(const Plan &plan, int chain, int sg, Variant *v) {
    const Chain &c = plan.chains[chain];
    if (sg < 1 || sg > c.oS) return set_error(TRK_ERR_INVALID, "generic kernel: bad s-chunk %d", sg);
    int rc = c.R;
    while (rc > 1 && lds_bytes(c, rc, sg) > kLdsBudget) rc = (rc + 1) / 2;
    if (lds_bytes(c, rc, sg) > kLdsBudget)
        return set_error(TRK_ERR_UNSUPPORTED,
                         "generic kernel: second/last core outputs too large for LDS");
    v->kind = TRK_KERNEL_GENERIC;
    v->chain = chain;
    v->tile[0] = 1;
    v->tile[1] = 1;
    v->tile[2] = sg;
    v->tile[3] = c.oL;
    v->tile[4] = rc;
    v->block = kThreads;
    v->lds_bytes = lds_bytes(c, rc, sg);
    v->launch = launch_generic;
    static const char kNames[] = "012";
    snprintf(v->name, sizeof(v->name), "ring3_generic<%c%c%c,rc=%d,sc=%d>", kNames[c.order[0]],
             kNames[c.order[1]], kNames[c.order[2]], rc, sg);
    return TRK_OK;
}

int launch_generic(const Plan &plan, const Variant &v, const void *packed, const void *x,
                   void *y, int tokens, Epi epi, hipStream_t stream) {
    const Chain &c = plan.chains[v.chain];
    GenericArgs a;
    a.T = tokens;
    a.in_features = plan.in_features;
    a.out_features = plan.out_features;
    a.R = c.R;
    a.RC = v.tile[4];
    a.SG = v.tile[2];
    a.nSG = (c.oS + a.SG - 1) / a.SG;
    a.nF = c.nF;
    a.nS = c.nS;
    a.nL = c.nL;
    a.oF = c.oF;
    a.oS = c.oS;
    a.oL = c.oL;
    a.KF = c.KF;
    a.K2 = c.K2;
    a.sxF = c.sxF;
    a.sxS = c.sxS;
    a.sxL = c.sxL;
    a.syF = c.syF;
    a.syS = c.syS;
    a.syL = c.syL;
    const char *base = static_cast<const char *>(packed);
    const dim3 grid(c.oF * a.nSG, std::max(1, std::min(tokens, 65535)));
    switch (plan.dtype) {
#define TRK_LAUNCH_GENERIC(DT)                                                                 \
    case DT: {                                                                                 \
        using T = Elem<DT>::T;                                                                 \
        hipLaunchKernelGGL(ring3_generic_kernel<DT>, grid, dim3(kThreads), v.lds_bytes, stream, \
                           static_cast<const T *>(x), reinterpret_cast<const T *>(base + c.offF), \
                           reinterpret_cast<const T *>(base + c.offS),                         \
                           reinterpret_cast<const T *>(base + c.offL), y, a, epi.aux, epi.mode); \
        break;                                                                                 \
    }
        TRK_LAUNCH_GENERIC(TRK_DTYPE_F16)
        TRK_LAUNCH_GENERIC(TRK_DTYPE_BF16)
        TRK_LAUNCH_GENERIC(TRK_DTYPE_F32)
#undef TRK_LAUNCH_GENERIC
        default:
            return set_error(TRK_ERR_INVALID, "trk_forward: unknown dtype");
    }
    return check_hip(hipGetLastError(), "trk_forward: generic kernel launch");
}

int launch_empty(hipStream_t stream) {
    hipLaunchKernelGGL(ring3_empty_kernel, dim3(1), dim3(64), 0, stream);
    return check_hip(hipGetLastError(), "trk_empty_launch");
}

}  // namespace trk

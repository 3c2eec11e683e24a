// Packing of the three cores into the per-chain sections of the packed buffer.
//
// Replaces pack_cores (src/factorized_inference/tr_kernel.py:86-99): same idea (the same
// values re-laid out for the kernels, zero padding only, no expansion and no dense W), own
// layouts. For each chain (contraction order F, S, L) of the plan:
//   Fk[f][r1][r2][KF]  = Fc[r1][f][iF][r2]   for iF < nF, else 0
//   Sk[s][r3][K2]      = Sc[r2][s][iS][r3]   at k = (r2/sg)*sg*nS + iS*sg + r2%sg < nS*R,
//                                            else 0
//   Lk[iL][l][K]       = Lc[r3][l][iL][r1]   at K = (r3/lg)*lg*R + r1*lg + r3%lg
// (sg = lg = R: the natural orders k = iS*R + r2, K = r1*R + r3). A chain with sfrag stores
// Sk in the order the register-resident 32x32x16 A fragments are loaded: for each tile of 32
// rows (s, r3) and each step of 16 k, the 64 lanes' 8-element pieces one after another
// (lane = 32 * (k % 16 / 8) + row % 32), rows past oS*R zero. Only the sections a chain owns
// are written; the others are shared with an earlier chain of the same order.
// where a chain core Xc[in][o][i][out] is the core G[in][o][i][out] of a forward order and
// G[out][o][i][in] of a backward one. Bits are copied, so the dtype does not matter beyond
// its width.
#include <algorithm>

#include "trk_internal.h"

namespace trk {
namespace {

// index of G[alpha][o][i][beta] in a core of shape [R][O][I][R]
__device__ inline size_t core_index(int alpha, int o, int i, int beta, int O, int I, int R) {
    return ((size_t(alpha) * O + o) * I + i) * R + beta;
}

struct PackArgs {
    int R, Rc, forward;  // kernel rank; rank of the cores read (ring indices >= Rc pack zero)
    int nF, nS, nL, oF, oS, oL, KF, K2, sg, lg, sfrag;
    size_t nFk, nSk, nLk;  // element counts of the three sections
};

template <typename W>
__global__ void __launch_bounds__(256) pack_chain_kernel(const W *__restrict__ gF,
                                                         const W *__restrict__ gS,
                                                         const W *__restrict__ gL,
                                                         W *__restrict__ Fk, W *__restrict__ Sk,
                                                         W *__restrict__ Lk, PackArgs a) {
    const size_t total = a.nFk + a.nSk + a.nLk;
    const int R = a.R;
    for (size_t d = blockIdx.x * size_t(blockDim.x) + threadIdx.x; d < total;
         d += size_t(gridDim.x) * blockDim.x) {
        if (d < a.nFk) {
            const int iF = int(d % a.KF);
            size_t rest = d / a.KF;
            const int r2 = int(rest % R);
            rest /= R;
            const int r1 = int(rest % R);
            const int f = int(rest / R);
            W v = W(0);
            if (iF < a.nF && r1 < a.Rc && r2 < a.Rc)
                v = gF[a.forward ? core_index(r1, f, iF, r2, a.oF, a.nF, a.Rc)
                                 : core_index(r2, f, iF, r1, a.oF, a.nF, a.Rc)];
            Fk[d] = v;
        } else if (d < a.nFk + a.nSk) {
            const size_t e = d - a.nFk;
            int k, row;
            if (a.sfrag) {  // [tile][k / 16][lane][8]
                const int lane = int(e / 8 % 64), ks = a.K2 / 16;
                const size_t rest = e / 512;
                k = int(rest % ks) * 16 + lane / 32 * 8 + int(e % 8);
                row = int(rest / ks) * 32 + lane % 32;
            } else {
                k = int(e % a.K2);
                row = int(e / a.K2);
            }
            const int r3 = row % R, s = row / R;
            W v = W(0);
            if (k < a.nS * R && s < a.oS) {
                const int span = a.sg * a.nS, rem = k % span;
                const int iS = rem / a.sg, r2 = k / span * a.sg + rem % a.sg;
                if (r2 < a.Rc && r3 < a.Rc)
                    v = gS[a.forward ? core_index(r2, s, iS, r3, a.oS, a.nS, a.Rc)
                                     : core_index(r3, s, iS, r2, a.oS, a.nS, a.Rc)];
            }
            Sk[e] = v;
        } else {
            const size_t e = d - a.nFk - a.nSk;
            const int kk = int(e % (size_t(R) * R)), span = a.lg * R, rem = kk % span;
            const int r1 = rem / a.lg, r3 = kk / span * a.lg + rem % a.lg;
            size_t rest = e / (size_t(R) * R);
            const int l = int(rest % a.oL);
            const int iL = int(rest / a.oL);
            W v = W(0);
            if (r1 < a.Rc && r3 < a.Rc)
                v = gL[a.forward ? core_index(r3, l, iL, r1, a.oL, a.nL, a.Rc)
                                 : core_index(r1, l, iL, r3, a.oL, a.nL, a.Rc)];
            Lk[e] = v;
        }
    }
}

template <typename W>
int pack_all(const Plan &plan, const void *const g[3], void *packed, hipStream_t stream) {
    char *base = static_cast<char *>(packed);
    for (int ci = 0; ci < plan.nchains; ++ci) {
        const Chain &c = plan.chains[ci];
        PackArgs a;
        a.R = c.R;
        a.Rc = plan.core_rank;
        a.forward = c.forward;
        a.nF = c.nF;
        a.nS = c.nS;
        a.nL = c.nL;
        a.oF = c.oF;
        a.oS = c.oS;
        a.oL = c.oL;
        a.KF = c.KF;
        a.K2 = c.K2;
        a.sg = c.sg;
        a.lg = c.lg;
        a.sfrag = c.sfrag;
        a.nFk = c.ownF ? size_t(c.oF) * c.R * c.R * c.KF : 0;
        a.nSk = c.ownS ? size_t(c.sfrag ? (c.oS * c.R + 31) / 32 * 32 : c.oS * c.R) * c.K2 : 0;
        a.nLk = c.ownL ? size_t(c.nL) * c.oL * c.R * c.R : 0;
        const size_t total = a.nFk + a.nSk + a.nLk;
        if (total == 0) continue;
        const int blocks = int(std::min<size_t>((total + 255) / 256, 4096));
        hipLaunchKernelGGL(pack_chain_kernel<W>, dim3(blocks), dim3(256), 0, stream,
                           static_cast<const W *>(g[c.order[0]]),
                           static_cast<const W *>(g[c.order[1]]),
                           static_cast<const W *>(g[c.order[2]]),
                           reinterpret_cast<W *>(base + c.offF),
                           reinterpret_cast<W *>(base + c.offS),
                           reinterpret_cast<W *>(base + c.offL), a);
        const int st = check_hip(hipGetLastError(), "trk_pack: launch");
        if (st != TRK_OK) return st;
    }
    return TRK_OK;
}

}  // namespace

int launch_pack(const Plan &plan, const void *g1, const void *g2, const void *g3, void *packed,
                hipStream_t stream) {
    const void *g[3] = {g1, g2, g3};
    if (plan.elem == 4) return pack_all<uint32_t>(plan, g, packed, stream);
    return pack_all<uint16_t>(plan, g, packed, stream);
}

}  // namespace trk

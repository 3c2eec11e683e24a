// Internal declarations shared by the HIP sources of libtrk (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "trk.h"

namespace trk {

constexpr int kMaxVariants = 256;  // an autotuning build compiles up to ~180 tiles per shape
constexpr int kMaxChains = 12;

// One contraction order, in chain terms. The cores are re-indexed as chain cores
//   Fc[r1][f][iF][r2], Sc[r2][s][iS][r3], Lc[r3][l][iL][r1]
// (r1 = link L-F, r2 = link F-S, r3 = link S-L). A forward order follows the ring
// (G1 -> G2 -> G3 up to rotation) and keeps every core as it is; a backward order swaps the
// two ring indices of every core. In the packed buffer each chain has three sections:
//   Fk[f][r1][r2][KF]  (iF fastest, zero-padded to KF)    first core, stage-1 operand
//   Sk[s][r3][K2]      (k = (r2/sg)*sg*nS + iS*sg + r2%sg, zero-padded to K2)
//                                                        second core, stage-2 operand
//   Lk[iL][l][K]       (K = (r3/lg)*lg*R + r1*lg + r3%lg) last core, stage-3 operand
// The K-order groups sg and lg equal R for the natural orders (iS, r2) and (r1, r3); the MFMA
// kernels use smaller groups, which make their result stores bank-conflict free, and the
// generic kernel reads any grouping. Chains of one order share the sections whose layout
// agrees.
struct Chain {
    int order[3];    // F, S, L: core indices
    int forward;     // 1 if the order follows the ring
    int nF, nS, nL;  // input modes of F, S, L
    int oF, oS, oL;  // output modes of F, S, L
    int R;
    int KF, K2;      // padded stage-1 and stage-2 contraction lengths
    int sg, lg;      // K-order groups of the Sk and Lk sections
    int sfrag;       // 1: Sk in 32x32x16 fragment order (trk_pack.hip)
    int sxF, sxS, sxL;  // element strides of iF, iS, iL in a row of x
    int syF, syS, syL;  // element strides of f, s, l in a row of y
    size_t offF, offS, offL;  // byte offsets of Fk, Sk, Lk in the packed buffer
    int ownF, ownS, ownL;     // 1 where this chain is the first with that section (packs it)
};

struct Plan;
struct Variant;

// Output stage of a launch (enum trk_epilogue): `mode` is the epilogue kind, plus kAuxF32
// when aux is fp32 rather than the plan's dtype.
struct Epi {
    const void *aux;
    int mode;
};
constexpr int kEpiKindMask = 15;
constexpr int kAuxF32 = 16;

using LaunchFn = int (*)(const Plan &, const Variant &, const void *packed, const void *x,
                         void *y, int tokens, Epi epi, hipStream_t stream);
// y = silu(G x) * (U x) for the gate and up operators of one plan layout (trk_forward_swiglu)
using LaunchPairFn = int (*)(const Plan &, const Variant &, const void *packed_g,
                             const void *packed_u, const void *x, void *y, int tokens,
                             hipStream_t stream);

struct Variant {
    int kind;        // trk_kernel_kind
    int chain;       // index into Plan::chains
    int tile[5];     // TT, FC, SC, LC, IC (generic: IC = ring-link chunk)
    int block;       // threads per workgroup
    int lds_bytes;   // dynamic LDS per workgroup
    int t_min, t_max;
    int xcd_local;   // XCDs the launch's work runs on: 0 = all 8; 1, 2, 4 (KCfg::XL; grid x 8/XL)
    char name[64];
    LaunchFn launch;
    LaunchPairFn launch_pair;  // fused SwiGLU gate/up launcher, or null
};

struct Plan {
    int in_modes[3], out_modes[3], rank, dtype, elem;
    int core_rank;  // rank of the cores trk_pack reads (<= rank; the rest is zero padding)
    int in_features, out_features;
    int nchains;
    Chain chains[kMaxChains];
    int nvariants;
    Variant variants[kMaxVariants];
    size_t packed_bytes;
};

// error reporting (trk_api.hip)
int set_error(int status, const char *fmt, ...);
int check_hip(hipError_t err, const char *what);

// chain geometry (trk_api.hip)
void describe_chain(const int in_modes[3], const int out_modes[3], int rank, const int order[3],
                    Chain *chain);
// index of the plan's chain with this order and K-order groups, added if new (-1: full)
int plan_chain(Plan *plan, const int order[3], int sg, int lg, int sfrag);

// Entry points a variant module (a generated table built at prepare time) exports, and the
// layout check its loader applies: the module's sizeof(Plan) must equal the library's.
using ModuleRegisterFn = int (*)(Plan *plan);
using ModuleSizeFn = size_t (*)();
constexpr const char *kModuleRegister = "trk_module_register";
constexpr const char *kModulePlanSize = "trk_module_plan_size";
constexpr const char *kModuleAbi = "trk_module_abi";

// kernels and their launchers
int launch_pack(const Plan &plan, const void *g1, const void *g2, const void *g3, void *packed,
                hipStream_t stream);                                   // trk_pack.hip
// generic kernel variant of `chain` whose workgroups own `sg` second-core outputs each
int generic_configure(const Plan &plan, int chain, int sg, Variant *v);  // trk_generic.hip
int launch_generic(const Plan &plan, const Variant &v, const void *packed, const void *x,
                   void *y, int tokens, Epi epi, hipStream_t stream);  // trk_generic.hip
int launch_empty(hipStream_t stream);                                  // trk_generic.hip
int launch_empty_args(hipStream_t stream);                             // trk_generic.hip
// elementwise consumers of fp32 outputs (trk_consume.hip)
int launch_silu_mul(const float *g, const float *u, void *out, int out_dtype, size_t n,
                    hipStream_t stream);
int launch_add(const void *h, const float *y, void *out, int dtype, size_t n, hipStream_t stream);

// MFMA variants of the declared shapes (csrc/gen/, one generated translation unit per shape,
// written by factorized_inference/tilegen.py): appends the variants of the plan's shape and
// returns how many were added.
int mfma_register_generated(Plan *plan);

}  // namespace trk

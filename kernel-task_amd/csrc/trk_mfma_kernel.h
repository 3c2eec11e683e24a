#pragma once
// MFMA (gfx950 matrix core) variants of the fused tensor-ring kernel, fp16 and bf16: the
// kernel template, its launch and the variant-table helpers. The tables themselves are
// generated per declared shape (csrc/gen/trk_gen_<shape>.hip, written by
// factorized_inference/tilegen.py), one translation unit per shape.
//
// Role of the reference's V3 / V3T / V3G kernels (tr_ring.cu:543-751, :822-1056,
// csrc/v3g/v3g.cuh:142-431); own design for CDNA4:
//
// * Output-stationary workgroups. A workgroup owns a tile of the output: TT tokens x FC
//   digits f of the first chain core x SC digits s of the second x LC digits l of the last,
//   and loops over every ring piece (iL, r1) itself. There is no fp32 workspace, no atomic
//   reduction across workgroups and no last-block finish, so nothing crosses the per-XCD L2
//   caches and a call leaves no state behind. The price is recomputing stage 1 once per
//   (s, l) chunk, which the chain order and tile choice keep small.
// * Any contraction order. The host packs the cores for the chain (F, S, L) the variant
//   uses (trk_pack.hip); the order is picked per shape to cut the rank^3 stage.
// * Three MFMA GEMMs per step of IC last-core input digits, operands and results in LDS,
//   each stored K-contiguous so every fragment is one 16- or 8-byte LDS read:
//     stage 1  U^T[(f,r1,r2), (iL',t,iS)] = Fs[(f,r1,r2), iF]  . Xs[(iL',t,iS), iF]
//     stage 2  V^T[(s,r3), (iL',r1,t,f)]  = Ss[(s,r3),(iS,r2)] . Ub[(iL',r1,t,f),(iS,r2)]
//     stage 3  Y[(t,f,s), l]            += Vb[(t,f,s),(iL',r1,r3)] . Ls[iL'][l][(r1,r3)]
//   A stage's fp32 accumulator rows run along the next stage's K index, so each lane writes
//   its 4 results as one 8-byte vector in exactly the layout the next stage reads.
//   Stage 3 accumulates Y in registers over all steps; with fewer Y tiles than waves, its K
//   range is split over waves and the partial tiles are summed through LDS at the end.
//   Pipelined tiles (PIPE) double-buffer the last-core and x slices so that stage 3 of a
//   step and stage 1 of the next share one barrier interval: two barriers per step, not four.
// * 16x16x32 MFMAs (16x16x16 for a K of 16 alone; a trailing 16 after 32-wide steps is one
//   more 16x16x32 MFMA with a zero upper half), wave64, 4 or 8 waves per workgroup;
//   the register-resident (WIDE) family runs stage 2 on 32x32x16 MFMAs.
//
// Variants are compiled for the declared shapes and their tuned token ranges; plans for
// other shapes use the generic kernel (trk_generic.hip).
#include <algorithm>
#include <cstdio>
#include <type_traits>

#include "trk_internal.h"
#include "trk_types.h"

namespace trk {
namespace {

using f32x4 = float __attribute__((ext_vector_type(4)));

// The kernel body's helper lambdas capture register arrays (prefetched slices, accumulators)
// by reference: one that the compiler leaves as a call puts those arrays in scratch memory
// (measured: a 3.5x slower tile), so every one is inlined.
#define TRK_INLINE __attribute__((always_inline))
using f32x16 = float __attribute__((ext_vector_type(16)));

// Accumulator of a 16x16xK MFMA chain. Each MFMA of Ops takes and returns the accumulator
// type of its own K, so a chain that mixes 16x16x32 and 16x16x16 MFMAs on one accumulator
// does not compile: such a mixed chain gave wrong sums on gfx950 in one schedule (the first two
// of every four accumulator elements short of their last contributions). A K that ends in 16
// after 32-wide steps therefore finishes with one more 16x16x32 MFMA whose upper K half is
// zero; 16x16x16 MFMAs only serve a K of 16 alone, on an Acc<16> of their own.
template <int K>
struct Acc {
    f32x4 v;
};

template <int DT>
struct Ops;

template <>
struct Ops<TRK_DTYPE_F16> {
    using E = _Float16;
    using V8 = _Float16 __attribute__((ext_vector_type(8)));
    using V4 = _Float16 __attribute__((ext_vector_type(4)));
    using E4 = V4;
    __device__ static Acc<32> k32(V8 a, V8 b, Acc<32> c) {
        return {__builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c.v, 0, 0, 0)};
    }
    __device__ static Acc<16> k16(V4 a, V4 b, Acc<16> c) {
        return {__builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c.v, 0, 0, 0)};
    }
    __device__ static f32x16 w16(V8 a, V8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
};

template <>
struct Ops<TRK_DTYPE_BF16> {
    using E = __bf16;
    using V8 = __bf16 __attribute__((ext_vector_type(8)));
    using V4 = short __attribute__((ext_vector_type(4)));  // the K16 bf16 MFMA takes raw bits
    using E4 = __bf16 __attribute__((ext_vector_type(4)));
    __device__ static Acc<32> k32(V8 a, V8 b, Acc<32> c) {
        return {__builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c.v, 0, 0, 0)};
    }
    __device__ static Acc<16> k16(V4 a, V4 b, Acc<16> c) {
        return {__builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c.v, 0, 0, 0)};
    }
    __device__ static f32x16 w16(V8 a, V8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
};

// fp32: the same fragments (8 or 4 K-consecutive elements per lane) as sequences of fp32
// MFMAs of K 4 (16x16x4) or 2 (32x32x2), each taking one element per lane: step q runs the K
// positions {q, 8 + q, 16 + q, 24 + q} (16x16x32 fragment) or {q, 8 + q} (32x32x16), so the
// sum over q covers the fragment's K range once, in full fp32 (no reduced-precision inputs).
template <>
struct Ops<TRK_DTYPE_F32> {
    using E = float;
    using V8 = float __attribute__((ext_vector_type(8)));
    using V4 = float __attribute__((ext_vector_type(4)));
    using E4 = V4;
    __device__ static Acc<32> k32(V8 a, V8 b, Acc<32> c) {
#pragma unroll
        for (int q = 0; q < 8; ++q) c.v = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], b[q], c.v, 0, 0, 0);
        return c;
    }
    __device__ static Acc<16> k16(V4 a, V4 b, Acc<16> c) {
#pragma unroll
        for (int q = 0; q < 4; ++q) c.v = __builtin_amdgcn_mfma_f32_16x16x4f32(a[q], b[q], c.v, 0, 0, 0);
        return c;
    }
    __device__ static f32x16 w16(V8 a, V8 b, f32x16 c) {
#pragma unroll
        for (int q = 0; q < 8; ++q) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[q], b[q], c, 0, 0, 0);
        return c;
    }
};

constexpr int cdiv(int a, int b) { return (a + b - 1) / b; }
constexpr int rup(int a, int b) { return cdiv(a, b) * b; }
constexpr int pick(int m, int a, int b, int c) { return m == 0 ? a : (m == 1 ? b : c); }

// One compiled variant: dtype, shape, contraction order and workgroup tile.
struct KCfg {
    int dt;
    int F, S, L;     // contraction order (core indices)
    int i0, i1, i2;  // input modes (i, j, k)
    int o0, o1, o2;  // output modes (p, q, r)
    int R;
    int TT, FC, SC, LC, IC;  // tokens, f / s / l digits per workgroup, iL digits per step
    int KS3;                 // waves sharing one stage-3 tile (split of its K range)
    int NACC;                // independent accumulator chains per stage-3 tile and wave
    int WIDE;                // 0: core slices in LDS. 1, 2 or 4: the first- and second-core
                             // slices live in registers, and WIDE waves split the stage-2
                             // rows while 4 / WIDE waves split its columns
    int MF2;                 // WIDE stage-2 MFMA: 16 (16x16x32) or 32 (32x32x16, twice the
                             // matrix-core throughput of 16x16x32 on gfx950)
    int NW;                  // waves per workgroup: 4 (one per SIMD) or 8 (two per SIMD)
    int PIPE;                // 1: the last-core and x slices are double-buffered, and stage 3
                             // of a step shares a barrier interval with stage 1 of the next
                             // (two barriers per step instead of four); 2: the stage results
                             // (Ub, Vb) are double-buffered too, and stages 1, 2 and 3 of three
                             // consecutive steps share one barrier interval; 0: one buffer
    int S1;                  // WIDE stage 1: row tiles per wave (the waves split the columns
                             // NW * S1 / M1T ways); 0: the default split (below)
    int XL;                  // XCDs the launch's work runs on: 0 = all 8; 1, 2 or 4 = the
                             // first XL. The grid is 8 / XL times larger and the dispatcher
                             // deals workgroups to the 8 XCDs round-robin; those dealt to XCDs
                             // XL..7 exit at once, so the working ones share XL L2s: each core
                             // slice crosses from HBM at most XL times and a cache line of y is
                             // written back by at most XL L2s (for launches that fit XL x 32 CUs)
    int YM;                  // workgroup -> (unit, token tile) numbering (unit_of_workgroup):
                             // 0 = per token tile, 1 = over the whole launch, each XCD taking
                             // one contiguous range of (token tile, unit), so every unit of a
                             // token tile, hence every writer of its lines of y, shares an L2
    int SL;                  // 1: the second-core slice arrives while the first stage 1 runs.
                             // WIDE: each wave reads it after the first step's slices are
                             // committed (the slice loads fill the CU's vector-memory queue,
                             // and a wave cannot pass them until its last one is issued);
                             // LDS-staged: it is read with the other slices but written to
                             // LDS after the first stage 1. 0: read, and written, with the
                             // first-core slice
    int TP;                  // pair-and-tail stage 2 (Geo::TAIL): 1 = the tail waves, which run
                             // one MFMA per K step, hold the SIMDs' issue priority while they
                             // run it (s_setprio), so that they finish before the waves with
                             // whole row tiles instead of after them, waiting on LDS alone
};

// K orders of the packed second- and last-core sections a variant reads (its chain's layout):
//   stage-2 K of (iS, r2)      = (r2 / SG) * SG * nS + iS * SG + r2 % SG
//   stage-3 K of (iL', r1, r3) = iL' * R^2 + (r3 / LG) * LG * R + r1 * LG + r3 % LG
// A group of R is the natural order (iS, r2) / (iL', r1, r3). Smaller groups put the four
// results one lane stores (4 consecutive r2 or r3) next to those of the neighbouring lanes, so
// that the stage-1 and stage-2 result stores of a half-wave fill every LDS bank once: with
// the natural order a rank-16 16x16 tile stores its lanes 32 bytes apart (2-way bank
// conflicts) and a 32x32 tile 32 bytes apart across its token planes (up to 4-way); measured
// on gfx950 the conflicting stores take 2.6x as long as contiguous ones. At rank 8 the natural
// orders already fill the banks for 16x16 tiles; its 32x32 tiles need a last-core group of 4.
constexpr int s_group(const KCfg &c) { return c.R == 8 ? 8 : 4; }
// The W32 family loads its second-core slice into registers as 32x32x16 A fragments. Its chain
// stores Sk in that fragment order (one contiguous 1 KB piece per wave load instead of 32
// rows x 32 bytes: measured 15.4 -> 12.6 us at rank 16, T=32), when the slice starts on a
// 32-row tile: the workgroup owns every s, or s-chunks of whole tiles.
constexpr bool s_frag(const KCfg &c) {
    const int oS = c.S == 0 ? c.o0 : c.S == 1 ? c.o1 : c.o2;
    return c.WIDE && c.MF2 == 32 && (c.SC == oS || c.SC * c.R % 32 == 0);
}
constexpr int l_group(const KCfg &c) { return c.R == 8 && !(c.WIDE && c.MF2 == 32) ? 8 : 4; }
// Bank conflicts of the stage-2 result stores: the largest number of lanes of a half-wave
// (32 lanes, the ones one LDS pass serves for 8-byte stores) that touch one of the 64 4-byte
// banks, for Vb planes `plane` elements apart. Lane addresses as the kernel computes them for
// the first tile (the others add a tile constant): 32x32 tiles (w32) store rows 0..3 of
// column lane; 16x16 tiles store rows 4 * (lane / 16) .. + 3 of column lane % 16.
constexpr int vb_store_degree(bool w32, int Q, int R, int LG, int P3, int plane) {
    int hits[64] = {};
    for (int lane = 0; lane < 32; ++lane) {
        const int m = w32 ? 0 : 4 * (lane / 16), n = w32 ? lane : lane % 16;
        const int r3 = m % R, q = n / Q;
        const int el = (m / R) * P3 + r3 / LG * LG * R + r3 % LG + (n % Q) * plane +
                       q / R * R * R + q % R * LG;
        const int bank = el * 2 / 4 % 64;
        ++hits[bank];
        ++hits[(bank + 1) % 64];
    }
    int worst = 0;
    for (int b = 0; b < 64; ++b) worst = hits[b] > worst ? hits[b] : worst;
    return worst;
}
// Bank conflicts of the stage-3 A-fragment reads of Vb (16x16x32 fragments): the largest
// number of the first 32 lanes that read one 16-byte unit modulo 512 bytes, over every 16-row
// tile, with rows (t, f, s) at (row / SC) * plane + (row % SC) * P3.
constexpr int vb_read_degree(int M3T, int SC, int P3, int plane) {
    int worst = 0;
    for (int mt = 0; mt < M3T; ++mt) {
        int hits[32] = {};
        for (int lane = 0; lane < 32; ++lane) {
            const int m3 = mt * 16 + lane % 16;
            const int el = m3 / SC * plane + m3 % SC * P3;
            const int u = (el / 8 + lane / 16) % 32;
            worst = ++hits[u] > worst ? hits[u] : worst;
        }
    }
    return worst;
}
// Vb layout: row pitch p3 (the 16x16 pitch p3a or K3 + 8) and plane pitch SC * p3 + pad (pad a
// multiple of 8 elements below 128, so rows stay 16-byte aligned), chosen to minimise the
// bank conflicts of the stage-2 stores and the stage-3 reads, a conflicted store counting five
// times a conflicted read (measured on gfx950: conflict-free 8-byte stores run at about a
// third of the read bandwidth, and a conflicted store takes 2.6x a clean one). Returns
// p3 * 256 + pad.
constexpr int vb_layout(bool w32, int Q, int R, int LG, int K3, int p3a, int SC, int M3T) {
    int best = p3a * 256, cost = 1 << 30;
    for (int c = 0; c < 2; ++c) {
        const int p3 = c == 0 ? p3a : K3 + 8;
        if (c == 1 && p3 == p3a) break;
        for (int pad = 0; pad < 128; pad += 8) {
            const int plane = SC * p3 + pad;
            const int k = 5 * vb_store_degree(w32, Q, R, LG, p3, plane) +
                          vb_read_degree(M3T, SC, p3, plane);
            if (k < cost) best = p3 * 256 + pad, cost = k;
        }
    }
    return best;
}

// LDS row pitches (elements; K a multiple of 16). Measured on gfx950, a ds_read_b128 serves
// 32 lanes per pass from 128 banks, so a fragment read is conflict free when those 32 lanes
// touch 32 distinct 16-byte units modulo 512 bytes. A 32x32x16 fragment (32 rows, then the
// same rows 16 bytes on) needs an odd pitch in 16-byte units; a 16x16x32 fragment (16 rows,
// then the same rows 16 bytes on) needs a pitch of 2 modulo 4 units, whose 16 rows take the
// even units and leave the odd ones to the second lane group.
constexpr int pitch16(int K) { return K + 8 * ((6 - K / 8 % 4) % 4); }
constexpr int pitch32(int K) { return K + 8; }

// Elements of Vb: rows 0 .. M3P-1 at (row / SC) * plane + (row % SC) * P3, each P3 long.
constexpr int vb_elems(int M3P, int SC, int P3, int plane) {
    return (M3P - 1) / SC * plane + ((M3P - 1) % SC + 1) * P3;
}

// Elements of a tile's LDS buffers for row pitches pf, p2, p3, pl (Vb planes unpadded).
constexpr int lds_elems(bool wide, int M1, int M2P, int ls_rows, int N1P, int N2R, int M3P,
                        int SC, int NBUF, int NBUF2, int pf, int p2, int p3, int pl) {
    return (wide ? 16 : M1 * pf + M2P * p2) + NBUF * (ls_rows * pl + N1P * pf) +
           NBUF2 * (N2R * p2 + vb_elems(M3P, SC, p3, SC * p3));
}

template <KCfg C>
struct Geo {
    static constexpr int R = C.R, R2 = R * R;
    static constexpr int nF = pick(C.F, C.i0, C.i1, C.i2);
    static constexpr int nS = pick(C.S, C.i0, C.i1, C.i2);
    static constexpr int nL = pick(C.L, C.i0, C.i1, C.i2);
    static constexpr int oF = pick(C.F, C.o0, C.o1, C.o2);
    static constexpr int oS = pick(C.S, C.o0, C.o1, C.o2);
    static constexpr int oL = pick(C.L, C.o0, C.o1, C.o2);
    static constexpr int IN = C.i0 * C.i1 * C.i2, OUT = C.o0 * C.o1 * C.o2;
    static constexpr int SXF = pick(C.F, C.i1 * C.i2, C.i2, 1);
    static constexpr int SXS = pick(C.S, C.i1 * C.i2, C.i2, 1);
    static constexpr int SXL = pick(C.L, C.i1 * C.i2, C.i2, 1);
    static constexpr int SYF = pick(C.F, C.o1 * C.o2, C.o2, 1);
    static constexpr int SYS = pick(C.S, C.o1 * C.o2, C.o2, 1);
    static constexpr int SYL = pick(C.L, C.o1 * C.o2, C.o2, 1);
    static constexpr int KF = rup(nF, 16), K2 = rup(nS * R, 16);
    // element bytes, and elements per 16-byte vector (the unit of the global <-> LDS copies)
    static constexpr int EB = C.dt == TRK_DTYPE_F32 ? 4 : 2, VPE = 16 / EB;
    static constexpr int TT = C.TT, FC = C.FC, SC = C.SC, LC = C.LC, IC = C.IC, KS3 = C.KS3;
    static constexpr int NACC = C.NACC;
    static constexpr bool WIDE = C.WIDE != 0;
    // stage 1: A = Fs [M1][KF], B = Xs [N1][KF]. The B rows are (iL', t, iS) with iS padded
    // to nSP, a multiple of 16, so that every 16-row tile has one (iL', t) and its stores
    // go to a per-tile constant plus a per-lane constant offset.
    static constexpr int nSP = rup(nS, 16);
    static constexpr int M1 = FC * R2, M1T = M1 / 16;
    static constexpr int N1 = IC * TT * nSP, N1T = N1 / 16, N1P = N1;
    // stage 2: A = Ss [M2P][K2], B = Ub [N2P][K2]
    static constexpr int M2 = SC * R, M2T = cdiv(M2, 16), M2P = M2T * 16;
    static constexpr int N2 = IC * R * TT * FC, N2T = cdiv(N2, 16), N2P = N2T * 16;
    // stage 3: A = Vb [M3P][K3], B = Ls [IC][LCP][R2]
    static constexpr int M3 = TT * FC * SC, M3T = cdiv(M3, 16), M3P = M3T * 16;
    static constexpr int N3T = cdiv(LC, 16), LCP = N3T * 16;
    static constexpr int K3 = IC * R2;
    static constexpr int NW = C.NW, NT = 64 * NW;  // waves and threads per workgroup
    static constexpr int NT3 = M3T * N3T, G3 = NW / KS3, NYW = cdiv(NT3, G3);
    static constexpr int NSTEP = cdiv(nL, IC);
    static constexpr int NFC = cdiv(oF, FC), NSC = cdiv(oS, SC), NLC = cdiv(oL, LC);
    static constexpr int NBLK = NFC * NSC * NLC;  // workgroups per token tile
    // WIDE: each wave holds the A fragments of BM1 stage-1 and BM2 stage-2 row tiles; stage 2
    // runs on a WM2 x WN2 grid of waves (rows x columns)
    static constexpr int WM2 = WIDE ? C.WIDE : NW, WN2 = NW / WM2;
    static constexpr bool W32 = WIDE && C.MF2 == 32;  // stage 2 on 32x32 tiles
    static constexpr int M2T32 = cdiv(M2, 32), N2T32 = cdiv(N2, 32);
    // WIDE stage 1 on a WM1 x WN1 grid of waves (row groups of BM1 tiles x column phases).
    // By default every wave takes its own rows and all columns, or, with fewer row tiles than
    // waves, one row tile and a share of the columns (no wave idles); S1 sets larger row
    // groups, which read the x slice from LDS fewer times at the cost of registers.
    static constexpr int BM1 = C.S1 ? C.S1 : M1T < NW && NW % M1T == 0 ? 1 : cdiv(M1T, NW);
    static constexpr int WM1 = C.S1 || (M1T < NW && NW % M1T == 0) ? M1T / BM1 : NW;
    static constexpr int WN1 = NW / WM1;
    static constexpr int BM2 = cdiv(W32 ? M2T32 : M2T, WM2);
    static constexpr int N2R = W32 ? N2T32 * 32 : N2P;  // Ub rows (the last tile's padding)
    // W32 with one row tile per wave and fewer row tiles than waves (8): waves 0-3 take a row
    // tile each and waves 4-7 split the TAILR remaining row tiles' columns TAILJ ways. Waves
    // w and w+4 share a SIMD, so every SIMD gets nearly equal stage-2 work (for 5 row tiles:
    // 5 tile columns' worth on each SIMD instead of 8 on one).
    static constexpr int TAILR = M2T32 - NW / 2;
    static constexpr bool TAIL = W32 && WN2 == 1 && BM2 == 1 && NW == 8 && TAILR > 0 &&
                                 M2T32 < NW && (NW / 2) % TAILR == 0;
    static constexpr int TAILJ = TAIL ? (NW / 2) / TAILR : 1;
    static_assert(C.TP == 0 || (C.TP == 1 && TAIL), "TP needs the pair-and-tail stage 2");
    static constexpr int NBUF = C.PIPE ? 2 : 1;  // buffers of the per-step slices
    static constexpr int NBUF2 = C.PIPE == 2 ? 2 : 1;  // buffers of the stage results
    // LDS row pitches for the fragment shape each buffer is read with (Ub by 32x32x16 MFMAs in
    // the W32 family, everything else by 16x16x32 or 16x16x16 MFMAs) where the tile still fits
    // in LDS with them; otherwise 16 bytes past each K extent (conflict free for 32x32 reads)
    static constexpr bool CFP =
        lds_elems(WIDE, M1, M2P, IC * LCP, N1P, N2R, M3P, SC, NBUF, NBUF2, pitch16(KF),
                  W32 ? pitch32(K2) : pitch16(K2), pitch16(K3), pitch16(R2)) * EB <= 160 * 1024;
    static constexpr int PF = CFP ? pitch16(KF) : KF + 8;
    static constexpr int P2 = W32 ? pitch32(K2) : CFP ? pitch16(K2) : K2 + 8;
    static constexpr int PL = CFP ? pitch16(R2) : R2 + 8;
    // LDS layout, in elements
    static constexpr int oFs = 0, szFs = WIDE ? 8 : M1 * PF;
    static constexpr int oSs = oFs + szFs, szSs = WIDE ? 8 : M2P * P2;
    static constexpr int oLs = oSs + szSs, szLs = IC * LCP * PL;
    static constexpr int oXs = oLs + NBUF * szLs, szXs = N1P * PF;
    static constexpr int oUb = oXs + NBUF * szXs, szUb = N2R * P2;
    // Vb rows (t, f, s): planes of SC rows per (t, f), PLANE elements apart, rows P3 apart
    // (the layout with the fewest bank conflicts, its plane padding only where it fits in LDS)
    static constexpr int SG = s_group(C), LG = l_group(C), Q = TT * FC;
    static constexpr int oVb = oUb + NBUF2 * szUb;
    static constexpr int VBL = vb_layout(W32, Q, R, LG, K3, CFP ? pitch16(K3) : K3 + 8, SC, M3T);
    static constexpr int P3 = VBL / 256, PLANE_PAD = SC * P3 + VBL % 256;
    static constexpr int PLANE =
        (oVb + NBUF2 * vb_elems(M3P, SC, P3, PLANE_PAD)) * EB <= 160 * 1024 ? PLANE_PAD : SC * P3;
    static constexpr int szVb = vb_elems(M3P, SC, P3, PLANE);
    static constexpr int LDS_ELEMS = oVb + NBUF2 * szVb;
    static constexpr int LDS_BYTES = LDS_ELEMS * EB;
    static constexpr int RED_FLOATS = (KS3 - 1) * G3 * NYW * 256;
    // x loader. Contiguous iF: VX-element vectors straight into Xs rows. Otherwise: 16-byte
    // vectors (VPE elements) of the natural x row, scattered element by element, in batches of
    // XB per thread.
    static constexpr bool XROW = SXF == 1;
    static constexpr int vx_fits(int v) {
        return nF % v == 0 && SXS % v == 0 && SXL % v == 0 && IN % v == 0;
    }
    static constexpr int VX = !XROW                     ? 1
                              : VPE >= 8 && vx_fits(8) ? 8
                              : vx_fits(4)             ? 4
                              : vx_fits(2)             ? 2
                                                       : 1;
    static constexpr int XCPR = KF / VX;                      // vectors per Xs row (contiguous iF)
    static constexpr int NXV = N1 * XCPR;                     // vectors per step (contiguous iF)
    static constexpr int NXB = TT * IN / VPE;                 // vectors per step (scatter)
    static constexpr int XB = 8;

    static_assert(R % 8 == 0 && (R & (R - 1)) == 0, "MFMA variants need a power-of-two rank >= 8");
    static_assert(NW == 4 || NW == 8, "4 or 8 waves per workgroup");
    static_assert(C.XL == 0 || C.XL == 1 || C.XL == 2 || C.XL == 4, "XL is 0, 1, 2 or 4");
    static_assert(C.XL == 0 || NBLK % C.XL == 0, "XL must divide the workgroups of a token tile");
    static_assert(C.YM == 0 || (C.YM == 1 && C.XL == 0), "YM is 0, or 1 on all 8 XCDs");
    static_assert(C.SL == 0 || C.SL == 1, "SL is 0 or 1");
    static_assert(C.WIDE >= 0 && C.WIDE <= NW && (C.WIDE == 0 || NW % C.WIDE == 0),
                  "WIDE is 0 or divides the waves");
    static_assert(C.MF2 == 16 || (C.MF2 == 32 && WIDE), "MF2 is 16, or 32 with WIDE");
    static_assert(W32 || 16 % (FC * TT) == 0,
                  "FC * TT must divide 16 (stage-2 store offsets of 16x16 tiles)");
    static_assert(KS3 >= 1 && NW % KS3 == 0, "KS3 must divide the waves");
    static_assert(NACC >= 1 && (K3 / 32 / KS3) % NACC == 0, "NACC must divide a wave's K steps");
    static_assert(FC <= oF && SC <= oS && LC <= oL && IC <= nL && TT >= 1, "tile too large");
    static_assert(LDS_BYTES <= 160 * 1024, "workgroup tile exceeds the 160 KB of LDS");
    static_assert(RED_FLOATS * 4 <= szUb * EB, "stage-3 reduction does not fit in Ub");
    static_assert(nL % IC == 0, "IC must divide the last core's input mode");
    static_assert(R % SG == 0 && R % LG == 0 && SG % 4 == 0 && LG % 4 == 0,
                  "K-order groups must hold whole 4-element stores");
    static_assert(C.PIPE >= 0 && C.PIPE <= 2 && (C.PIPE == 0 || NSTEP > 1),
                  "a pipelined tile needs two steps");
    static_assert(XROW || IN % VPE == 0, "scatter loader reads x rows in 16-byte vectors");
    static_assert(C.S1 == 0 || (WIDE && M1T % C.S1 == 0 && NW % (M1T / C.S1) == 0),
                  "S1 must split the stage-1 rows into a divisor of the waves");
};


// LDS <- global through VGPRs for NB blocks of BLOCK 16-byte vectors, spread over the NT
// threads of a workgroup: block b is read from src + b * stride (vectors), its first `valid`
// vectors from memory and the rest zero. issue() starts every read of the copy; commit()
// writes the LDS as rows of ROW vectors at a pitch of PITCH vectors (the compiler waits for
// exactly the loads whose registers it stores).
template <int NB, int BLOCK, int ROW, int NT, int PITCH>
struct RegCopy {
    static_assert(BLOCK % ROW == 0, "a copy block holds whole LDS rows");
    static constexpr int TOTAL = NB * BLOCK, PER = cdiv(TOTAL, NT);
    uint4 r[PER];
    __device__ __forceinline__ void issue(const void *src, size_t stride, int valid) {
        const uint4 *s = static_cast<const uint4 *>(src);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = threadIdx.x + j * NT, b = i / BLOCK, w = i % BLOCK;
            r[j] = make_uint4(0u, 0u, 0u, 0u);
            if ((TOTAL % NT == 0 || i < TOTAL) && w < valid) r[j] = s[b * stride + w];
        }
    }
    __device__ __forceinline__ void commit(void *dst) const {
        uint4 *d = static_cast<uint4 *>(dst);
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int i = threadIdx.x + j * NT;
            if (TOTAL % NT == 0 || i < TOTAL) d[i / ROW * PITCH + i % ROW] = r[j];
        }
    }
};

template <int BYTES>
struct VecOf;
template <>
struct VecOf<16> { using T = uint4; };
template <>
struct VecOf<8> { using T = uint2; };
template <>
struct VecOf<4> { using T = unsigned int; };
template <>
struct VecOf<2> { using T = unsigned short; };

// Register blocking of one LDS GEMM stage with MT x NT output tiles of 16x16 and KS K
// steps: blocks of BM x BN tiles go round-robin to the 4 waves; per K step a wave reads BM
// A fragments and BN B fragments from LDS and runs BM*BN MFMAs on them. The choice weighs
// a wave's MFMA issue time against its LDS fragment traffic, with at most 16 accumulator
// tiles per wave.
struct Blocking {
    int bm, bn;
};
constexpr Blocking choose_blocking(int MT, int NT, int KS, int NW) {
    Blocking best{1, 1};
    long best_cost = -1;
    for (int bm = 1; bm <= 4; ++bm)
        for (int bn = 1; bn <= 8; ++bn) {
            if (bm * bn > 16 || bm > MT || bn > NT) continue;
            const int blocks = cdiv(MT, bm) * cdiv(NT, bn);
            const long per_wave = cdiv(blocks, NW);
            const long cost = per_wave * KS * (16L * bm * bn + 12L * (bm + bn)) + per_wave * 40;
            if (best_cost < 0 || cost < best_cost) {
                best_cost = cost;
                best = Blocking{bm, bn};
            }
        }
    return best;
}

// One LDS GEMM stage: D[MT*16][NT*16] = A[.][K] . B[.][K]^T (rows K-contiguous, pitch P),
// register-blocked as above; each finished tile goes to st(mt, nt, d).
template <class O, int MT, int NT, int K, int P, int NW, class Store>
__device__ __forceinline__ void lds_gemm(const typename O::E *A, const typename O::E *B, int wave,
                                         int lrow, int lgrp, Store &&st) {
    using V8 = typename O::V8;
    using V4 = typename O::V4;
    constexpr int K32 = K / 32, K16 = (K % 32) / 16;
    constexpr Blocking BK = choose_blocking(MT, NT, K32 + K16, NW);
    constexpr int BM = BK.bm, BN = BK.bn, NBM = cdiv(MT, BM), NBN = cdiv(NT, BN);
    constexpr int BLOCKS = NBM * NBN;
#pragma unroll
    for (int j = 0; j < cdiv(BLOCKS, NW); ++j) {
        const int blk = wave + NW * j;
        if (BLOCKS % NW != 0 && blk >= BLOCKS) break;
        const int m0 = (blk / NBN) * BM, n0 = (blk % NBN) * BN;
        const typename O::E *a = A + (m0 * 16 + lrow) * P;
        const typename O::E *b = B + (n0 * 16 + lrow) * P;
        Acc<(K32 > 0 ? 32 : 16)> d[BM][BN];
#pragma unroll
        for (int i = 0; i < BM; ++i)
#pragma unroll
            for (int q = 0; q < BN; ++q) d[i][q].v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        if constexpr (K32 > 0) {
#pragma unroll
            for (int k = 0; k < K32; ++k) {
                V8 af[BM], bf[BN];
#pragma unroll
                for (int i = 0; i < BM; ++i)
                    af[i] = (MT % BM == 0 || m0 + i < MT)
                                ? *reinterpret_cast<const V8 *>(a + i * 16 * P + 32 * k + 8 * lgrp)
                                : V8{};
#pragma unroll
                for (int q = 0; q < BN; ++q)
                    bf[q] = (NT % BN == 0 || n0 + q < NT)
                                ? *reinterpret_cast<const V8 *>(b + q * 16 * P + 32 * k + 8 * lgrp)
                                : V8{};
#pragma unroll
                for (int i = 0; i < BM; ++i)
#pragma unroll
                    for (int q = 0; q < BN; ++q) d[i][q] = O::k32(af[i], bf[q], d[i][q]);
            }
        }
        if constexpr (K16 && K32 > 0) {
            // trailing 16 of K after 32-wide steps: one more 16x16x32 MFMA whose upper K half
            // (lanes 32-63) is zero, so the accumulation chain never mixes MFMA shapes (a
            // 16x16x16 MFMA reading the accumulator of a 16x16x32 one back to back has given
            // wrong sums on gfx950)
            V8 af[BM], bf[BN];
            const int kt = K - 16 + 8 * (lgrp & 1);  // stays inside the row for every lane
#pragma unroll
            for (int i = 0; i < BM; ++i)
                af[i] = (lgrp < 2 && (MT % BM == 0 || m0 + i < MT))
                            ? *reinterpret_cast<const V8 *>(a + i * 16 * P + kt)
                            : V8{};
#pragma unroll
            for (int q = 0; q < BN; ++q)
                bf[q] = (lgrp < 2 && (NT % BN == 0 || n0 + q < NT))
                            ? *reinterpret_cast<const V8 *>(b + q * 16 * P + kt)
                            : V8{};
#pragma unroll
            for (int i = 0; i < BM; ++i)
#pragma unroll
                for (int q = 0; q < BN; ++q) d[i][q] = O::k32(af[i], bf[q], d[i][q]);
        } else if constexpr (K16) {  // K of 16 alone: one 16x16x16 MFMA per tile
            V4 af[BM], bf[BN];
#pragma unroll
            for (int i = 0; i < BM; ++i)
                af[i] = (MT % BM == 0 || m0 + i < MT)
                            ? *reinterpret_cast<const V4 *>(a + i * 16 * P + K - 16 + 4 * lgrp)
                            : V4{};
#pragma unroll
            for (int q = 0; q < BN; ++q)
                bf[q] = (NT % BN == 0 || n0 + q < NT)
                            ? *reinterpret_cast<const V4 *>(b + q * 16 * P + K - 16 + 4 * lgrp)
                            : V4{};
#pragma unroll
            for (int i = 0; i < BM; ++i)
#pragma unroll
                for (int q = 0; q < BN; ++q) d[i][q] = O::k16(af[i], bf[q], d[i][q]);
        }
#pragma unroll
        for (int i = 0; i < BM; ++i)
#pragma unroll
            for (int q = 0; q < BN; ++q)
                if ((MT % BM == 0 || m0 + i < MT) && (NT % BN == 0 || n0 + q < NT))
                    st(m0 + i, n0 + q, d[i][q].v);
    }
}

// A operand held in registers: the fragments of BMW 16-row tiles (rows row0 + i*16 + lane
// row) over a K range of K, read once from a K-contiguous global matrix (rows at or past
// `rows` read as zero). Used by the WIDE variants for the first- and second-core slices.
template <class O, int BMW, int K>
struct RegA {
    static constexpr int K32 = K / 32, K16 = (K % 32) / 16;
    typename O::V8 a8[BMW][K32 > 0 ? K32 : 1];
    typename O::V4 a4[BMW];  // a K of 16 alone (16x16x16 fragments)
    typename O::V8 t8[BMW];  // a trailing 16 after 32-wide steps, upper K half zero
    __device__ __forceinline__ void load(const typename O::E *__restrict__ src, int row0, int rows,
                                         int lrow, int lgrp) {
#pragma unroll
        for (int i = 0; i < BMW; ++i) {
            const int row = row0 + i * 16 + lrow;
            const typename O::E *p = src + size_t(row) * K;
#pragma unroll
            for (int k = 0; k < K32; ++k)
                a8[i][k] = row < rows ? *reinterpret_cast<const typename O::V8 *>(p + 32 * k + 8 * lgrp)
                                      : typename O::V8{};
            if constexpr (K16 && K32 > 0)
                t8[i] = row < rows && lgrp < 2
                            ? *reinterpret_cast<const typename O::V8 *>(p + K - 16 + 8 * (lgrp & 1))
                            : typename O::V8{};
            else if constexpr (K16)
                a4[i] = row < rows ? *reinterpret_cast<const typename O::V4 *>(p + K - 16 + 4 * lgrp)
                                   : typename O::V4{};
        }
    }
};

// One LDS GEMM stage with the A operand in registers (RegA, this wave's BMW row tiles) over
// the column tiles nt = wn, wn + WN, ... below NT. They go in blocks of BN; per K step the
// wave runs BMW x BN independent MFMAs on the block's BN B fragments (LDS rows of pitch P)
// while the fragments of the next K step are already being read (two register buffers,
// kept in that order by scheduling barriers). Each finished column tile goes to
// st(nt, d[BMW]).
template <class O, int BMW, int K, int P, int NT, int WN, class Store>
__device__ __forceinline__ void reg_gemm(const RegA<O, BMW, K> &A, const typename O::E *B, int wn,
                                         int lrow, int lgrp, Store &&st) {
    using V8 = typename O::V8;
    using V4 = typename O::V4;
    constexpr int K32 = K / 32, K16 = (K % 32) / 16;
    constexpr int NTW = cdiv(NT, WN);                     // column tiles per wave (at most)
    constexpr int BN0 = 16 / BMW < 1 ? 1 : 16 / BMW;      // at most 16 accumulator tiles
    constexpr int BN = BN0 < NTW ? BN0 : NTW;
#pragma unroll
    for (int j0 = 0; j0 < NTW; j0 += BN) {
        // column tile q of the block is nt = wn + WN * (j0 + q); absent when nt >= NT
        auto have = [&](int q) { return j0 + q < NTW && (NT % WN == 0 || wn + WN * (j0 + q) < NT); };
        const typename O::E *b = B + ((wn + WN * j0) * 16 + lrow) * P;
        auto frag8 = [&](int q, int k) {
            return *reinterpret_cast<const V8 *>(b + q * WN * 16 * P + 32 * k + 8 * lgrp);
        };
        Acc<(K32 > 0 ? 32 : 16)> d[BN][BMW];
#pragma unroll
        for (int q = 0; q < BN; ++q)
#pragma unroll
            for (int i = 0; i < BMW; ++i) d[q][i].v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        V8 cur[BN], nxt[BN];
        if constexpr (K32 > 0) {
#pragma unroll
            for (int q = 0; q < BN; ++q)
                if (have(q)) cur[q] = frag8(q, 0);
        }
        if constexpr (K32 > 0) {
#pragma unroll
            for (int k = 0; k < K32; ++k) {
                if (k + 1 < K32) {
#pragma unroll
                    for (int q = 0; q < BN; ++q)
                        if (have(q)) nxt[q] = frag8(q, k + 1);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < BN; ++q)
                    if (have(q))
#pragma unroll
                        for (int i = 0; i < BMW; ++i)
                            d[q][i] = O::k32(A.a8[i][k], cur[q], d[q][i]);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int q = 0; q < BN; ++q) cur[q] = nxt[q];
            }
        }
        if constexpr (K16 && K32 > 0) {
            // trailing 16 of K: a 16x16x32 MFMA with the upper K half zero, so that the
            // accumulation chain keeps one MFMA shape (as in lds_gemm)
            V8 bf[BN];
#pragma unroll
            for (int q = 0; q < BN; ++q)
                bf[q] = have(q) && lgrp < 2 ? *reinterpret_cast<const V8 *>(
                                                  b + q * WN * 16 * P + K - 16 + 8 * (lgrp & 1))
                                            : V8{};
#pragma unroll
            for (int q = 0; q < BN; ++q)
                if (have(q))
#pragma unroll
                    for (int i = 0; i < BMW; ++i) d[q][i] = O::k32(A.t8[i], bf[q], d[q][i]);
        } else if constexpr (K16) {
            V4 bf[BN];
#pragma unroll
            for (int q = 0; q < BN; ++q)
                if (have(q))
                    bf[q] = *reinterpret_cast<const V4 *>(b + q * WN * 16 * P + K - 16 + 4 * lgrp);
#pragma unroll
            for (int q = 0; q < BN; ++q)
                if (have(q))
#pragma unroll
                    for (int i = 0; i < BMW; ++i) d[q][i] = O::k16(A.a4[i], bf[q], d[q][i]);
        }
#pragma unroll
        for (int q = 0; q < BN; ++q)
            if (have(q)) {
                f32x4 out[BMW];
#pragma unroll
                for (int i = 0; i < BMW; ++i) out[i] = d[q][i].v;
                st(wn + WN * (j0 + q), out);
            }
    }
}

// A operand of 32x32x16 MFMAs held in registers: BMW 32-row tiles (rows row0 + i*32 + lane%32)
// over K (a multiple of 16), lane holding K elements 16*s + 8*(lane/32) .. +8 of its row for
// each K step s, read once from a K-contiguous global matrix (rows at or past `rows` zero).
template <class O, int BMW, int K>
struct RegA32 {
    static_assert(K % 16 == 0, "32x32x16 fragments need K a multiple of 16");
    typename O::V8 a[BMW][K / 16];
    __device__ __forceinline__ void load(const typename O::E *__restrict__ src, int row0, int rows,
                                         int lane) {
#pragma unroll
        for (int i = 0; i < BMW; ++i) {
            const int row = row0 + i * 32 + (lane & 31);
            const typename O::E *p = src + size_t(row) * K + 8 * (lane >> 5);
#pragma unroll
            for (int k = 0; k < K / 16; ++k)
                a[i][k] = row < rows ? *reinterpret_cast<const typename O::V8 *>(p + 16 * k)
                                     : typename O::V8{};
        }
    }
    // The same fragments from a matrix stored in fragment order ([tile][k step][lane][8], see
    // trk_pack.hip); row0 is a multiple of 32, so tile i starts at (row0 + 32 i) * K.
    __device__ __forceinline__ void load_frag(const typename O::E *__restrict__ src, int row0,
                                              int rows, int lane) {
#pragma unroll
        for (int i = 0; i < BMW; ++i) {
            const int row = row0 + i * 32 + (lane & 31);
            const typename O::E *p = src + size_t(row0 + i * 32) * K + 8 * lane;
#pragma unroll
            for (int k = 0; k < K / 16; ++k)
                a[i][k] = row < rows ? *reinterpret_cast<const typename O::V8 *>(p + 512 * k)
                                     : typename O::V8{};
        }
    }
};

// reg_gemm on 32x32 tiles: A in registers (RegA32, BMW row tiles), the column tiles
// nt = wn, wn + WN, ... below NT (32 columns each) in blocks of BN, B fragments read from
// LDS rows of pitch P (lane: row nt*32 + lane%32, K elements 16*s + 8*(lane/32) .. +8), the
// next K step's fragments read while this step's MFMAs run. st(nt, d[BMW]) gets each
// finished column tile; d[i][4*g + e] is row 8*g + 4*(lane/32) + e, column lane%32.
template <class O, int BMW, int K, int P, int NT, int WN, class Store>
__device__ __forceinline__ void reg_gemm32(const RegA32<O, BMW, K> &A, const typename O::E *B,
                                           int wn, int lane, Store &&st) {
    using V8 = typename O::V8;
    constexpr int KS = K / 16;
    constexpr int NTW = cdiv(NT, WN);
    constexpr int BN0 = 4 / BMW < 1 ? 1 : 4 / BMW;  // at most 4 accumulator tiles (64 VGPRs)
    constexpr int BN = BN0 < NTW ? BN0 : NTW;
#pragma unroll
    for (int j0 = 0; j0 < NTW; j0 += BN) {
        auto have = [&](int q) { return j0 + q < NTW && (NT % WN == 0 || wn + WN * (j0 + q) < NT); };
        const typename O::E *b = B + ((wn + WN * j0) * 32 + (lane & 31)) * P + 8 * (lane >> 5);
        auto frag = [&](int q, int k) {
            return *reinterpret_cast<const V8 *>(b + q * WN * 32 * P + 16 * k);
        };
        f32x16 d[BN][BMW];
#pragma unroll
        for (int q = 0; q < BN; ++q)
#pragma unroll
            for (int i = 0; i < BMW; ++i)
#pragma unroll
                for (int e = 0; e < 16; ++e) d[q][i][e] = 0.0f;
        V8 cur[BN], nxt[BN];
#pragma unroll
        for (int q = 0; q < BN; ++q)
            if (have(q)) cur[q] = frag(q, 0);
#pragma unroll
        for (int k = 0; k < KS; ++k) {
            if (k + 1 < KS) {
#pragma unroll
                for (int q = 0; q < BN; ++q)
                    if (have(q)) nxt[q] = frag(q, k + 1);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < BN; ++q)
                if (have(q))
#pragma unroll
                    for (int i = 0; i < BMW; ++i) d[q][i] = O::w16(A.a[i][k], cur[q], d[q][i]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int q = 0; q < BN; ++q) cur[q] = nxt[q];
        }
#pragma unroll
        for (int q = 0; q < BN; ++q)
            if (have(q)) st(wn + WN * (j0 + q), d[q]);
    }
}

// Hook of ring3_unit for callers without one (the standalone kernel).
struct NoHook {
    __device__ void operator()() const {}
};

// One workgroup's unit of work: the tile b (f, s and l chunks, in the order of NBLK) of token
// tile tile_y, on the LDS buffers the caller declares (each buffer its own object where the
// caller can, so that the compiler sees they never alias). Every thread of the workgroup
// calls it. The standalone kernel below calls it once per workgroup; a persistent caller may
// call it for several units and layers, with a barrier (__syncthreads) between units.
// hook, when given, is called by every thread once the unit's core-slice loads are in flight
// (with SL, the second-core slice's come after the first commit, past the hook)
// and before any load of x, which is then issued after it: a persistent caller's wait for the
// layer that writes x (the core slices do not depend on it). Without a hook the loads keep
// the standalone order. COHERENT_X reads x with device-scope loads, which the CU's L1 does not
// serve: for x written earlier in the same launch by workgroups on other CUs (a persistent
// caller), whose lines an older read may have left in this CU's L1.
// Sections of the packed cores one pass of ring3_unit reads.
template <class E>
struct CoreSections {
    const E *fk, *sk, *lk;
};

// A load of `T` (4, 8 or 16 bytes) at device scope: relaxed atomic loads of its 4- or 8-byte
// words (the memory model's device-scope load, which does not use the CU's L1).
template <class T>
__device__ __forceinline__ T load_device_scope(const T *p) {
    static_assert(sizeof(T) % 4 == 0 && sizeof(T) <= 16, "4-, 8- or 16-byte loads");
    T r;
    if constexpr (sizeof(T) % 8 == 0) {
        auto *src = reinterpret_cast<const unsigned long long *>(p);
        auto *dst = reinterpret_cast<unsigned long long *>(&r);
#pragma unroll
        for (int i = 0; i < int(sizeof(T) / 8); ++i)
            dst[i] = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        auto *src = reinterpret_cast<const unsigned *>(p);
        auto *dst = reinterpret_cast<unsigned *>(&r);
#pragma unroll
        for (int i = 0; i < int(sizeof(T) / 4); ++i)
            dst[i] = __hip_atomic_load(src + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return r;
}

template <KCfg C, bool EPI, class Hook = NoHook, bool PAIR = false, bool COHERENT_X = false>
__device__ __forceinline__ void ring3_unit(const typename Ops<C.dt>::E *__restrict__ x,
                                           const typename Ops<C.dt>::E *__restrict__ Fk0,
                                           const typename Ops<C.dt>::E *__restrict__ Sk0,
                                           const typename Ops<C.dt>::E *__restrict__ Lk0, void *y,
                                           int T, int epi_mode, const void *aux, int b, int tile_y,
                                           typename Ops<C.dt>::E *__restrict__ Fs,
                                           typename Ops<C.dt>::E *__restrict__ Ss,
                                           typename Ops<C.dt>::E *__restrict__ Ls,
                                           typename Ops<C.dt>::E *__restrict__ Xs,
                                           typename Ops<C.dt>::E *__restrict__ Ub,
                                           typename Ops<C.dt>::E *__restrict__ Vb,
                                           Hook &&hook = Hook{},
                                           CoreSections<typename Ops<C.dt>::E> second = {}) {
    constexpr bool HOOKED = !std::is_same_v<std::decay_t<Hook>, NoHook>;
    using G = Geo<C>;
    using O = Ops<C.dt>;
    using E = typename O::E;
    using E4 = typename O::E4;
    constexpr int R = G::R, R2 = G::R2;
    // the sections the current pass reads: the operator's, then (PAIR) the second one's
    const E *__restrict__ Fk = Fk0;
    const E *__restrict__ Sk = Sk0;
    const E *__restrict__ Lk = Lk0;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lrow = lane & 15, lgrp = lane >> 4;

    const int l0 = (b % G::NLC) * G::LC;
    b /= G::NLC;
    const int s0 = (b % G::NSC) * G::SC;
    const int f0 = (b / G::NSC) * G::FC;
    const int t0 = tile_y * G::TT;
    // digits of each core this workgroup owns: compile-time constants when the chunks divide
    // the modes, which removes the bounds branches around the slice loads
    const int FCv = G::oF % G::FC == 0 ? G::FC : min(G::FC, G::oF - f0);
    const int SCv = G::oS % G::SC == 0 ? G::SC : min(G::SC, G::oS - s0);
    const int LCv = G::oL % G::LC == 0 ? G::LC : min(G::LC, G::oL - l0);

    // Global -> LDS for one step of IC last-core input digits: the last-core slice and x are
    // read into registers (issue), then written to Ls and Xs[(iL', t, iS)][iF] (commit).
    // Every global read of a step is in flight before the first wait.
    // Loader threads: all of them, or (pipelined tiles with the pair-and-tail stage 2) the
    // first half. There waves 4-7, which share SIMDs 0-3 with waves 0-3, finish their stage-2
    // tail about 500 clocks after waves 0-3 (measured): with the commit on waves 0-3 they go
    // from stage 2 straight to the barrier (3-4 % at 1920->2880 R16, T=32 and 128). On tiles
    // without the tail the same split measured 1-10 % slower.
    constexpr int LT = (C.PIPE == 1 && G::TAIL) ? G::NT / 2 : G::NT;
    const bool loader = LT == G::NT || tid < LT;
    using XV = typename VecOf<G::EB * G::VX>::T;
    constexpr int XPER = G::XROW ? cdiv(G::NXV, LT) : cdiv(G::NXB, LT);
    constexpr int XREG = G::XROW ? XPER : (XPER < G::XB ? XPER : G::XB);
    XV xr[G::XROW ? XREG : 1];
    uint4 xb[G::XROW ? 1 : XREG];
    // contiguous-iF loader: vector v of the step covers Xs[n][c*VX, c*VX+VX) of row
    // n = (iL', t, iS); what lies outside x (K padding, iS >= nS, absent tokens) is zero, so
    // these vectors write every element of Xs[:, 0:KF)
    auto x_row_load = [&](int v, int iL0) TRK_INLINE {
        const int n = v / G::XCPR, c = v % G::XCPR;
        const int iS = n % G::nSP, t = (n / G::nSP) % G::TT, iL = iL0 + n / (G::nSP * G::TT);
        XV r{};
        if ((G::NXV % LT == 0 || v < G::NXV) && c * G::VX < G::nF && iS < G::nS &&
            t0 + t < T) {
            const XV *p = reinterpret_cast<const XV *>(x + size_t(t0 + t) * G::IN + iS * G::SXS +
                                                       iL * G::SXL + c * G::VX);
            if constexpr (COHERENT_X)
                r = load_device_scope(p);
            else
                r = *p;
        }
        return r;
    };
    // scatter loader: one 16-byte x vector. Pipelined tiles load every vector, reading the
    // tile's first vector where v lies outside x (x_scatter_store skips those): there a zeroed
    // register with a masked load into it ran 1-4 % slower on the Llama-up tiles of 2-256
    // tokens. The other tiles keep the masked load, which measured 2-22 % faster for them.
    auto x_scatter_load = [&](int v) TRK_INLINE {
        const bool in_x = v < G::NXB && t0 + v / (G::IN / G::VPE) < T;
        const uint4 *row = reinterpret_cast<const uint4 *>(x + size_t(t0) * G::IN);
        uint4 r = make_uint4(0u, 0u, 0u, 0u);
        if constexpr (C.PIPE != 0) {
            if constexpr (COHERENT_X)
                r = load_device_scope(row + (in_x ? v : 0));
            else
                r = row[in_x ? v : 0];
        } else if (in_x) {
            if constexpr (COHERENT_X)
                r = load_device_scope(row + v);
            else
                r = row[v];
        }
        return r;
    };
    auto x_scatter_store = [&](int v, uint4 r, int iL0, E *xs) TRK_INLINE {
        const int t = v / (G::IN / G::VPE);
        if (v >= G::NXB || t0 + t >= T) return;
        const E *e = reinterpret_cast<const E *>(&r);
#pragma unroll
        for (int q = 0; q < G::VPE; ++q) {
            const int flat = (v % (G::IN / G::VPE)) * G::VPE + q;
            const int m0 = flat / (C.i1 * C.i2), m1 = (flat / C.i2) % C.i1, m2 = flat % C.i2;
            const int iF = pick(C.F, m0, m1, m2), iS = pick(C.S, m0, m1, m2);
            const int ilp = pick(C.L, m0, m1, m2) - iL0;
            if (ilp >= 0 && ilp < G::IC) xs[((ilp * G::TT + t) * G::nSP + iS) * G::PF + iF] = e[q];
        }
    };
    constexpr int VPE = G::VPE;
    RegCopy<1, G::WIDE ? 1 : G::M1 * G::KF / VPE, G::WIDE ? 1 : G::KF / VPE, G::NT, G::PF / VPE> cF;
    RegCopy<1, G::WIDE ? 1 : G::M2P * G::K2 / VPE, G::WIDE ? 1 : G::K2 / VPE, G::NT, G::P2 / VPE> cS;
    RegCopy<G::IC, G::LCP * R2 / VPE, R2 / VPE, LT, G::PL / VPE> cL;
    auto issue_l = [&](int iL0) TRK_INLINE {  // the last-core slice of the step at input digit iL0
        if (loader) cL.issue(Lk + (size_t(iL0) * G::oL + l0) * R2, size_t(G::oL) * R2 / VPE, LCv * R2 / VPE);
    };
    auto issue_x = [&](int iL0) TRK_INLINE {  // x for the step at input digit iL0
        if (!loader) return;
        if constexpr (G::XROW) {
#pragma unroll
            for (int j = 0; j < XREG; ++j) xr[j] = x_row_load(tid + j * LT, iL0);
        } else {
#pragma unroll
            for (int j = 0; j < XREG; ++j) xb[j] = x_scatter_load(tid + j * LT);
        }
    };
    auto issue_step = [&](int iL0) TRK_INLINE {
        issue_l(iL0);
        issue_x(iL0);
    };
    // The commits wait only for the loads whose registers they store: the compiler's
    // per-register wait counts (loads complete in issue order), so loads issued after them
    // (the register-resident slices in the prologue) stay in flight.
    auto commit_l = [&](int buf) TRK_INLINE {  // into buffer `buf` of Ls
        if (loader) cL.commit(Ls + buf * G::szLs);
    };
    auto commit_x = [&](int iL0, int buf) TRK_INLINE {  // into buffer `buf` of Xs
        E *xs = Xs + buf * G::szXs;
        if (!loader) return;
        if constexpr (G::XROW) {
#pragma unroll
            for (int j = 0; j < XREG; ++j) {
                const int v = tid + j * LT;
                if (G::NXV % LT == 0 || v < G::NXV)
                    *reinterpret_cast<XV *>(xs + (v / G::XCPR) * G::PF + (v % G::XCPR) * G::VX) =
                        xr[j];
            }
        } else {
#pragma unroll
            for (int j = 0; j < XREG; ++j) x_scatter_store(tid + j * LT, xb[j], iL0, xs);
            for (int j0 = XREG; j0 < XPER; j0 += XREG) {  // further batches, one latency each
#pragma unroll
                for (int j = 0; j < XREG; ++j)
                    xb[j] = j0 + j < XPER ? x_scatter_load(tid + (j0 + j) * LT)
                                          : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
                for (int j = 0; j < XREG; ++j)
                    if (j0 + j < XPER) x_scatter_store(tid + (j0 + j) * LT, xb[j], iL0, xs);
            }
        }
    };
    auto commit_step = [&](int iL0, int buf) TRK_INLINE {  // into buffer `buf` of Ls and Xs
        commit_l(buf);
        commit_x(iL0, buf);
    };

    // stage-1 row group and column phase of this wave (WIDE; constants when trivial)
    const int wm1 = G::WM1 == G::NW ? wave : wave % G::WM1;
    const int wn1 = G::WN1 == 1 ? 0 : wave / G::WM1;
    // stage-2 row group and column phase of this wave (WIDE)
    constexpr int HW = G::NW / 2;
    const int wm2 = G::TAIL ? (wave < HW ? wave : HW + (wave - HW) / G::TAILJ) : wave % G::WM2;
    const int wn2 = G::TAIL ? (wave < HW ? 0 : (wave - HW) % G::TAILJ) : wave / G::WM2;
    // LDS-staged tiles issue the first step's last-core slice and x first: the commit and
    // stage 1 need them, while the core slices committed after them can still be in flight.
    // (Register-resident tiles keep the slices first: their prologue is bound by the CU's
    // vector-memory rate, and measured 1-2 % faster in that order. The exception are the
    // tiles with half-workgroup loaders, 1 % faster with the step's slices first.)
    // PAIR: two passes over the same tile, the first with the operator's cores, the second
    // with `second`'s; the first pass's reduced outputs (gate) stay in registers of the waves
    // that store, which own the same outputs in both passes, and the store writes
    // silu(gate) * (second pass). Each pass is a whole unit: prologue, steps, reduction.
    Acc<32> acc[G::NYW][G::NACC];
    const int g3 = wave / G::KS3, part3 = wave % G::KS3;
    f32x4 gate[PAIR ? G::NYW : 1];
#pragma unroll 1
    for (int pass = 0; pass < (PAIR ? 2 : 1); ++pass) {
    if (PAIR && pass == 1) {
        Fk = second.fk;
        Sk = second.sk;
        Lk = second.lk;
    }
    constexpr bool STEP_FIRST = !G::WIDE || LT < G::NT;
    if constexpr (HOOKED) issue_l(0);
    else if constexpr (STEP_FIRST) issue_step(0);
    // the first- and second-core slices stay resident for the whole call
    RegA<O, G::BM1, G::KF> fa;
    std::conditional_t<G::W32, RegA32<O, G::BM2, G::K2>, RegA<O, G::BM2, G::K2>> sa;
    auto load_sa = [&]() TRK_INLINE {
        if constexpr (G::W32 && s_frag(C))
            sa.load_frag(Sk + size_t(s0) * R * G::K2, wm2 * G::BM2 * 32, SCv * R, lane);
        else if constexpr (G::W32)
            sa.load(Sk + size_t(s0) * R * G::K2, wm2 * G::BM2 * 32, SCv * R, lane);
        else
            sa.load(Sk + size_t(s0) * R * G::K2, wm2 * G::BM2 * 16, SCv * R, lrow, lgrp);
    };
    if constexpr (G::WIDE) {
        fa.load(Fk + size_t(f0) * R2 * G::KF, wm1 * G::BM1 * 16, FCv * R2, lrow, lgrp);
        if constexpr (!C.SL) load_sa();
    } else {
        cF.issue(Fk + size_t(f0) * R2 * G::KF, 0, FCv * R2 * G::KF / VPE);
        cS.issue(Sk + size_t(s0) * R * G::K2, 0, SCv * R * G::K2 / VPE);
    }
    if constexpr (HOOKED) {
        hook();
        issue_x(0);
    } else if constexpr (!STEP_FIRST) {
        issue_step(0);
    }
    // While the loads fly: zero what no load writes. The contiguous-iF loader writes all of
    // Xs; the scatter loader leaves the K padding, the rows iS >= nS and the rows of absent
    // tokens (TT > 1) to this fill, which writes only those.
    if constexpr (!G::XROW && (G::KF > G::nF || G::nSP > G::nS || G::TT > 1)) {
        constexpr int CH = G::KF / VPE;  // 16-byte chunks per row
        for (int i = tid; i < G::NBUF * G::N1 * CH; i += G::NT) {  // every buffer of Xs
            const int b = i / (G::N1 * CH), n = (i / CH) % G::N1, c = i % CH;
            E *xs = Xs + b * G::szXs;
            const bool empty_row = n % G::nSP >= G::nS || t0 + (n / G::nSP) % G::TT >= T;
            if (empty_row || VPE * c >= G::nF) {
                *reinterpret_cast<uint4 *>(xs + n * G::PF + VPE * c) = make_uint4(0u, 0u, 0u, 0u);
            } else if (G::nF % VPE != 0 && VPE * c + VPE > G::nF) {
                for (int e = G::nF; e < VPE * c + VPE; ++e) xs[n * G::PF + e] = E(0.0f);
            }
        }
    }
    if constexpr (G::K2 > G::nS * R) {
        constexpr int pad = G::K2 - G::nS * R;
        for (int i = tid; i < G::NBUF2 * G::N2R * pad; i += G::NT)  // every buffer of Ub
            Ub[(i / pad) * G::P2 + G::nS * R + i % pad] = E(0.0f);
    }
    commit_step(0, 0);
    if constexpr (!G::WIDE) {
        cF.commit(Fs);
        if constexpr (!C.SL) cS.commit(Ss);
    }
    __syncthreads();
    if constexpr (C.SL) load_sa();  // SL: after the first step's slices are in LDS

    // LDS store offsets of the stage-1 (Ub) and stage-2 (Vb) results, split into a part that
    // depends on the tile only and a part that depends on the lane only.
    //   Ub[(iL', r1, t, f)][(iS, r2)]:  stage-1 rows m = (f, r1, r2), columns n = (iL', t, iS)
    //   Vb[(t, f, s)][(iL', r1, r3)]:   stage-2 rows m = (s, r3), columns n = (iL', r1, t, f)
    //   (the K positions follow the chain's K orders, groups SG and LG)
    auto ub_row = [](int m) {
        const int r2 = m % R;
        return ((m / R) % R * G::TT * G::FC + m / R2) * G::P2 + r2 / G::SG * G::SG * G::nS +
               r2 % G::SG;
    };
    auto ub_col = [](int n) {
        const int iS = n % G::nSP, t = (n / G::nSP) % G::TT, ilp = n / (G::nSP * G::TT);
        return (ilp * R * G::TT * G::FC + t * G::FC) * G::P2 + iS * G::SG;
    };
    auto vb_row = [](int m) {
        const int r3 = m % R;
        return (m / R) * G::P3 + r3 / G::LG * G::LG * R + r3 % G::LG;
    };
    auto vb_col = [](int n) {  // (t, f) is n % Q, (iL', r1) is n / Q
        const int q = n / G::Q;
        return (n % G::Q) * G::PLANE + q / R * R2 + q % R * G::LG;
    };
    auto ub_tile = [&](int mt, int nt) { return ub_row(mt * 16) + ub_col(nt * 16); };
    auto vb_tile = [&](int mt, int nt) { return vb_row(mt * 16) + vb_col(nt * 16); };
    const int ub_lane = ub_row(4 * lgrp) + ub_col(lrow);
    const int vb_lane = vb_row(4 * lgrp) + vb_col(lrow);
    // 32x32 stage-2 tiles: rows mt*32 + 8*g + 4*(lane/32) + e, columns nt*32 + lane%32. With
    // Q = TT * FC not dividing 32 the column part does not split into tile and lane parts:
    // (t, f) = n % Q changes with both, and vb_col32 computes it per tile and lane.
    auto vb_tile32 = [&](int mt, int nt) { return vb_row(mt * 32) + vb_col(nt * 32); };
    const int vb_lane32 = vb_row(4 * (lane >> 5)) + vb_col(lane & 31);
    const int vb_lane32_row = vb_row(4 * (lane >> 5));
    auto vb_col32 = [&](int mt, int nt) TRK_INLINE {  // tile (mt, nt) plus this lane's offset
        if constexpr (32 % G::Q == 0)
            return vb_lane32 + vb_tile32(mt, nt);
        else
            return vb_lane32_row + vb_row(mt * 32) + vb_col(nt * 32 + (lane & 31));
    };

#pragma unroll
    for (int j = 0; j < G::NYW; ++j)
#pragma unroll
        for (int c = 0; c < G::NACC; ++c) acc[j][c].v = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int K3STEPS = G::K3 / 32, PERK = K3STEPS / G::KS3;
    static_assert(K3STEPS % G::KS3 == 0, "stage-3 K steps must split evenly over KS3 waves");

    auto put4 = [&](E *dst, f32x4 d) TRK_INLINE {
        E4 h = {E(d[0]), E(d[1]), E(d[2]), E(d[3])};
        *reinterpret_cast<E4 *>(dst) = h;
    };
    // stage 1 on the x slice in xs (a buffer of Xs)
    auto stage1 = [&](const E *xs, E *ub) TRK_INLINE {
        // stage 1: U^T = F . Xs^T  ->  Ub[(iL',r1,t,f)][(iS,r2)]. A tile (mt, nt) stores at
        // ub_tile(mt, nt) + ub_lane: the rows (f, r1, r2) of mt*16 + 4*lgrp and the columns
        // (iL', t, iS) of nt*16 + lrow split into tile and lane parts (R and 16 are powers of
        // two and nSP is a multiple of 16, so no part carries into another).
        if constexpr (G::WIDE) {
            // a wave whose row tiles all lie past the last one has no stage-1 work
            if (G::M1T % (G::WM1 * G::BM1) == 0 || wm1 * G::BM1 < G::M1T)
            reg_gemm<O, G::BM1, G::KF, G::PF, G::N1T, G::WN1>(fa, xs, wn1, lrow, lgrp, [&](int nt, const f32x4 *d) {
                if (G::nS % 16 != 0 && (nt % (G::nSP / 16)) * 16 + lrow >= G::nS) return;
#pragma unroll
                for (int i = 0; i < G::BM1; ++i) {
                    const int mt = wm1 * G::BM1 + i;
                    if (G::M1T % (G::WM1 * G::BM1) == 0 || mt < G::M1T)
                        put4(ub + ub_lane + ub_tile(mt, nt), d[i]);
                }
            });
        } else {
            lds_gemm<O, G::M1T, G::N1T, G::KF, G::PF, G::NW>(Fs, xs, wave, lrow, lgrp, [&](int mt, int nt, f32x4 d) {
                if (G::nS % 16 == 0 || (nt % (G::nSP / 16)) * 16 + lrow < G::nS)
                    put4(ub + ub_lane + ub_tile(mt, nt), d);
            });
        }
    };
    auto stage2 = [&](const E *ub, E *vb) TRK_INLINE {
        // stage 2: V^T = S . Ub^T  ->  Vb[(t,f,s)][(iL',r1,r3)], rows (s, r3) of mt*16 + 4*lgrp
        // and columns (iL', r1, t, f) of nt*16 + lrow split into tile and lane parts alike
        if constexpr (G::W32) {
            auto st = [&](int nt, const f32x16 *d) TRK_INLINE {
                if (G::N2 % 32 != 0 && nt * 32 + (lane & 31) >= G::N2) return;
#pragma unroll
                for (int i = 0; i < G::BM2; ++i) {
                    const int mt = wm2 * G::BM2 + i;
#pragma unroll
                    for (int g = 0; g < 4; ++g)
                        if (G::M2 % (32 * G::WM2) == 0 || mt * 32 + 8 * g + 4 * (lane >> 5) < G::M2)
                            put4(vb + vb_col32(mt, nt) + vb_row(8 * g),
                                 f32x4{d[i][4 * g], d[i][4 * g + 1], d[i][4 * g + 2], d[i][4 * g + 3]});
                }
            };
            if constexpr (G::TAIL) {
                if (wave < HW) {
                    reg_gemm32<O, 1, G::K2, G::P2, G::N2T32, 1>(sa, ub, 0, lane, st);
                } else {
                    if constexpr (C.TP) __builtin_amdgcn_s_setprio(1);
                    reg_gemm32<O, 1, G::K2, G::P2, G::N2T32, G::TAILJ>(sa, ub, wn2, lane, st);
                    if constexpr (C.TP) __builtin_amdgcn_s_setprio(0);
                }
            } else if (G::M2T32 % G::WM2 == 0 || wm2 * G::BM2 < G::M2T32) {  // else no rows
                reg_gemm32<O, G::BM2, G::K2, G::P2, G::N2T32, G::WN2>(sa, ub, wn2, lane, st);
            }
        } else if constexpr (G::WIDE) {
            if (G::M2T % G::WM2 == 0 || wm2 * G::BM2 < G::M2T)  // else this wave has no rows
            reg_gemm<O, G::BM2, G::K2, G::P2, G::N2T, G::WN2>(sa, ub, wn2, lrow, lgrp, [&](int nt, const f32x4 *d) {
                if (G::N2 % 16 != 0 && nt * 16 + lrow >= G::N2) return;
#pragma unroll
                for (int i = 0; i < G::BM2; ++i) {
                    const int mt = wm2 * G::BM2 + i;
                    if (G::M2 % (16 * G::WM2) == 0 || mt * 16 + 4 * lgrp < G::M2)
                        put4(vb + vb_lane + vb_tile(mt, nt), d[i]);
                }
            });
        } else {
            lds_gemm<O, G::M2T, G::N2T, G::K2, G::P2, G::NW>(Ss, ub, wave, lrow, lgrp, [&](int mt, int nt, f32x4 d) {
                if ((G::N2 % 16 == 0 || nt * 16 + lrow < G::N2) &&
                    (G::M2 % 16 == 0 || mt * 16 + 4 * lgrp < G::M2))
                    put4(vb + vb_lane + vb_tile(mt, nt), d);
            });
        }
    };
    // stage 3 on the last-core slice in ls (a buffer of Ls)
    auto stage3 = [&](const E *vb, const E *ls) TRK_INLINE {
        // stage 3: Y[(t,f,s), l] += Vb . Ls; each wave of a group takes PERK of the K steps,
        // reading the fragments of QB steps before running their MFMAs
        constexpr int QB = PERK < 16 ? PERK : 16;
        static_assert(PERK % QB == 0 && QB % G::NACC == 0, "stage-3 batches must divide evenly");
#pragma unroll
        for (int j = 0; j < G::NYW; ++j) {
            const int tile = g3 + G::G3 * j;
            if (G::NT3 % G::G3 == 0 || tile < G::NT3) {
                const int mt = tile / G::N3T, nt = tile % G::N3T;
                const int m3 = mt * 16 + lrow;  // Vb row (t, f, s)
                const E *a = vb + m3 / G::SC * G::PLANE + m3 % G::SC * G::P3;
                const int l = nt * 16 + lrow;
#pragma unroll
                for (int q0 = 0; q0 < PERK; q0 += QB) {
                    typename O::V8 af[QB], bf[QB];
#pragma unroll
                    for (int q = 0; q < QB; ++q) {
                        const int k = (part3 * PERK + q0 + q) * 32;
                        af[q] = *reinterpret_cast<const typename O::V8 *>(a + k + 8 * lgrp);
                        bf[q] = *reinterpret_cast<const typename O::V8 *>(
                            ls + ((k / R2) * G::LCP + l) * G::PL + k % R2 + 8 * lgrp);
                    }
#pragma unroll
                    for (int q = 0; q < QB; ++q)
                        acc[j][q % G::NACC] = O::k32(af[q], bf[q], acc[j][q % G::NACC]);
                }
            }
        }
    };

    // SL on LDS-staged tiles: the second-core slice, loaded in the prologue, goes to LDS after
    // the first stage 1, which does not read it (stage 2 does, after the next barrier)
    auto late_s = [&]() TRK_INLINE {
        if constexpr (!G::WIDE && C.SL) cS.commit(Ss);
    };
    if constexpr (C.PIPE == 1) {
        // Two buffers of Ls and Xs. Step k+1's slices are committed while step k's are still
        // being read, and stage 3 of step k runs in the same barrier interval as stage 1 of
        // step k+1 (they touch disjoint buffers: Vb and Ls[k] against Xs[k+1] and Ub), so a
        // step costs two barriers and each wave has two stages' MFMAs to interleave.
        //   before the loop: Ls/Xs[0] committed; stage 1(0); barrier; stage 2(0)
        //   step k: commit k+1 into buffer (k+1)&1; barrier; issue loads of k+2;
        //           stage 3(k) on Ls[k&1] and stage 1(k+1) on Xs[(k+1)&1]; barrier; stage 2(k+1)
        // Buffer (k+1)&1 was last read by stage 3(k-1) and stage 1(k-1), both before the
        // second barrier of step k-1.
        issue_step(G::IC);
        stage1(Xs, Ub);
        late_s();
        __syncthreads();
        stage2(Ub, Vb);
        for (int step = 0; step < G::NSTEP; ++step) {
            const int next = step + 1;
            if (next < G::NSTEP) commit_step(next * G::IC, next & 1);
            __syncthreads();
            if (next + 1 < G::NSTEP) issue_step((next + 1) * G::IC);
            stage3(Vb, Ls + (step & 1) * G::szLs);
            if (next < G::NSTEP) stage1(Xs + (next & 1) * G::szXs, Ub);
            __syncthreads();
            if (next < G::NSTEP) stage2(Ub, Vb);
        }
    } else if constexpr (C.PIPE == 2) {
        // Ub and Vb double-buffered as well: barrier interval i holds stage 1 of step i, stage
        // 2 of step i-1 and stage 3 of step i-2, on disjoint buffers (Xs[i&1] -> Ub[i&1];
        // Ub[(i-1)&1] -> Vb[(i-1)&1]; Vb[i&1] and Ls[i&1] -> y), one barrier per step. Waves
        // 0..NW/2-1 take stage 2 first and waves NW/2.. last, so that the two waves sharing a
        // SIMD overlap one's MFMA-bound stage 2 with the other's LDS-bound stages 1 and 3.
        // A buffer written in interval i was last read in interval i-1 or i-2, and is read
        // next in interval i+1 or i+2: the barrier that opens each interval orders them.
        // x of step i+1 and the last-core slice of step i-1 are loaded during interval i and
        // committed before the barrier of interval i+1 (the prologue put step 0's slices in
        // Xs[0] and Ls[0]).
        for (int i = 0; i < G::NSTEP + 2; ++i) {
            const bool s1 = i < G::NSTEP, s2 = i >= 1 && i - 1 < G::NSTEP, s3 = i >= 2;
            if (i >= 1 && i < G::NSTEP) commit_x(i * G::IC, i & 1);
            if (i >= 3) commit_l(i & 1);  // the slice of step i-2
            if (i >= 1) __syncthreads();   // interval 0 follows the prologue's barrier
            if (i + 1 < G::NSTEP) issue_x((i + 1) * G::IC);
            if (i >= 2 && i - 1 < G::NSTEP) issue_l((i - 1) * G::IC);
            E *ub_i = Ub + (i & 1) * G::szUb, *ub_p = Ub + ((i - 1) & 1) * G::szUb;
            E *vb_p = Vb + ((i - 1) & 1) * G::szVb, *vb_i = Vb + (i & 1) * G::szVb;
            const E *xs_i = Xs + (i & 1) * G::szXs, *ls_i = Ls + (i & 1) * G::szLs;
            if (wave < G::NW / 2) {
                if (s2) stage2(ub_p, vb_p);
                if (s3) stage3(vb_i, ls_i);
                if (s1) stage1(xs_i, ub_i);
            } else {
                if (s3) stage3(vb_i, ls_i);
                if (s1) stage1(xs_i, ub_i);
                if (s2) stage2(ub_p, vb_p);
            }
            if (i == 0) late_s();  // before the barrier that opens the first stage 2
        }
    } else {
        for (int step = 0; step < G::NSTEP; ++step) {
            const int iL0 = step * G::IC;
            if (step > 0) {
                __syncthreads();  // stage 3 of the previous step is done with Ls and Vb
                commit_step(iL0, 0);  // its loads were issued at the start of the previous step
                __syncthreads();
            }
            // prefetch the next step's last-core slice and x into registers; they land while
            // this step computes, so a step pays no memory latency of its own
            if (step + 1 < G::NSTEP) issue_step(iL0 + G::IC);
            stage1(Xs, Ub);
            if (step == 0) late_s();
            __syncthreads();
            stage2(Ub, Vb);
            __syncthreads();
            stage3(Vb, Ls);
        }
    }

    // sum the independent chains, then the K-split partials of the waves through LDS
#pragma unroll
    for (int j = 0; j < G::NYW; ++j)
#pragma unroll
        for (int c = 1; c < G::NACC; ++c) acc[j][0].v += acc[j][c].v;
    if constexpr (G::KS3 > 1) {
        __syncthreads();
        float *red = reinterpret_cast<float *>(Ub);
        if (part3 > 0) {
#pragma unroll
            for (int j = 0; j < G::NYW; ++j)
                *reinterpret_cast<f32x4 *>(red + (((part3 - 1) * G::G3 + g3) * G::NYW + j) * 256 +
                                           lane * 4) = acc[j][0].v;
        }
        __syncthreads();
        if (part3 == 0) {
#pragma unroll
            for (int j = 0; j < G::NYW; ++j)
#pragma unroll
                for (int p = 1; p < G::KS3; ++p)
                    acc[j][0].v += *reinterpret_cast<const f32x4 *>(
                        red + (((p - 1) * G::G3 + g3) * G::NYW + j) * 256 + lane * 4);
        }
    }
    if constexpr (PAIR) {
        if (pass == 0) {
#pragma unroll
            for (int j = 0; j < G::NYW; ++j) gate[j] = acc[j][0].v;
            __syncthreads();  // the next pass rewrites the LDS this one reads last
        }
    }
    }  // pass
    if (part3 != 0) return;

    // write y[t, f, s, l] (permuted back to (p, q, r) by the compile-time strides) through
    // the epilogue: the plan's dtype (its own unrolled loop of plain stores), or fp32, or
    // fused with a residual add or a SiLU gate, whose inputs are all read before any store
    auto y_at = [&](int j, int i, size_t *o) {
        const int tile = g3 + G::G3 * j;
        const int mt = tile / G::N3T, nt = tile % G::N3T;
        const int l = nt * 16 + lrow, m = mt * 16 + 4 * lgrp + i;
        const int s = m % G::SC, f = (m / G::SC) % G::FC, t = m / (G::SC * G::FC);
        *o = size_t(t0 + t) * G::OUT + (f0 + f) * G::SYF + (s0 + s) * G::SYS + (l0 + l) * G::SYL;
        return tile < G::NT3 && l < LCv && m < G::M3 && s < SCv && f < FCv && t0 + t < T;
    };
    if constexpr (!EPI) {
#pragma unroll
        for (int j = 0; j < G::NYW; ++j) {
            const int tile = g3 + G::G3 * j;
            if (tile >= G::NT3) continue;
            const int mt = tile / G::N3T, nt = tile % G::N3T;
            const int l = nt * 16 + lrow;
            if (l >= LCv) continue;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = mt * 16 + 4 * lgrp + i;
                const int s = m % G::SC, f = (m / G::SC) % G::FC, t = m / (G::SC * G::FC);
                if (m < G::M3 && s < SCv && f < FCv && t0 + t < T)
                    static_cast<E *>(y)[size_t(t0 + t) * G::OUT + (f0 + f) * G::SYF +
                                        (s0 + s) * G::SYS + (l0 + l) * G::SYL] = E(acc[j][0].v[i]);
            }
        }
    } else {
        float a[G::NYW][4];
#pragma unroll
        for (int j = 0; j < G::NYW; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                size_t o;
                if constexpr (PAIR)
                    a[j][i] = gate[j][i];
                else
                    a[j][i] = y_at(j, i, &o) ? epi_aux<C.dt>(aux, epi_mode, o) : 0.0f;
            }
#pragma unroll
        for (int j = 0; j < G::NYW; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                size_t o;
                if (y_at(j, i, &o)) epi_put<C.dt>(y, epi_mode, o, acc[j][0].v[i], a[j][i]);
            }
    }
}

// The work unit (tile index within a token tile, .x) and token tile (.y) of workgroup
// (bx, by), or .x = -1 for a workgroup that has no work. The dispatcher deals workgroups to
// the 8 XCDs, each with its own L2, round-robin in launch order (x fastest), so workgroup
// lin = by * NBLK + bx runs on XCD lin % 8. A launch on XL XCDs keeps the workgroups dealt to
// XCDs 0..XL-1. Otherwise the units are renumbered so that consecutive ones share an XCD:
//   YM = 0  within each token tile (with NBLK a multiple of 8): consecutive units have the
//           same first-core digit f, hence the same first-core slice, which each XCD then
//           fetches for its share of f only;
//   YM = 1  over the whole launch: XCD x takes the x-th contiguous range of the launch's
//           (token tile, unit) pairs, ordered token tile first. Every unit of a token tile,
//           and so every workgroup writing a given line of y, is then on one XCD (at most two
//           at a range boundary): one L2 writes each line back, where per-token-tile
//           numbering spreads a line's first-core digits over up to 8 L2s. Each XCD needs the
//           slices of every f (and only its token tiles' rows of x).
// Both numberings are bijections of the launch's workgroups onto its (unit, token tile) pairs.
template <KCfg C>
__device__ __forceinline__ int2 unit_of_workgroup(int bx, int by) {
    using G = Geo<C>;
    if constexpr (C.XL) {
        if (bx % 8 >= C.XL) return {-1, by};
        const int w = (bx / 8) * C.XL + bx % 8;  // XCD w % XL, 0 <= w < NBLK
        return {(w % C.XL) * (G::NBLK / C.XL) + w / C.XL, by};
    } else if constexpr (C.YM) {
        const int n = G::NBLK * int(gridDim.y), lin = by * G::NBLK + bx;
        const int xcd = lin % 8, base = n / 8, rem = n % 8;
        // XCD xcd holds workgroups xcd, xcd + 8, ...: base + (xcd < rem) of them, the k-th
        // taking pair g of the XCD's range, which starts after those of XCDs 0..xcd-1
        const int g = xcd * base + (xcd < rem ? xcd : rem) + lin / 8;
        return {g % G::NBLK, g / G::NBLK};
    } else if constexpr (G::NBLK % 8 == 0) {
        return {(bx % 8) * (G::NBLK / 8) + bx / 8, by};
    }
    return {bx, by};
}

inline const char *xl_tag(int xl) {
    return xl == 1 ? "_xl" : xl == 2 ? "_x2" : xl == 4 ? "_x4" : "";
}

// EPI: false compiles the plain store of the plan's dtype only (epi_mode is ignored); true
// compiles every epilogue, chosen at run time by epi_mode. Two instantiations keep the plain
// path's code exactly as it is without epilogues (measured: a run-time branch in its store
// loop cost up to 0.8 us at tokens 8-32).
template <KCfg C, bool EPI>
__global__ void __launch_bounds__(Geo<C>::NT)
    ring3_mfma_kernel(const typename Ops<C.dt>::E *__restrict__ x,
                      const typename Ops<C.dt>::E *__restrict__ Fk,
                      const typename Ops<C.dt>::E *__restrict__ Sk,
                      const typename Ops<C.dt>::E *__restrict__ Lk, void *y, int T,
                      int epi_mode, const void *aux) {  // aux may equal y
    // The arguments fill 14 dwords, all of which arrive preloaded in SGPRs
    // (-amdgpu-kernarg-preload-count): one more would be fetched from the kernel-argument
    // segment, which lives in host memory when HIP_FORCE_DEV_KERNARG=0, and the first LDS
    // wait (lgkmcnt also counts scalar loads) would stall on that PCIe read.
    using G = Geo<C>;
    using E = typename Ops<C.dt>::E;
    // One LDS array per buffer: distinct objects let the compiler see that stores to one
    // buffer never alias reads of another, so it can hoist fragment reads across stores.
    __shared__ __attribute__((aligned(16))) E Fs[G::szFs];
    __shared__ __attribute__((aligned(16))) E Ss[G::szSs];
    __shared__ __attribute__((aligned(16))) E Ls[G::NBUF * G::szLs];
    __shared__ __attribute__((aligned(16))) E Xs[G::NBUF * G::szXs];
    __shared__ __attribute__((aligned(16))) E Ub[G::NBUF2 * G::szUb];
    __shared__ __attribute__((aligned(16))) E Vb[G::NBUF2 * G::szVb];

    const int2 u = unit_of_workgroup<C>(blockIdx.x, blockIdx.y);
    if (u.x < 0) return;  // uniform per workgroup, before any barrier or access
    ring3_unit<C, EPI>(x, Fk, Sk, Lk, y, T, epi_mode, aux, u.x, u.y, Fs, Ss, Ls, Xs, Ub, Vb);
}

template <KCfg C>
int launch_mfma(const Plan &plan, const Variant &v, const void *packed, const void *x, void *y,
                int tokens, Epi epi, hipStream_t stream) {
    using G = Geo<C>;
    using E = typename Ops<C.dt>::E;
    const Chain &c = plan.chains[v.chain];
    const char *base = static_cast<const char *>(packed);
    const E *fk = reinterpret_cast<const E *>(base + c.offF);
    const E *sk = reinterpret_cast<const E *>(base + c.offS);
    const E *lk = reinterpret_cast<const E *>(base + c.offL);
    // one launch covers at most 65535 token tiles (the grid's y limit); more tokens go in
    // consecutive launches on the same stream, each on its own rows of x, y and aux
    constexpr int kMaxTiles = 65535;
    const int per_launch = kMaxTiles * G::TT;
    const size_t y_elem = (epi.mode & kEpiKindMask) == TRK_EPI_F32 ? 4 : sizeof(E);
    const size_t aux_elem = (epi.mode & kAuxF32) ? 4 : sizeof(E);
    for (int t0 = 0; t0 < tokens; t0 += per_launch) {
        const int n = tokens - t0 < per_launch ? tokens - t0 : per_launch;
        const dim3 grid(G::NFC * G::NSC * G::NLC * (C.XL ? 8 / C.XL : 1), (n + G::TT - 1) / G::TT);
        const E *xe = static_cast<const E *>(x) + size_t(t0) * G::IN;
        void *yc = static_cast<char *>(y) + size_t(t0) * G::OUT * y_elem;
        const void *ac =
            epi.aux ? static_cast<const char *>(epi.aux) + size_t(t0) * G::OUT * aux_elem : nullptr;
        // hipLaunchKernel with the argument array: ~0.2 us less host time per launch than the
        // <<<>>> form (no call-configuration push and pop around the host stub), measured
        int tn = n, mode = epi.mode;
        void *args[] = {&xe, &fk, &sk, &lk, &yc, &tn, &mode, &ac};
        const void *fn = epi.mode == TRK_EPI_STORE
                             ? reinterpret_cast<const void *>(&ring3_mfma_kernel<C, false>)
                             : reinterpret_cast<const void *>(&ring3_mfma_kernel<C, true>);
        const int st = check_hip(hipLaunchKernel(fn, grid, dim3(G::NT), args, 0, stream),
                                 "trk_forward: MFMA kernel launch");
        if (st != TRK_OK) return st;
    }
    return TRK_OK;
}

// y = silu(G x) * (U x) for two operators of one shape and plan layout (the gate and up
// projections of a SwiGLU block) in one launch: packed_g and packed_u hold their cores at the
// same section offsets. 12 argument dwords, all preloaded.
template <KCfg C>
__global__ void __launch_bounds__(Geo<C>::NT)
    ring3_pair_kernel(const typename Ops<C.dt>::E *__restrict__ x, const char *__restrict__ packed_g,
                      const char *__restrict__ packed_u, void *y, int offF, int offS, int offL,
                      int T) {
    using G = Geo<C>;
    using E = typename Ops<C.dt>::E;
    __shared__ __attribute__((aligned(16))) E Fs[G::szFs];
    __shared__ __attribute__((aligned(16))) E Ss[G::szSs];
    __shared__ __attribute__((aligned(16))) E Ls[G::NBUF * G::szLs];
    __shared__ __attribute__((aligned(16))) E Xs[G::NBUF * G::szXs];
    __shared__ __attribute__((aligned(16))) E Ub[G::NBUF2 * G::szUb];
    __shared__ __attribute__((aligned(16))) E Vb[G::NBUF2 * G::szVb];
    const int2 u = unit_of_workgroup<C>(blockIdx.x, blockIdx.y);
    if (u.x < 0) return;
    const CoreSections<E> up{reinterpret_cast<const E *>(packed_u + offF),
                             reinterpret_cast<const E *>(packed_u + offS),
                             reinterpret_cast<const E *>(packed_u + offL)};
    ring3_unit<C, true, NoHook, true>(x, reinterpret_cast<const E *>(packed_g + offF),
                                      reinterpret_cast<const E *>(packed_g + offS),
                                      reinterpret_cast<const E *>(packed_g + offL), y, T,
                                      TRK_EPI_SILU_MUL, nullptr, u.x, u.y, Fs, Ss, Ls, Xs,
                                      Ub, Vb, NoHook{}, up);
}

template <KCfg C>
int launch_pair(const Plan &plan, const Variant &v, const void *packed_g, const void *packed_u,
                const void *x, void *y, int tokens, hipStream_t stream) {
    using G = Geo<C>;
    using E = typename Ops<C.dt>::E;
    const Chain &c = plan.chains[v.chain];
    constexpr int kMaxTiles = 65535;
    const int per_launch = kMaxTiles * G::TT;
    for (int t0 = 0; t0 < tokens; t0 += per_launch) {
        const int n = tokens - t0 < per_launch ? tokens - t0 : per_launch;
        const dim3 grid(G::NFC * G::NSC * G::NLC * (C.XL ? 8 / C.XL : 1), (n + G::TT - 1) / G::TT);
        const E *xe = static_cast<const E *>(x) + size_t(t0) * G::IN;
        const char *pg = static_cast<const char *>(packed_g), *pu = static_cast<const char *>(packed_u);
        void *yc = static_cast<void *>(static_cast<E *>(y) + size_t(t0) * G::OUT);
        int oF = int(c.offF), oS = int(c.offS), oL = int(c.offL), tn = n;
        void *args[] = {&xe, &pg, &pu, &yc, &oF, &oS, &oL, &tn};
        const int st = check_hip(hipLaunchKernel(reinterpret_cast<const void *>(&ring3_pair_kernel<C>),
                                                 grid, dim3(G::NT), args, 0, stream),
                                 "trk_forward_swiglu: MFMA kernel launch");
        if (st != TRK_OK) return st;
    }
    return TRK_OK;
}

struct Entry {
    KCfg cfg;
    int t_min, t_max;  // default token range (0, 0: only reachable by index)
    int lds_bytes;
    LaunchFn launch;
    LaunchPairFn launch_pair;  // the fused SwiGLU gate/up kernel of this tile, or null
};

// One shape of the variant table (dtype, chain order, modes, rank); tile() completes it.
struct Shape {
    int dt, F, S, L, i0, i1, i2, o0, o1, o2, R;
};
constexpr KCfg tile(Shape s, int TT, int FC, int SC, int LC, int IC, int KS3, int NACC,
                    int WIDE = 0, int MF2 = 16, int NW = 4, int PIPE = 0, int S1 = 0,
                    int XL = 0, int YM = 0, int SL = 0, int TP = 0) {
    return KCfg{s.dt, s.F, s.S, s.L, s.i0, s.i1, s.i2, s.o0, s.o1, s.o2, s.R,
                TT, FC, SC, LC, IC, KS3, NACC, WIDE, MF2, NW, PIPE, S1, XL, YM, SL, TP};
}

#define TRK_ENTRY(CFG, TMIN, TMAX) \
    {CFG, TMIN, TMAX, Geo<CFG>::LDS_BYTES, launch_mfma<CFG>, nullptr},
// a tile of a shape that serves as the gate and up projections of SwiGLU blocks
#define TRK_ENTRY_PAIR(CFG, TMIN, TMAX) \
    {CFG, TMIN, TMAX, Geo<CFG>::LDS_BYTES, launch_mfma<CFG>, launch_pair<CFG>},

// Appends the variants of `entries` that match the plan's shape and dtype; returns how many.
inline int register_entries(Plan *plan, const Entry *entries, int count) {
    int added = 0;
    for (const Entry *p = entries; p != entries + count; ++p) {
        const Entry &e = *p;
        const KCfg &k = e.cfg;
        const int ins[3] = {k.i0, k.i1, k.i2}, outs[3] = {k.o0, k.o1, k.o2};
        if (k.dt != plan->dtype || k.R != plan->rank || !std::equal(ins, ins + 3, plan->in_modes) ||
            !std::equal(outs, outs + 3, plan->out_modes))
            continue;
        if (plan->nvariants == kMaxVariants) break;
        const int order[3] = {k.F, k.S, k.L};
        const int chain = plan_chain(plan, order, s_group(k), l_group(k), s_frag(k));
        if (chain < 0) continue;
        Variant &v = plan->variants[plan->nvariants++];
        v.kind = TRK_KERNEL_MFMA;
        v.chain = chain;
        v.tile[0] = k.TT;
        v.tile[1] = k.FC;
        v.tile[2] = k.SC;
        v.tile[3] = k.LC;
        v.tile[4] = k.IC;
        v.block = 64 * k.NW;
        v.lds_bytes = e.lds_bytes;
        v.t_min = e.t_min;
        v.t_max = e.t_max;
        v.launch = e.launch;
        v.launch_pair = e.launch_pair;
        v.xcd_local = k.XL;
        if (k.WIDE) {
            char s1[8] = "";
            if (k.S1) std::snprintf(s1, sizeof(s1), "_s%d", k.S1);
            std::snprintf(v.name, sizeof(v.name),
                          "ring3_mfma_wide%d%s%s%s%s%s%s%s%s<%d%d%d,%d,%d,%d,%d,%d,%d,%d>", k.WIDE,
                          k.MF2 == 32 ? "x32" : "", k.NW == 8 ? "w8" : "",
                          k.PIPE == 2 ? "p2" : k.PIPE ? "p" : "", s1, xl_tag(k.XL),
                          k.YM ? "_g" : "", k.SL ? "_sl" : "", k.TP ? "_tp" : "", k.F,
                          k.S, k.L, k.TT, k.FC, k.SC, k.LC, k.IC, k.KS3, k.NACC);
        } else {
            std::snprintf(v.name, sizeof(v.name), "ring3_mfma%s%s%s%s%s<%d%d%d,%d,%d,%d,%d,%d,%d,%d>",
                          k.NW == 8 ? "_w8" : "", k.PIPE == 2 ? "_p2" : k.PIPE ? "_p" : "",
                          xl_tag(k.XL), k.YM ? "_g" : "", k.SL ? "_sl" : "", k.F,
                          k.S, k.L, k.TT, k.FC,
                          k.SC, k.LC, k.IC, k.KS3, k.NACC);
        }
        ++added;
    }
    return added;
}

}  // namespace
}  // namespace trk

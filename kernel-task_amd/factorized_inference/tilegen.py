"""Tile generator: MFMA variant tables for declared operator shapes.

    python -m factorized_inference.tilegen            (from kernel-task_amd/; writes csrc/gen/)

The MFMA kernel (csrc/trk_mfma_kernel.h) is compiled per shape and workgroup tile. Every
shape declared in DECLARED below (the BASELINE configs and the reference's Qwen3.8-27B
shapes) gets a generated table:

  1. chain order: the order (F, S, L) with the least MFMA work after padding (stage-1 K to
     16, the second core's input mode to 16 rows, stage-2 K to 16, the last core's outputs to
     16), ties to the order with the least unpadded work;
  2. candidate tiles: single-token tiles that split the ring over many workgroups, mid-size
     tiles that own all second-core outputs, and register-resident (WIDE) tiles with
     32x32x16 stage-2 MFMAs for large token counts; each checked against the kernel's
     compile-time constraints, its 160 KB LDS budget and a register estimate;
  3. token ranges: from the autotuner's measurements (csrc/gen/tuned.json, written by
     kernel-task_amd/benchmarks/autotune.py on an MI355X) when they exist, else a rule.
     Once a shape is tuned, only the tiles that won a token range are compiled.

The extended search (--extended, the autotuner's input) widens step 2: further chain orders
within 15 % of the least padded work, 1-8 tokens per workgroup in every family, quarter and
eighth second-core tiles, single-token tiles without the stage-3 wave reduction, more
last-core inputs per step, a 4-row-group register-resident family on 8 waves, one token
(and one token with two first-core digits) per register-resident workgroup, the two
pipelined main loops (PIPE 1 and 2) of every multi-step tile, single-token tiles placed on
1, 2 or 4 XCDs, larger stage-1 row groups (S1) of the previous winners, the previous
winners with their second-core slice arriving during the first stage 1 (SL) and with the
issue priority of their stage-2 tail waves (TP, where they have some), and the neighbours
of the previous register-resident winners (tokens, first-core digits, main loop, S1 and
stage-3 split varied together).

Role of the reference's V3G generators (tools/gen_v3g_tilings.py, tools/gen_v3g_tuned.py,
src/factorized_inference/v3g_tuned.py:4-17): a compiled variant list for the Qwen3.8-27B
layer shapes (tools/qwen_shapes.py:20-27) and a measured table of the fastest tiling per
token count. Own design: the tile space, the checks and the table format are this
kernel's.
"""
from __future__ import annotations

import json
import re
from dataclasses import asdict, dataclass, field, replace
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE.parent / "csrc"
GEN_DIR = CSRC / "gen"
TUNED = GEN_DIR / "tuned.json"

DTYPES = {"f16": "TRK_DTYPE_F16", "bf16": "TRK_DTYPE_BF16", "f32": "TRK_DTYPE_F32"}
ELEM_BYTES = {"f16": 2, "bf16": 2, "f32": 4}
LDS_LIMIT = 160 * 1024
# registers a wave may give to the register-resident core slices (4 waves: one wave per
# SIMD; 8 waves: two per SIMD, half the register file each)
WIDE_VGPR_BUDGET = {4: 136, 8: 128}
WIDE_VGPR_RELAXED = {4: 168, 8: 152}  # offered only when no tile fits the budget above
ORDERS = ((0, 1, 2), (1, 2, 0), (2, 0, 1), (0, 2, 1), (1, 0, 2), (2, 1, 0))


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


def rup(a: int, b: int) -> int:
    return cdiv(a, b) * b


@dataclass(frozen=True)
class ShapeDecl:
    """One operator shape to compile MFMA variants for."""

    name: str
    ins: tuple
    outs: tuple
    rank: int
    dtype: str = "bf16"
    order: tuple | None = None  # chain order override (default: least padded MFMA work)
    swiglu: bool = False  # the gate/up projections of SwiGLU blocks: compile the fused pair kernel

    @property
    def key(self) -> str:
        i, o = self.ins, self.outs
        return (f"{self.dtype}_{i[0]}x{i[1]}x{i[2]}_{o[0]}x{o[1]}x{o[2]}_r{self.rank}")


@dataclass(frozen=True)
class Tile:
    """Workgroup tile of ring3_mfma (csrc/trk_mfma_kernel.h, struct KCfg)."""

    TT: int
    FC: int
    SC: int
    LC: int
    IC: int
    KS3: int
    NACC: int
    WIDE: int = 0
    MF2: int = 16
    NW: int = 4
    PIPE: int = 0  # 1: double-buffered slices, two barriers per step; 2: also double-buffered
    #                stage results, three steps' stages in one barrier interval
    S1: int = 0    # WIDE stage-1 row tiles per wave (0: the kernel's default split)
    XL: int = 0    # XCDs the launch's work runs on: 0 = all 8; 1, 2 or 4 (KCfg::XL)
    YM: int = 0    # 1: workgroups numbered over the whole launch, one contiguous range of
    #                (token tile, unit) per XCD (KCfg::YM); 0: within each token tile
    SL: int = 0    # 1: the second-core slice arrives while the first stage 1 runs: read after
    #                the first commit (register-resident) or written to LDS after the first
    #                stage 1 (LDS-staged) (KCfg::SL)
    TP: int = 0    # 1: the tail waves of a pair-and-tail stage 2 hold the issue priority while
    #                they run it (KCfg::TP; tiles with tail waves only)

    def args(self) -> str:
        """Arguments of tile(shape, ...) in the variant tables."""
        a = [self.TT, self.FC, self.SC, self.LC, self.IC, self.KS3, self.NACC]
        # each optional argument is spelled out when it or any later one differs from its default
        tail = [self.PIPE, self.S1, self.XL, self.YM, self.SL, self.TP]
        last = max((i for i, v in enumerate(tail) if v), default=-1)
        if last >= 0 or (self.WIDE, self.MF2, self.NW) != (0, 16, 4):
            a += [self.WIDE, self.MF2, self.NW]
        a += tail[:last + 1]
        return ", ".join(map(str, a))


# The linear layers of Qwen3.8-27B as tensor-ring shapes, the reference's own list
# (tools/qwen_shapes.py:20-27), at ring ranks 8 and 16 in bf16 (tools/qwen_bench.py).
QWEN = {
    "mlp_gate_up": ((20, 16, 16), (16, 34, 32)),
    "mlp_down": ((34, 32, 16), (16, 16, 20)),
    "attn_q_gate": ((20, 16, 16), (16, 24, 32)),
    "attn_kv": ((20, 16, 16), (8, 8, 16)),
    "o_proj": ((24, 16, 16), (16, 16, 20)),
    "gdn_qkvz": ((20, 16, 16), (16, 32, 32)),
}
# The BASELINE configs: 1920 -> 2880 at ranks 8 and 16 in fp16 (chain order (G3, G2, G1), whose
# stage-1 x reads are contiguous in iF), the Llama-3-8B up/down projections in bf16, and
# 1920 -> 2880 at rank 8 in fp32 (config 1, the reference's CPU case; fp32 MFMAs here).
BASELINE = [
    ShapeDecl("r8", (8, 12, 20), (12, 10, 24), 8, "f16", (2, 1, 0)),
    ShapeDecl("r16", (8, 12, 20), (12, 10, 24), 16, "f16", (2, 1, 0)),
    ShapeDecl("llama_up", (16, 16, 16), (16, 28, 32), 8, "bf16", swiglu=True),
    ShapeDecl("llama_down", (16, 28, 32), (16, 16, 16), 16, "bf16"),
    ShapeDecl("r8_fp32", (8, 12, 20), (12, 10, 24), 8, "f32", (2, 1, 0)),
]
DECLARED = BASELINE + [ShapeDecl(f"qwen_{name}", ins, outs, rank, swiglu=name == "mlp_gate_up")
                       for name, (ins, outs) in QWEN.items() for rank in (8, 16)]


@dataclass
class Chain:
    order: tuple
    nF: int
    nS: int
    nL: int
    oF: int
    oS: int
    oL: int
    IN: int
    xrow: bool = field(default=False)


def chain_of(shape: ShapeDecl, order: tuple) -> Chain:
    F, S, L = order
    n, o = shape.ins, shape.outs
    return Chain(order, n[F], n[S], n[L], o[F], o[S], o[L], n[0] * n[1] * n[2], xrow=F == 2)


def padded_work(shape: ShapeDecl, order: tuple) -> tuple[int, int]:
    """(MFMA multiply-adds per token after padding, unpadded multiply-adds per token) of
    the three stages when one workgroup owns all second- and last-core outputs."""
    c, R = chain_of(shape, order), shape.rank
    s1 = c.oF * R * R * c.nL * rup(c.nS, 16) * rup(c.nF, 16)
    s2 = c.oS * R * c.nL * R * c.oF * rup(c.nS * R, 16)
    s3 = c.oF * c.oS * rup(c.oL, 16) * c.nL * R * R
    u1 = c.IN * c.oF * R * R
    u2 = c.nS * c.nL * c.oF * c.oS * R ** 3
    u3 = c.nL * c.oF * c.oS * c.oL * R * R
    return s1 + s2 + s3, u1 + u2 + u3


def choose_order(shape: ShapeDecl) -> tuple:
    if shape.order is not None:
        return tuple(shape.order)
    return min(ORDERS, key=lambda o: padded_work(shape, o))


ALT_ORDER_SLACK = 1.15  # extended search: further orders within 15 % of the least padded work


def search_orders(shape: ShapeDecl, extended: bool = False) -> list[tuple]:
    """Chain orders whose tiles are candidates: the shape's order, and with extended=True
    every other order within ALT_ORDER_SLACK of the least padded work (a smaller stage-2 K
    or a better-balanced stage-2 row count can outweigh a few percent more work)."""
    first = choose_order(shape)
    if not extended:
        return [first]
    least = min(padded_work(shape, o)[0] for o in ORDERS)
    rest = sorted((o for o in ORDERS if o != first and
                   padded_work(shape, o)[0] <= ALT_ORDER_SLACK * least),
                  key=lambda o: padded_work(shape, o)[0])
    return [first] + rest


def order_tag(order: tuple) -> str:
    return "".join(map(str, order))


def vb_store_degree(w32: bool, q: int, R: int, lg: int, p3: int, plane: int) -> int:
    """Worst LDS bank multiplicity of a half-wave's stage-2 result store (vb_store_degree in
    trk_mfma_kernel.h): 32 lanes of 8-byte stores over 64 banks of 4 bytes."""
    hits = [0] * 64
    for lane in range(32):
        m, n = (0, lane) if w32 else (4 * (lane // 16), lane % 16)
        r3, qq = m % R, n // q
        el = ((m // R) * p3 + r3 // lg * lg * R + r3 % lg + (n % q) * plane
              + qq // R * R * R + qq % R * lg)
        bank = el * 2 // 4 % 64
        hits[bank] += 1
        hits[(bank + 1) % 64] += 1
    return max(hits)


def vb_read_degree(m3t: int, sc: int, p3: int, plane: int) -> int:
    """Worst 16-byte-unit multiplicity of the stage-3 Vb fragment reads (vb_read_degree in
    trk_mfma_kernel.h): the first 32 lanes of every 16-row tile, units modulo 512 bytes."""
    worst = 0
    for mt in range(m3t):
        hits = [0] * 32
        for lane in range(32):
            m3 = mt * 16 + lane % 16
            el = m3 // sc * plane + m3 % sc * p3
            u = (el // 8 + lane // 16) % 32
            hits[u] += 1
        worst = max(worst, max(hits))
    return worst


def vb_layout(w32: bool, q: int, R: int, lg: int, k3: int, p3a: int, sc: int,
              m3t: int) -> tuple[int, int]:
    """(row pitch, plane pad) of the kernel's Vb (vb_layout in trk_mfma_kernel.h): the 16x16
    pitch p3a or k3 + 8, and a pad below 128, minimising 5 x store + read conflicts."""
    best, cost = (p3a, 0), 1 << 30
    for p3 in dict.fromkeys((p3a, k3 + 8)):
        for pad in range(0, 128, 8):
            plane = sc * p3 + pad
            c = 5 * vb_store_degree(w32, q, R, lg, p3, plane) + vb_read_degree(m3t, sc, p3, plane)
            if c < cost:
                best, cost = (p3, pad), c
    return best


def pitch16(k: int) -> int:
    """LDS row pitch of a buffer read as 16x16x32 fragments (pitch16 in trk_mfma_kernel.h):
    2 modulo 4 units of 16 bytes."""
    return k + 8 * ((6 - k // 8 % 4) % 4)


def pitch32(k: int) -> int:
    """LDS row pitch of a buffer read as 32x32x16 fragments: an odd number of 16-byte units."""
    return k + 8


def geometry(shape: ShapeDecl, order: tuple, t: Tile) -> dict:
    """The kernel's compile-time geometry (struct Geo) for one tile, with the reason the
    kernel would reject it ("" when it compiles). Mirrors the static_asserts of Geo."""
    c, R = chain_of(shape, order), shape.rank
    R2 = R * R
    eb = ELEM_BYTES[shape.dtype]
    g = {}
    KF, K2, nSP = rup(c.nF, 16), rup(c.nS * R, 16), rup(c.nS, 16)
    M1 = t.FC * R2
    M1T = M1 // 16
    N1 = t.IC * t.TT * nSP
    M2 = t.SC * R
    M2T = cdiv(M2, 16)
    M2P = M2T * 16
    N2 = t.IC * R * t.TT * t.FC
    N2T = cdiv(N2, 16)
    N2P = N2T * 16
    M3 = t.TT * t.FC * t.SC
    M3T = cdiv(M3, 16)
    M3P = M3T * 16
    N3T = cdiv(t.LC, 16)
    LCP = N3T * 16
    K3 = t.IC * R2
    NW = t.NW
    NT3 = M3T * N3T
    wide = t.WIDE != 0
    W32 = wide and t.MF2 == 32
    WM2 = t.WIDE if wide else NW
    G3 = NW // t.KS3 if t.KS3 and NW % t.KS3 == 0 else 1
    NYW = cdiv(NT3, G3)
    nbuf, nbuf2 = (2 if t.PIPE else 1), (2 if t.PIPE == 2 else 1)
    N2R = cdiv(N2, 32) * 32 if W32 else N2P

    def lds_elems(pf, p2, p3, pl):  # as lds_elems in trk_mfma_kernel.h (Vb planes unpadded)
        vb = (M3P - 1) // t.SC * t.SC * p3 + ((M3P - 1) % t.SC + 1) * p3
        return ((16 if wide else M1 * pf + M2P * p2) + nbuf * (t.IC * LCP * pl + N1 * pf)
                + nbuf2 * (N2R * p2 + vb))
    # pitches for the fragment shape each buffer is read with, where the tile fits with them
    cfp = eb * lds_elems(pitch16(KF), pitch32(K2) if W32 else pitch16(K2), pitch16(K3),
                         pitch16(R2)) <= LDS_LIMIT
    PF, PL = (pitch16(KF), pitch16(R2)) if cfp else (KF + 8, R2 + 8)
    P2 = pitch32(K2) if W32 else pitch16(K2) if cfp else K2 + 8
    M2T32, N2T32 = cdiv(M2, 32), cdiv(N2, 32)
    if t.S1:
        BM1, WM1 = t.S1, M1T // t.S1 if M1T % t.S1 == 0 else 0
    elif M1T < NW and NW % M1T == 0:
        BM1, WM1 = 1, M1T
    else:
        BM1, WM1 = cdiv(M1T, NW), NW
    BM2 = cdiv(M2T32 if W32 else M2T, WM2)
    # the pair-and-tail stage 2 (Geo::TAIL): waves 4-7 split the row tiles past the first 4
    tailr = M2T32 - NW // 2
    g["TAIL"] = (W32 and NW // WM2 == 1 and BM2 == 1 and NW == 8 and tailr > 0 and M2T32 < NW
                 and (NW // 2) % tailr == 0)
    sz = {
        "Fs": 8 if wide else M1 * PF,
        "Ss": 8 if wide else M2P * P2,
        "Ls": nbuf * t.IC * LCP * PL,
        "Xs": nbuf * N1 * PF,
        "Ub": nbuf2 * N2R * P2,
    }
    # Vb: the layout with the fewest conflicts, plane padding only where it fits (as the kernel)
    lg = 8 if R == 8 and not W32 else 4  # l_group in trk_mfma_kernel.h
    P3, pad = vb_layout(W32, t.TT * t.FC, R, lg, K3, pitch16(K3) if cfp else K3 + 8, t.SC, M3T)
    vb = lambda plane: nbuf2 * ((M3P - 1) // t.SC * plane + ((M3P - 1) % t.SC + 1) * P3)  # noqa: E731
    sz["Vb"] = vb(t.SC * P3 + pad)
    if eb * sum(sz.values()) > LDS_LIMIT:
        sz["Vb"] = vb(t.SC * P3)
    lds = eb * sum(sz.values())
    red_floats = (t.KS3 - 1) * G3 * NYW * 256
    k3steps = K3 // 32 if K3 % 32 == 0 else 0
    perk = k3steps // t.KS3 if t.KS3 else 0
    qb = min(perk, 16)
    g.update(LDS_BYTES=lds, NBLK=cdiv(c.oF, t.FC) * cdiv(c.oS, t.SC) * cdiv(c.oL, t.LC),
             NSTEP=cdiv(c.nL, t.IC), BM1=BM1, BM2=BM2, NYW=NYW, K2=K2, KF=KF)
    # register-resident slices (WIDE): A fragments held by each wave (an 8-element fragment
    # is 4 VGPRs in 16 bits, 8 in fp32)
    if wide:
        v8 = 2 * eb
        # a trailing 16 of K after 32-wide steps is held as a full 8-element fragment
        tail = lambda k: (v8 if k >= 32 else v8 // 2) if k % 32 else 0  # noqa: E731
        fa = BM1 * (KF // 32 * v8 + tail(KF))
        sa = BM2 * (K2 // 16) * v8 if W32 else BM2 * (K2 // 32 * v8 + tail(K2))
        g["slice_vgprs"] = fa + sa
    nblk = g["NBLK"]
    checks = [
        (R % 8 == 0 and R & (R - 1) == 0, "rank must be a power of two >= 8"),
        (NW in (4, 8), "4 or 8 waves"),
        (0 <= t.WIDE <= NW and (t.WIDE == 0 or NW % t.WIDE == 0), "WIDE divides the waves"),
        (t.MF2 == 16 or (t.MF2 == 32 and wide), "MF2 is 16, or 32 with WIDE"),
        (W32 or 16 % (t.FC * t.TT) == 0, "FC * TT must divide 16 (16x16 stage-2 tiles)"),
        (t.KS3 >= 1 and NW % t.KS3 == 0, "KS3 must divide the waves"),
        (k3steps > 0 and k3steps % t.KS3 == 0, "stage-3 K steps must split over KS3"),
        (t.NACC >= 1 and perk % t.NACC == 0, "NACC must divide a wave's K steps"),
        (qb > 0 and perk % qb == 0 and qb % t.NACC == 0, "stage-3 batches must divide"),
        (t.FC <= c.oF and t.SC <= c.oS and t.LC <= c.oL and t.IC <= c.nL and t.TT >= 1,
         "tile too large"),
        (c.nL % t.IC == 0, "IC must divide the last core's input mode"),
        (t.PIPE in (0, 1, 2) and (t.PIPE == 0 or c.nL // t.IC > 1), "a pipelined tile needs two steps"),
        (t.S1 == 0 or (wide and WM1 > 0 and NW % WM1 == 0), "S1 must split the stage-1 rows"),
        (t.XL in (0, 1, 2, 4), "XL is 0, 1, 2 or 4"),
        (t.XL == 0 or nblk % t.XL == 0, "XL must divide the workgroups of a token tile"),
        (t.YM == 0 or (t.YM == 1 and t.XL == 0), "YM is 0, or 1 on all 8 XCDs"),
        (t.SL in (0, 1), "SL is 0 or 1"),
        (t.TP == 0 or (t.TP == 1 and g["TAIL"]), "TP needs the pair-and-tail stage 2"),
        (c.xrow or c.IN % (16 // eb) == 0, "scatter loader reads x rows in 16-byte vectors"),
        (lds <= LDS_LIMIT, f"LDS {lds} B exceeds 160 KB"),
        (red_floats * 4 <= N2R * P2 * eb, "stage-3 reduction does not fit in Ub"),
        (not wide or g["slice_vgprs"] <= WIDE_VGPR_RELAXED[NW],
         "register-resident slices too large"),
    ]
    g["reject"] = next((why for ok, why in checks if not ok), "")
    return g


def _divisors_desc(n: int) -> list[int]:
    return [d for d in range(n, 0, -1) if n % d == 0]


def _fit(shape, order, make, ics) -> Tile | None:
    """The first tile make(ic) over ics that the kernel accepts."""
    for ic in ics:
        t = make(ic)
        if t is not None and not geometry(shape, order, t)["reject"]:
            return t
    return None


def _fit_budget(shape, order, make, ics, budget: int) -> Tile | None:
    """The first register-resident tile make(ic) over ics whose core slices take at most
    `budget` registers and that passes every other check of the kernel."""
    for ic in ics:
        t = make(ic)
        g = geometry(shape, order, t)
        if g["reject"] in ("", "register-resident slices too large") and g["slice_vgprs"] <= budget:
            return t
    return None


def candidates(shape: ShapeDecl, order: tuple | None = None,
               extended: bool = False) -> dict[str, Tile]:
    """Named candidate tiles for one shape (each accepted by the kernel's constraints).
    extended=True adds tiles with 2, 4 or 8 tokens per workgroup in every family and
    single-token tiles over the whole last-core input mode (a wider search for the
    autotuner)."""
    order = order or choose_order(shape)
    c, R = chain_of(shape, order), shape.rank
    ics = _divisors_desc(c.nL)
    # K3 = IC * R^2 of 512-1024 keeps the per-step LDS traffic balanced at one token
    small_ics = [d for d in ics if d * R * R <= 1024] or ics[-1:]
    out: dict[str, Tile] = {}

    def add(name, make, pool):
        t = _fit(shape, order, make, pool)
        if t is not None and t not in out.values():
            out[name] = t

    LC = c.oL
    # one token: the ring split over many workgroups, stage 3's K split over the waves
    add("t1_s1", lambda ic: Tile(1, 1, 1, LC, ic, 4, 1), small_ics)
    add("t1_s2", lambda ic: Tile(1, 1, min(2, c.oS), LC, ic, 4, 1), small_ics)
    add("t1_s1_w8", lambda ic: Tile(1, 1, 1, LC, ic, 8, 1, 0, 16, 8), small_ics)
    # a few tokens: a workgroup owns half or all of the second core's outputs
    half = cdiv(c.oS, 2)
    add("mid_half", lambda ic: Tile(1, 1, half, LC, ic, 1, 2), ics)
    add("mid_all", lambda ic: Tile(1, 1, c.oS, LC, ic, 1, 2), ics)
    # many tokens: register-resident core slices, 4 tokens per workgroup, 32x32 stage 2
    def wide_tile(wide, nw, budget):
        for sc_max in range(c.oS, 0, -1):
            chunks = cdiv(c.oS, sc_max)
            sc = cdiv(c.oS, chunks)  # balanced chunks
            make = lambda ic, sc=sc: Tile(4, 1, sc, LC, ic, 2, 1, wide, 32, nw)  # noqa: E731
            t = _fit_budget(shape, order, make, [d for d in ics if d <= 2] or ics[-1:], budget)
            if t is not None:
                return t
        return None

    # (4 row groups on 8 waves: two stage-2 row tiles per wave, so each B fragment read from
    # LDS feeds two MFMAs, with two waves per SIMD; searched in the extended set only)
    families = ((4, 4), (8, 8)) + (((4, 8),) if extended else ())
    for wide, nw in families:
        t = wide_tile(wide, nw, WIDE_VGPR_BUDGET[nw])
        if t is not None and t not in out.values():
            out[f"wide{wide}x32" + ("w8" if nw == 8 else "")] = t
    # one token per register-resident workgroup, twice the base tile's last-core inputs per
    # step where they fit, pipelined when it takes several steps: the family that won 5-64
    # tokens on every tuned BASELINE shape (the untuned rule's pick there)
    base = out.get("wide8x32w8")
    if base is not None:
        for ic in (2 * base.IC, base.IC):
            if ic > c.nL or c.nL % ic:
                continue
            t = Tile(1, 1, base.SC, LC, ic, 1, 2, base.WIDE, 32, base.NW,
                     1 if cdiv(c.nL, ic) > 1 else 0)
            if not geometry(shape, order, t)["reject"] and t not in out.values():
                out["wide8x32w8_t1"] = t
                break
    if extended:
        # XCD-local single-token tiles (every workgroup on one XCD: one L2 fetches each core
        # slice once and owns every line of y). Few workgroups read the replicated last-core
        # slice through that one L2, so each owns all or half of the second core's outputs.
        for sc, tag in ((c.oS, "all"), (half, "half")):
            add(f"t1_{tag}_xl", lambda ic, sc=sc: Tile(1, 1, sc, LC, ic, 4, 1, XL=1), small_ics)
            add(f"t1_{tag}_w8_xl", lambda ic, sc=sc: Tile(1, 1, sc, LC, ic, 4, 1, 0, 16, 8, XL=1),
                small_ics)
        add("t1_s1_icall", lambda ic: Tile(1, 1, 1, LC, ic, 4, 1), ics)
        add("t1_s2_icall", lambda ic: Tile(1, 1, min(2, c.oS), LC, ic, 4, 1), ics)
        # 8 waves with stage 3's K split four ways (measured 3-6 % faster for Llama down at
        # 1-2 tokens than the eight-way split)
        for sc in (1, 2):
            add(f"t1_s{sc}_w8_k4", lambda ic, sc=sc: Tile(1, 1, min(sc, c.oS), LC, ic, 4, 1, 0, 16, 8),
                small_ics)
        # single-token tiles that split the last core's outputs over 2-8 workgroups: each
        # reads part of the last-core slice that every workgroup otherwise reads whole, and
        # owns 1-4 second-core digits (measured 12 % faster for Llama up at one token)
        for lc in (d for d in range(c.oL - 1, 1, -1) if c.oL % d == 0 and c.oL // d <= 8):
            for sc in sorted({1, 2, 4} & set(range(1, c.oS + 1))):
                for nw, ks3 in ((4, 4), (8, 8)):
                    add(f"t1_l{lc}_s{sc}" + ("_w8" if nw == 8 else "") + f"_k{ks3}",
                        lambda ic, lc=lc, sc=sc, nw=nw, ks3=ks3: Tile(
                            1, 1, sc, lc, ic, ks3, 1, 0, 16, nw), small_ics)
        # stage 3 on fewer waves with independent accumulator chains: no cross-wave
        # reduction (a barrier and an LDS round trip) at the price of a longer K loop
        for sc in (1, 2):
            for ks3, nacc in ((1, 4), (2, 2)):
                add(f"t1_s{sc}_k{ks3}n{nacc}", lambda ic, sc=sc, ks3=ks3, nacc=nacc: Tile(
                    1, 1, min(sc, c.oS), LC, ic, ks3, nacc), small_ics)
        for tt in (2, 4):
            add(f"mid_half_t{tt}", lambda ic, tt=tt: Tile(tt, 1, half, LC, ic, 1, 2), ics)
            add(f"mid_all_t{tt}", lambda ic, tt=tt: Tile(tt, 1, c.oS, LC, ic, 1, 2), ics)
        # a quarter or an eighth of the second core's outputs per workgroup, stage 3's K
        # split over two waves when the K steps allow it
        for part in (4, 8):
            sc = cdiv(c.oS, part)
            if 2 < sc < half:
                for ks3 in (2, 1):
                    before = len(out)
                    add(f"mid_1of{part}_k{ks3}", lambda ic, sc=sc, ks3=ks3: Tile(
                        1, 1, sc, LC, ic, ks3, 2), ics)
                    if len(out) > before:
                        break
        for wide, nw in families:
            fam = f"wide{wide}x32" + ("w8" if nw == 8 else "")
            base = out.get(fam)
            if base is None:
                continue
            for tt, ks3, nacc in ((8, 2, 1), (4, 1, 2), (8, 1, 2), (2, 1, 4), (2, 1, 2)):
                add(f"{fam}_t{tt}k{ks3}n{nacc}",
                    lambda ic, tt=tt, ks3=ks3, nacc=nacc, base=base: Tile(
                        tt, 1, base.SC, LC, ic, ks3, nacc, wide, 32, nw),
                    [base.IC] + [d for d in ics if d < base.IC])
            # more last-core inputs per step (fewer steps and barriers), over the register
            # budget if need be: a few spilled registers may still win
            for mult in (2, 4):
                ic = base.IC * mult
                if ic > c.nL or c.nL % ic:
                    continue
                # (2 tokens: twice the inputs per step in the LDS of 4 tokens' tiles; measured
                # 5 % faster for Llama down at 32 tokens; stage 3 split four ways puts its two
                # output tiles on all 8 waves)
                for tt, ks3, nacc in ((4, 2, 1), (4, 1, 2), (2, 1, 2), (2, 2, 1), (2, 4, 1)):
                    t = Tile(tt, 1, base.SC, LC, ic, ks3, nacc, wide, 32, nw)
                    if not geometry(shape, order, t)["reject"] and t not in out.values():
                        out[f"{fam}_t{tt}k{ks3}n{nacc}_ic{ic}"] = t
                # one token per workgroup (twice the workgroups of the 2-token tiles, with
                # the LDS left for the pipelined schedules), or one token with two
                # first-core digits (the 2-token tiles' stage-2 columns from one token's x).
                # Measured on Llama down: 9 % faster at 9-16 tokens, 3 % at 17-32.
                for tt, fc, ks3, nacc in ((1, 1, 1, 2), (1, 1, 2, 1), (1, 2, 1, 2)):
                    t = Tile(tt, fc, base.SC, LC, ic, ks3, nacc, wide, 32, nw)
                    if not geometry(shape, order, t)["reject"] and t not in out.values():
                        tag = f"f{fc}" if fc > 1 else f"t{tt}"
                        out[f"{fam}_{tag}k{ks3}n{nacc}_ic{ic}"] = t
            # first-core chunks that no power of two gives (TT * FC not dividing 16; the
            # 32x32 stage-2 stores then compute their column offsets per lane): 3 of 24
            # digits makes one token's workgroups 8, so that 32 tokens fill the 256 CUs once
            # (measured at 1920->2880 R16 T=32: 12.03 -> 11.27 us against the 192
            # workgroups of 2 tokens x 2 digits)
            # one token with the second core's outputs split in two or four, stage 1 recomputed
            # per chunk: at few tokens the one-token tiles of all second-core digits are too few
            # workgroups to fill 256 CUs (measured at Llama down T=8: 128 workgroups of 16 digits
            # 16.1 us, 256 of 8 digits 11.8 us)
            for part in (2, 4):
                sc = cdiv(c.oS, part)
                if nw != 8 or sc >= base.SC:
                    continue
                for ic in (base.IC, 2 * base.IC):
                    if ic > c.nL or c.nL % ic:
                        continue
                    t = Tile(1, 1, sc, LC, ic, 2, 1, wide, 32, nw)
                    if not geometry(shape, order, t)["reject"] and t not in out.values():
                        out[f"{fam}_sc{sc}k2n1_ic{ic}"] = t
            # and both at once: first-core chunks of 2-8 digits with the whole, half or a
            # quarter of the second core, so that some chunking fills 256 CUs at each token
            # count (e.g. 1920->2880 R16 T=16: 3 first-core x 5 second-core digits, 256
            # workgroups)
            for fc in (f for f in range(2, 9) if nw == 8 and c.oF % f == 0):
                for part in (1, 2, 4):
                    sc = cdiv(c.oS, part)
                    t = Tile(1, fc, sc, LC, base.IC, 2, 1, wide, 32, nw)
                    if not geometry(shape, order, t)["reject"] and t not in out.values():
                        out[f"{fam}_f{fc}sc{sc}k2n1_ic{base.IC}"] = t
            for fc in (f for f in range(3, 9) if nw == 8 and c.oF % f == 0 and 16 % f):
                for ks3 in (2, 4):
                    for ic in (base.IC, 2 * base.IC):
                        if ic > c.nL or c.nL % ic:
                            continue
                        t = Tile(1, fc, base.SC, LC, ic, ks3, 1, wide, 32, nw)
                        if not geometry(shape, order, t)["reject"] and t not in out.values():
                            out[f"{fam}_f{fc}k{ks3}n1_ic{ic}"] = t
        # the pipelined main loops for every multi-step tile found so far that still fits
        for name, t in list(out.items()):
            if cdiv(c.nL, t.IC) > 1:
                for pipe, tag in ((1, "_p"), (2, "_p2")):
                    p = replace(t, PIPE=pipe)
                    if not geometry(shape, order, p)["reject"] and p not in out.values():
                        out[name + tag] = p
        # single-token tiles placed on 1, 2 or 4 XCDs where each workgroup of one token tile
        # still gets a CU of its own (32 per XCD): fewer L2s fetch the core slices and write
        # back the lines of y, at the same per-workgroup latency
        for name, t in list(out.items()):
            if t.TT != 1 or t.WIDE or t.XL:
                continue
            nblk = geometry(shape, order, t)["NBLK"]
            for xl in (1, 2, 4):
                p = replace(t, XL=xl)
                if (nblk <= 32 * xl and not geometry(shape, order, p)["reject"]
                        and p not in out.values()):
                    out[name + ("_xl" if xl == 1 else f"_x{xl}")] = p
    if not any(n.startswith("wide") for n in out):
        # no register-resident tile within the budget (a long stage-2 K): offer the smallest
        # over-budget one, which may spill a few registers; the autotuner decides
        for wide, nw in ((4, 4), (8, 8)):
            t = wide_tile(wide, nw, WIDE_VGPR_RELAXED[nw])
            if t is not None and t not in out.values():
                out[f"wide{wide}x32" + ("w8" if nw == 8 else "") + "_relaxed"] = t
    return out


_VARIANT_NAME = re.compile(r"ring3_mfma(?:_wide(\d)(x32)?(w8)?(p2?)?(?:_s(\d+))?|(_w8)?(_p2?)?)"
                           r"(_xl|_x[24])?(_g)?(_sl)?(_tp)?<(\d)(\d)(\d),"
                           r"(\d+),(\d+),(\d+),(\d+),(\d+),(\d+),(\d+)>")


def parse_variant_name(name: str) -> tuple[tuple, Tile]:
    """(chain order, tile) of an MFMA variant from its name in the plan (trk_variant_info)."""
    m = _VARIANT_NAME.fullmatch(name)
    if not m:
        raise ValueError(f"not an MFMA variant name: {name!r}")
    wide = int(m.group(1) or 0)
    order = tuple(int(m.group(i)) for i in (12, 13, 14))
    TT, FC, SC, LC, IC, KS3, NACC = (int(m.group(i)) for i in range(15, 22))
    pipe_tag = m.group(4) or m.group(7) or ""
    pipe = 2 if pipe_tag.endswith("2") else 1 if pipe_tag else 0
    return order, Tile(TT, FC, SC, LC, IC, KS3, NACC, wide, 32 if m.group(2) else 16,
                       8 if (m.group(3) or m.group(6)) else 4, pipe, int(m.group(5) or 0),
                       {None: 0, "_xl": 1, "_x2": 2, "_x4": 4}[m.group(8)],
                       1 if m.group(9) else 0, 1 if m.group(10) else 0,
                       1 if m.group(11) else 0)


def rule_ranges(names: list[str]) -> dict[str, tuple[int, int]]:
    """Default token ranges before the shape is tuned."""
    ranges = {}
    pick = lambda *opts: next((o for o in opts if o in names), None)  # noqa: E731
    t1 = ("t1_s2", "t1_s1", "t1_s1_w8")
    # an over-budget register-resident tile takes its family's place
    original = {n.removesuffix("_relaxed"): n for n in names}
    names = list(original)
    for name, lo, hi in ((pick(*t1, "mid_half", "mid_all", "wide4x32", "wide8x32w8"), 1, 1),
                         (pick("mid_half", "mid_all", "wide4x32", "wide8x32w8", *t1), 2, 4),
                         (pick("wide8x32w8_t1", "mid_half", "mid_all", "wide4x32", "wide8x32w8",
                               *t1), 5, 16),
                         (pick("wide8x32w8_t1", "mid_all", "mid_half", "wide4x32", "wide8x32w8",
                               *t1), 17, 64),
                         (pick("wide8x32w8", "wide4x32", "mid_all", "mid_half", *t1), 65,
                          1 << 30)):
        if name is None:
            continue
        name = original[name]
        if name in ranges:  # extend the range a tile already serves
            ranges[name] = (min(ranges[name][0], lo), max(ranges[name][1], hi))
        else:
            ranges[name] = (lo, hi)
    return ranges


def load_tuned() -> dict:
    return json.loads(TUNED.read_text()) if TUNED.exists() else {}


def s1_variants(shape: ShapeDecl, order: tuple, t: Tile) -> dict[str, Tile]:
    """A register-resident tile with larger stage-1 row groups than the kernel's default split
    (fewer reads of the x slice from LDS, more registers), every one the kernel accepts."""
    out = {}
    if not t.WIDE or t.S1:
        return out
    m1t = t.FC * shape.rank * shape.rank // 16
    default = 1 if m1t < t.NW and t.NW % m1t == 0 else cdiv(m1t, t.NW)
    for s1 in (2, 4, 8, 16):
        if s1 > default and m1t % s1 == 0 and t.NW % (m1t // s1) == 0:
            v = replace(t, S1=s1)
            if not geometry(shape, order, v)["reject"]:
                out[f"_s{s1}"] = v
    return out


def neighbours(shape: ShapeDecl, order: tuple, t: Tile) -> dict[str, Tile]:
    """Local refinements of a register-resident tile that won a range of 5 tokens or more:
    1-4 tokens and 1-2 first-core digits per workgroup, each main loop, each stage-1 row
    group and two stage-3 splits, every one the kernel accepts (the autotuner's second pass;
    it gained 3-6 % at 3-256 tokens on the BASELINE shapes after the first)."""
    out = {}
    if not t.WIDE:
        return out
    for tt, fc in ((1, 1), (1, 2), (2, 1), (2, 2), (4, 1)):
        for pipe in (0, 1, 2):
            for s1 in (0, 2, 4, 8):
                for ks3, nacc in ((t.KS3, t.NACC), (1, 2), (2, 1)):
                    v = replace(t, TT=tt, FC=fc, PIPE=pipe, S1=s1, KS3=ks3, NACC=nacc)
                    if v != t and v not in out.values() and not geometry(shape, order, v)["reject"]:
                        out[f"~t{tt}f{fc}p{pipe}s{s1}k{ks3}n{nacc}"] = v
    return out


def search_candidates(shape: ShapeDecl, extended: bool = False) -> dict[str, tuple[tuple, Tile]]:
    """name -> (order, tile) over every searched order; tiles of an order other than the
    shape's own carry the suffix @FSL in their names."""
    first = choose_order(shape)
    out = {}
    for order in search_orders(shape, extended):
        tag = "" if order == first else "@" + order_tag(order)
        for name, t in candidates(shape, order, extended).items():
            out[name + tag] = (order, t)
    return out


def add_candidate(cands: dict, name: str, order: tuple, tile: Tile) -> str | None:
    """Adds (order, tile) to `cands` under `name`, or under `name#2`, `name#3`, ... when
    another tile holds that name (shortened names of two refined winners can agree); a tile
    already present is not added again. Returns the name used, or None."""
    if (order, tile) in cands.values():
        return None
    unique, k = name, 2
    while unique in cands:
        unique, k = f"{name}#{k}", k + 1
    cands[unique] = (order, tile)
    return unique


def table(shape: ShapeDecl, tuned: dict | None = None, all_candidates: bool = False,
          extended: bool = False) -> list[tuple[str, tuple, Tile, int, int]]:
    """[(name, order, tile, t_min, t_max)] for one shape: the tuned winners when the shape
    has measurements, else every candidate with the rule's ranges (0, 0: index only).
    A tuned entry's "extra" tiles are compiled index-only beside the winners (alternatives
    a caller may route token counts to, such as the XCD-local tiles).
    all_candidates=True ignores the measurements (the autotuner's input)."""
    tuned = load_tuned() if tuned is None else tuned
    entry = None if all_candidates else tuned.get(shape.key)
    if entry:
        rows = [(r["name"], tuple(r.get("order", entry["order"])), Tile(**r["tile"]),
                 r["t_min"], r["t_max"]) for r in entry["ranges"]]
        rows += [(r["name"], tuple(r.get("order", entry["order"])), Tile(**r["tile"]), 0, 0)
                 for r in entry.get("extra", [])]
        for name, order, t, _, _ in rows:
            why = geometry(shape, order, t)["reject"]
            if why:
                raise ValueError(f"{shape.key}: tuned tile {name} is rejected: {why}")
        return rows
    first = choose_order(shape)
    cands = search_candidates(shape, extended)
    ranges = rule_ranges([n for n, (o, _) in cands.items() if o == first])
    if all_candidates and shape.key in tuned:
        # the previous winners stay candidates, so a new search never loses a tile it had;
        # an extended search also tries their larger stage-1 row groups, each of them with its
        # second-core slice arriving during the first stage 1 (SL), those with tail waves in
        # stage 2 with the tail waves' issue priority (TP) and, for the register-resident
        # winners of 5 tokens or more, their neighbours (a local refinement)
        entry = tuned[shape.key]
        for r in entry["ranges"] + entry.get("extra", []):
            order = tuple(r.get("order", entry["order"]))
            if order not in ORDERS:
                continue
            tile = Tile(**r["tile"])
            name = r["name"]
            if order != first and "@" not in name:
                name += "@" + order_tag(order)
            base, _, tag = name.partition("@")
            tag = "@" + tag if tag else ""
            found = [(name, tile)]
            if extended:
                found += [(base + suffix + tag, v)
                          for suffix, v in s1_variants(shape, order, tile).items()]
                late = replace(tile, SL=1)
                if not tile.SL and not geometry(shape, order, late)["reject"]:
                    found.append((base + "_sl" + tag, late))
                prio = replace(tile, TP=1)
                if not tile.TP and not geometry(shape, order, prio)["reject"]:
                    found.append((base + "_tp" + tag, prio))
                if r.get("t_min", 0) >= 5:
                    found += [(base[:40] + suffix + tag, v)
                              for suffix, v in neighbours(shape, order, tile).items()]
            for n, t in found:
                add_candidate(cands, n, order, t)
    return [(n, o, t, *ranges.get(n, (0, 0))) for n, (o, t) in cands.items()]


def _fn_name(shape: ShapeDecl) -> str:
    return "mfma_register_gen_" + shape.key


def emit(shape: ShapeDecl, tuned: dict | None = None, all_candidates: bool = False,
         extended: bool = False) -> str:
    tuned = load_tuned() if tuned is None else tuned
    rows = table(shape, tuned, all_candidates, extended)
    orders = sorted({r[1] for r in rows}, key=lambda od: (od != choose_order(shape), od))
    i, o = shape.ins, shape.outs
    tuned_note = ("token ranges measured by kernel-task_amd/benchmarks/autotune.py"
                  if tuned.get(shape.key) and not all_candidates
                  else "every candidate, token ranges by rule (not tuned)")
    lines = [
        "// Generated by kernel-task_amd/factorized_inference/tilegen.py; do not edit.",
        f"// {shape.name}: ({i[0]},{i[1]},{i[2]}) -> ({o[0]},{o[1]},{o[2]}), rank "
        f"{shape.rank}, {shape.dtype}, chain order"
        f"{'s' if len(orders) > 1 else ''} "
        + ", ".join(f"({od[0]},{od[1]},{od[2]})" for od in orders) + f"; {tuned_note}.",
        '#include "trk_mfma_kernel.h"',
        "",
        "namespace trk {",
        "namespace {",
        "",
    ]
    for od in orders:
        lines.append(f"constexpr Shape kShape{order_tag(od)}{{{DTYPES[shape.dtype]}, {od[0]}, "
                     f"{od[1]}, {od[2]}, {i[0]}, {i[1]}, {i[2]}, {o[0]}, {o[1]}, {o[2]}, "
                     f"{shape.rank}}};")
    lines += ["", "const Entry kEntries[] = {"]
    for name, od, t, lo, hi in rows:
        macro = "TRK_ENTRY_PAIR" if shape.swiglu else "TRK_ENTRY"
        lines.append(f"    {macro}(tile(kShape{order_tag(od)}, {t.args()}), {lo}, {hi})  // {name}")
    lines += [
        "};",
        "",
        "}  // namespace",
        "",
        f"int {_fn_name(shape)}(Plan *plan) {{",
        "    return register_entries(plan, kEntries, int(sizeof(kEntries) / sizeof(kEntries[0])));",
        "}",
        "",
        "}  // namespace trk",
        "",
    ]
    return "\n".join(lines)


def emit_module(shape: ShapeDecl) -> str:
    """Source of a variant module for one shape that the library has no compiled tables for:
    the shape's candidate tiles with rule-based token ranges (untuned), and the entry points
    trk_plan_load_module looks up (include/trk.h). Built at prepare time by jit.py."""
    text = emit(shape, tuned={})
    table_fn = _fn_name(shape)
    # the table's registration function stays internal to the module
    text = text.replace(f"int {table_fn}(Plan *plan) {{", "int module_table(Plan *plan) {")
    # (modules are compiled with hidden visibility: only these three entry points export)
    export = 'extern "C" __attribute__((visibility("default")))'
    text = text.replace("}  // namespace trk\n", "}  // namespace trk\n\n"
                        f"{export} int trk_module_register(trk::Plan *plan) {{\n"
                        "    return trk::module_table(plan);\n}\n"
                        f"{export} size_t trk_module_plan_size() {{ return sizeof(trk::Plan); }}\n"
                        f"{export} int trk_module_abi() {{ return TRK_ABI_VERSION; }}\n")
    return text.replace("// Generated by kernel-task_amd/factorized_inference/tilegen.py; do not edit.",
                        "// Variant module generated at prepare time by "
                        "kernel-task_amd/factorized_inference/jit.py (tilegen.emit_module).")


def emit_index(shapes: list[ShapeDecl]) -> str:
    lines = [
        "// Generated by kernel-task_amd/factorized_inference/tilegen.py; do not edit.",
        "// Registers the generated MFMA variant tables (one translation unit per shape).",
        '#include "trk_internal.h"',
        "",
        "namespace trk {",
        "",
    ]
    lines += [f"int {_fn_name(s)}(Plan *plan);" for s in shapes]
    lines += ["", "int mfma_register_generated(Plan *plan) {", "    int added = 0;"]
    lines += [f"    added += {_fn_name(s)}(plan);" for s in shapes]
    lines += ["    return added;", "}", "", "}  // namespace trk", ""]
    return "\n".join(lines)


def write_all(shapes: list[ShapeDecl] = DECLARED, out_dir: Path = GEN_DIR,
              all_candidates: bool = False, extended: bool = False) -> list[Path]:
    """Write one translation unit per shape plus the index; stale generated units are
    removed. Returns the written sources. all_candidates=True compiles every candidate with
    rule ranges (for the autotuner) instead of the tuned winners."""
    out_dir.mkdir(parents=True, exist_ok=True)
    tuned = load_tuned()
    written = []
    for s in shapes:
        p = out_dir / f"trk_gen_{s.key}.hip"
        text = emit(s, tuned, all_candidates, extended)
        if not p.exists() or p.read_text() != text:
            p.write_text(text)
        written.append(p)
    index = out_dir / "trk_gen_index.hip"
    text = emit_index(shapes)
    if not index.exists() or index.read_text() != text:
        index.write_text(text)
    written.append(index)
    keep = {p.name for p in written}
    for stale in out_dir.glob("trk_gen_*.hip"):
        if stale.name not in keep:
            stale.unlink()
    return written


def describe(shapes: list[ShapeDecl] = DECLARED) -> list[dict]:
    """Per shape: order, work and the tiles with their geometry (for reports and tests)."""
    out = []
    for s in shapes:
        order = choose_order(s)
        padded, unpadded = padded_work(s, order)
        out.append({"shape": s.key, "name": s.name, "order": order,
                    "padded_mac_per_token": padded, "mac_per_token": unpadded,
                    "tiles": [{"name": n, "order": od, "tile": asdict(t), "t_min": lo,
                               "t_max": hi, **geometry(s, od, t)}
                              for n, od, t, lo, hi in table(s)]})
    return out


if __name__ == "__main__":
    import sys

    for path in write_all(all_candidates="--all" in sys.argv[1:],
                          extended="--extended" in sys.argv[1:]):
        print(path)

#!/usr/bin/env python3
"""Writes bsattn_tile_loop.inc: the tile loop of one attention work unit of
bsattn_fwd_kernel as one gfx950 inline-assembly block, with every register
assigned here.

A workgroup of eight waves (two per SIMD) covers a (head, 128-query) unit.
Wave w owns queries 32(w & 3) .. +31 -- the B operand of
v_mfma_f32_32x32x16_bf16 -- and one 64-key half, w >> 2, of every 128-key
tile. Per tile j each wave issues, in one instruction stream,

  * the scores of the next tile, S(j+1) = K(j+1) Q^T (16 MFMAs),
  * the product of the previous one, O += V(j-1)^T P(j-1) (16 MFMAs),
  * the online softmax of S(j) into P(j) (about 145 VALU instructions),
  * its share of the HBM -> LDS loads of K(j+2) and V(j) (8 buffer loads),

so its VALU work runs beside its own MFMAs, and the partner wave on the
same SIMD fills the issue slots the first one leaves. Scores and weights are
double-buffered (S(j) and S(j+1), P(j-1) and P(j)), so none of these depends
on another inside an iteration; one barrier per tile orders the loads against
the LDS reads. The register budget is 256 per wave (two waves per SIMD): O,
Q^T and the LDS operand ring live in AGPRs (LDS reads land there directly and
MFMAs read them in place), scores and weights in VGPRs.

Registers (physical, fixed here):
  a[0:63]     O^T accumulators, O(db) = a[16db : +15]
  a[64:95]    Q^T operands, Q(s) = a[64 + 4s : +3]
  a[96:119]   ring of six LDS operands (K or V^T), 4 AGPRs each
  a[120:122]  lane constants of the ragged-tile paths (inputs)
  v[0:63]     scores, S(buf, kb) = v[32buf + 16kb : +15]
  v[64:95]    bf16 weights, P(buf, kc) = v[64 + 16buf + 4kc : +3]
  v[96:97]    m, l                      (outputs)
  v[98:121]   lane address offsets      (inputs, not modified)
  v[122:126]  softmax temporaries
  s[64:88]    resources, column indices, raise mask (clobbered)
With AGPRs in use the compiler gives a wave at most 128 VGPRs and 128 AGPRs
when two waves share a SIMD; this map uses 127 and 123
(the compiler needs one VGPR of its own beside the block).

Run `python3 gen_tile_loop.py` in this directory after editing; the generated
file is committed, and tests/test_tile_loop_gen.py checks it is current.
"""
from __future__ import annotations

import os
import struct
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "bsattn_tile_loop.inc")

WAVES = 8                      # per workgroup, two per SIMD
ROWS_PER_WAVE = 128 // WAVES   # rows of each K/V tile one wave loads
LOADS = ROWS_PER_WAVE // 4     # 4 rows (1 KiB) per buffer load


# ---------------------------------------------------------------- registers
def O(db):
    b = 16 * db
    return f"a[{b}:{b + 15}]"


def Q(s):
    b = 64 + 4 * s
    return f"a[{b}:{b + 3}]"


RING = 96
RING_N = 6
LOOKAHEAD = 4             # operands in flight; <= RING_N - 2 keeps a WAR gap


def ring(e, lo=0, n=4):
    b = RING + 4 * e + lo
    return f"a[{b}:{b + n - 1}]"


def S(buf, kb):
    b = 32 * buf + 16 * kb
    return f"v[{b}:{b + 15}]"


def s_reg(buf, i):
    """Register of score i (0..31, i = 16kb + r)."""
    return 32 * buf + i


def P(buf, kc):
    b = 64 + 16 * buf + 4 * kc
    return f"v[{b}:{b + 3}]"


def p_reg(buf, kc, e):
    return 64 + 16 * buf + 4 * kc + e


M, L = 96, 97
KA0 = 98        # K operand address for d-step s: v[98 + s]
VA0 = 106       # V^T operand address (p, db): v[106 + 4p + db]
DK0 = 114       # K load lane offsets: v[114 + i], i < LOADS
DV0 = DK0 + LOADS  # V load lane offsets
MX, SW, AL, LA, LB = 122, 123, 124, 125, 126
T4 = (MX, SW, AL, LB)    # temporaries of the fast softmax
N_VGPR = 127
KEYOFF = 120    # a120: kh*64 + 4hh            (input)
LANE16 = 121    # a121: 16 * lane              (input)
ROWB = 122      # a122: ROWS_PER_WAVE*w + lane/16  (input)

# SGPRs (clobbered)
KRS = "s[64:67]"   # buffer resource of the K tile being loaded
VRS = "s[68:71]"
SJ, SC0, SC1, SC2, ST0, ST1 = "s72", "s73", "s74", "s75", "s76", "s77"
RAISE = "s[78:79]"
EXSAVE = "s[82:83]"
COLP = "s[84:85]"
SIDX, SCOL = "s86", "s87"
SM0 = "s88"        # the caller's m0, restored at the end
SGPR_CLOBBERS = list(range(64, 89))

KSLOT = 32768          # bytes per K or V tile slot
WAIT_LGKM_MAX = 15


def fbits(x: float) -> str:
    return hex(struct.unpack("<I", struct.pack("<f", x))[0])


NEG_INF = "0xff800000"
M_INIT = fbits(-3.0e38)
SLACK = fbits(8.0)
SUM_LIMIT = fbits(256.0)   # 2^SLACK


# ------------------------------------------------------------- MFMA streams
class Op:
    """One LDS operand and the MFMA that reads it."""

    def __init__(self, reads, mfmas):
        self.reads = reads      # ds_read lines; {R0}/{R1} = ring registers
        self.mfmas = mfmas      # MFMA lines; {R} = the ring operand


def s_ops(sbuf, kslot):
    ops = []
    for s in range(8):
        for kb in range(2):
            off = kslot * KSLOT + kb * 8192
            reads = [f"ds_read_b128 {{R0}}, v{KA0 + s} offset:{off}"]
            dst = S(sbuf, kb)
            src_c = "0" if s == 0 else dst
            mf = [f"v_mfma_f32_32x32x16_bf16 {dst}, {{R}}, {Q(s)}, {src_c}"]
            ops.append(Op(reads, mf))
    return ops


def pv_ops(pbuf, vslot):
    ops = []
    for kc in range(4):
        for db in range(4):
            off = vslot * KSLOT + kc * 4096
            reads = [f"ds_read_b64_tr_b16 {{R0}}, v{VA0 + db} offset:{off}",
                     f"ds_read_b64_tr_b16 {{R1}}, v{VA0 + 4 + db} offset:{off}"]
            acc = O(db)
            mf = [f"v_mfma_f32_32x32x16_bf16 {acc}, {{R}}, {P(pbuf, kc)}, {acc}"]
            ops.append(Op(reads, mf))
    return ops


# ------------------------------------------------------------ softmax (VALU)
def softmax_ops(sb, pb):
    """Online softmax of S(sb) into P(pb), as VALU lines in a dependency-safe
    order. Updates m and l and leaves alpha in AL and the raise mask."""
    x = [s_reg(sb, i) for i in range(32)]
    ops = []
    # Row max: two max3 chains over 16 scores each, interleaved.
    chains = []
    for base, t in ((0, MX), (16, SW)):
        c = [f"v_max3_f32 v{t}, v{x[base]}, v{x[base + 1]}, v{x[base + 2]}"]
        for k in range(3, 15, 2):
            c.append(f"v_max3_f32 v{t}, v{t}, v{x[base + k]}, v{x[base + k + 1]}")
        c.append(f"v_max_f32 v{t}, v{t}, v{x[base + 15]}")
        chains.append(c)
    for a, b in zip(*chains):
        ops += [a, b]
    ops.append(f"v_max_f32 v{MX}, v{MX}, v{SW}")
    # The other half-wave holds the same query's other 32 keys.
    ops.append(f"v_mov_b32 v{SW}, v{MX}")
    ops.append("s_nop 1")
    ops.append(f"v_permlane32_swap_b32 v{MX}, v{SW}")
    ops.append(f"v_max_f32 v{MX}, v{MX}, v{SW}")
    # Lazy rescale: m moves only when the tile max exceeds it by > 2^8.
    ops.append(f"v_mul_f32 v{MX}, %[c], v{MX}")
    ops.append(f"v_add_f32 v{SW}, {SLACK}, v{M}")
    ops.append(f"v_max_f32 v{MX}, v{M}, v{MX}")
    ops.append(f"v_mov_b32 v{LA}, 0")
    ops.append(f"v_cmp_gt_f32 {RAISE}, v{MX}, v{SW}")
    ops.append(f"v_mov_b32 v{LB}, 0")
    ops.append(f"v_cndmask_b32 v{SW}, v{M}, v{MX}, {RAISE}")
    ops.append(f"v_sub_f32 v{AL}, v{M}, v{SW}")
    ops.append(f"v_mov_b32 v{M}, v{SW}")
    ops.append(f"v_exp_f32 v{AL}, v{AL}")
    # Weights 2^(s*c - m) in batches of four, packed to bf16 P and summed in
    # fp32 into l (two chains). The pack and the sums of batch b-1 follow
    # batch b's exponentials, a batch behind their producers. The sums are
    # plain VALU adds: v_dot2c over the packed weights would run on the
    # matrix pipeline, and there each one costs the MFMAs about as many
    # cycles as half a 32x32x16 product.
    prev = []
    for b in range(8):
        idx = list(range(4 * b, 4 * b + 4))
        for i in idx:
            ops.append(f"v_fma_f32 v{x[i]}, v{x[i]}, %[c], -v{M}")
        if b == 0:
            ops.append(f"v_mul_f32 v{L}, v{L}, v{AL}")
        for i in idx:
            ops.append(f"v_exp_f32 v{x[i]}, v{x[i]}")
        ops.extend(prev)
        prev = []
        # score i (= 16kb + r) -> P chunk kc = 2kb + (r >= 8), element r & 7
        for pair in range(2):
            i0 = 4 * b + 2 * pair
            kb, r = i0 // 16, i0 % 16
            kc = 2 * kb + (r >> 3)
            e = (r & 7) >> 1
            prev.append(f"v_cvt_pk_bf16_f32 v{p_reg(pb, kc, e)}, v{x[i0]}, v{x[i0 + 1]}")
            prev.append(f"v_add_f32 v{LA}, v{LA}, v{x[i0]}")
            prev.append(f"v_add_f32 v{LB}, v{LB}, v{x[i0 + 1]}")
    ops.extend(prev)
    ops.append(f"v_add_f32 v{LA}, v{LA}, v{LB}")
    ops.append(f"v_add_f32 v{L}, v{L}, v{LA}")
    return ops



def softmax_fast_ops(sb, pb):
    """The online softmax of S(sb) into P(pb) for a tile that does not move m
    (almost every tile after a row's first): weights 2^(s*c - m) with the
    current m, packed to P and summed in fp32 into LA (one chain), with the
    scores left in place. No row max: the raise mask marks the lanes whose
    weights sum to more than 2^8, or to NaN. Every tile softmax_ops would
    raise m for has a weight above 2^8 and is marked; for a marked tile the
    block end reruns softmax_ops on the kept scores, so m, P and l are what
    softmax_ops gives. Unmarked, P is bit for bit the same (alpha is 1
    there) and l differs only in the order of the sum; l += LA is left to
    the block end. The row max and the alpha update are the ~30 VALU
    instructions a tile saves: past ~4 VALU instructions per MFMA the two
    waves of a SIMD no longer hide their VALU work under the matrix cores."""
    x = [s_reg(sb, i) for i in range(32)]
    t = T4
    ops = []
    for b in range(8):
        for k in range(4):
            ops.append(f"v_fma_f32 v{t[k]}, v{x[4 * b + k]}, %[c], -v{M}")
        for k in range(4):
            ops.append(f"v_exp_f32 v{t[k]}, v{t[k]}")
        for pair in range(2):
            i0 = 4 * b + 2 * pair
            kb, r = i0 // 16, i0 % 16
            dst = p_reg(pb, 2 * kb + (r >> 3), (r & 7) >> 1)
            ops.append(f"v_cvt_pk_bf16_f32 v{dst}, v{t[2 * pair]}, v{t[2 * pair + 1]}")
            if b == 0 and pair == 0:   # the chain starts from the tile's first pair
                ops.append(f"v_add_f32 v{LA}, v{t[0]}, v{t[1]}")
            else:
                ops.append(f"v_add_f32 v{LA}, v{LA}, v{t[2 * pair]}")
                ops.append(f"v_add_f32 v{LA}, v{LA}, v{t[2 * pair + 1]}")
    ops.append(f"s_mov_b32 {ST0}, {SUM_LIMIT}")
    ops.append(f"v_cmp_nge_f32 {RAISE}, {ST0}, v{LA}")
    return ops

def mask_ops(sb, pb):
    """Scores of keys >= seq_len set to -inf (ragged last tile). Uses three
    registers of the weight buffer P(pb), which holds nothing live here;
    ST0 = seq_len - key0."""
    t_key, t_inf, t_lim, t_koff = (p_reg(pb, 0, e) for e in range(4))
    ops = ["s_nop 15", "s_nop 15", f"v_mov_b32 v{t_inf}, {NEG_INF}",
           f"v_mov_b32 v{t_lim}, {ST0}", f"v_accvgpr_read_b32 v{t_koff}, a{KEYOFF}"]
    for kb in range(2):
        for r in range(16):
            off = 32 * kb + 8 * (r >> 2) + (r & 3)
            reg = s_reg(sb, 16 * kb + r)
            ops.append(f"v_add_u32 v{t_key}, {off}, v{t_koff}")
            ops.append(f"v_cmp_le_i32 vcc, v{t_lim}, v{t_key}")
            ops.append(f"v_cndmask_b32 v{reg}, v{reg}, v{t_inf}, vcc")
    return ops


# ------------------------------------------------------------- DMA (loads)
def rsrc_setup(which, col, base_lo, base_hi, rec, stride128):
    """Lines building the buffer resource of one tile: base + col*128*rs,
    num_records = rec - col*128*rs."""
    b = 64 if which == "k" else 68
    return [f"s_mul_i32 {ST0}, {col}, {stride128}",
            f"s_add_u32 s{b}, {base_lo}, {ST0}",
            f"s_addc_u32 s{b + 1}, {base_hi}, 0",
            f"s_sub_u32 s{b + 2}, {rec}, {ST0}",
            f"s_mov_b32 s{b + 3}, 0x20000"]


def dma_lines(which, slot):
    """This wave's buffer loads of its rows of a K or V tile into the slot,
    in order: one M0 for the tile, the loads' instruction offsets (which
    apply to the LDS and to the global address alike) for their 1 KiB steps;
    the lane offsets v[DK0/DV0 + i] are lowered by the same 1024 i."""
    m0 = "%[m0k]" if which == "k" else "%[m0v]"
    base = DK0 if which == "k" else DV0
    rs = KRS if which == "k" else VRS
    out = []
    for i in range(LOADS):
        ld = f"buffer_load_dwordx4 v{base + i}, {rs}, 0 offen offset:{1024 * i} lds"
        out.append(([f"s_add_u32 m0, {m0}, {slot * KSLOT}", "s_nop 0"] if i == 0 else []) + [ld])
    return out


# --------------------------------------------------------------- scheduling
class Emitter:
    def __init__(self):
        self.lines = []

    def emit(self, *ls):
        self.lines.extend(ls)


def schedule(em, ops, valu, dmas, lookahead=LOOKAHEAD, pre=None, dma_at=None):
    """Interleaves the MFMA operand pipeline (ops), the VALU list and the DMA
    groups into one stream. Operand o's reads go into ring entry o % RING_N
    and are issued `lookahead` operands ahead of its MFMA; before that MFMA
    the wait leaves only the reads of later operands outstanding. VALU
    instructions (in list order) follow the MFMAs evenly; DMA groups evenly
    or by the cumulative counts dma_at[k] due after MFMA k."""
    assert lookahead <= RING_N - 2
    n_ops = len(ops)
    n_mfma = sum(len(o.mfmas) for o in ops)
    valu = list(valu)
    dmas = list(dmas)
    issued = []  # operand index of each ds_read issued, in order

    def issue(o):
        e = o % RING_N
        two = len(ops[o].reads) == 2
        for rd in ops[o].reads:
            em.emit(rd.replace("{R0}", ring(e, 0, 2 if two else 4)).replace("{R1}", ring(e, 2, 2)))
            issued.append(o)

    if n_mfma == 0:
        if pre:
            em.emit(*pre)
        while dmas or valu:
            if dmas:
                em.emit(*dmas.pop(0))
            for _ in range(max(1, len(valu) // max(1, len(dmas) + 1))):
                if valu:
                    em.emit(valu.pop(0))
        return
    # The first operands' reads go out before the block's scalar set-up, so
    # their latency overlaps it.
    nxt = 0
    for o in range(min(lookahead, n_ops)):
        issue(o)
        nxt = o + 1
    if pre:
        em.emit(*pre)
    total_valu, total_dma = len(valu), len(dmas)
    done_valu = done_dma = k = 0
    for o in range(n_ops):
        if nxt < n_ops:
            issue(nxt)
            nxt += 1
        later = min(sum(1 for x in issued if x > o), WAIT_LGKM_MAX)
        em.emit(f"s_waitcnt lgkmcnt({later})")
        for mf in ops[o].mfmas:
            em.emit(mf.replace("{R}", ring(o % RING_N)))
            k += 1
            want_valu = (k * total_valu) // n_mfma
            while done_valu < want_valu and valu:
                em.emit(valu.pop(0))
                done_valu += 1
            want_dma = dma_at[k - 1] if dma_at else (k * total_dma + n_mfma - 1) // n_mfma
            while done_dma < want_dma and dmas:
                em.emit(*dmas.pop(0))
                done_dma += 1
    while valu:
        em.emit(valu.pop(0))
    while dmas:
        em.emit(*dmas.pop(0))


# ------------------------------------------------------------------ blocks
def fixup_code(em, label, sb, pb):
    """Out of line, for a FULL/LAST block whose fast softmax marked lanes:
    softmax_ops reruns on the kept scores S(sb) -- row max, lazy raise,
    alpha, the weights into P(pb) again, l = alpha l + their sum -- and if m
    moved in any lane, O *= alpha once the P V MFMAs have drained. The
    rescale's temporaries are the scores, consumed by then."""
    em.emit(f"{label}_fixup:")
    em.emit(*softmax_ops(sb, pb))
    em.emit(f"s_cmp_lg_u64 {RAISE}, 0", f"s_cbranch_scc0 {label}_rescaled")
    t = [s_reg(sb, i) for i in range(4)]
    em.emit("s_nop 15", "s_nop 15", "s_nop 15", "s_nop 15")
    for db in range(4):
        for r0 in range(0, 16, 4):
            for r in range(4):
                em.emit(f"v_accvgpr_read_b32 v{t[r]}, a{16 * db + r0 + r}")
            for r in range(4):
                em.emit(f"v_mul_f32 v{t[r]}, v{t[r]}, v{AL}")
            for r in range(4):
                em.emit(f"v_accvgpr_write_b32 a{16 * db + r0 + r}, v{t[r]}")
    em.emit("s_nop 2", f"s_branch {label}_rescaled")


def column_load():
    """col[j + 3] (clamped to n - 1; ST1 holds n - 1) for the K load two blocks
    on, issued at the start of a FIRST/FULL block so that its latency passes
    under the block's MFMAs; the block-end lgkmcnt(0) collects it. An SMEM
    load may complete out of order with the LDS reads, so with it in flight
    lgkmcnt(N) still means "the reads before the last N are done" (it may
    also wait for the load): the block's counted waits stay exact for LDS."""
    return [f"s_add_u32 {SIDX}, {SJ}, 3",
            f"s_min_u32 {SIDX}, {SIDX}, {ST1}",
            f"s_lshl_b32 {SIDX}, {SIDX}, 2",
            f"s_load_dword {SCOL}, {COLP}, {SIDX}"]


def block_end(em, kind, p, label, sb):
    """The fast softmax's outcome (FULL/LAST: marked lanes branch to the
    fixup, otherwise l += the tile's sum), waits (which also collect the
    column load of FIRST/FULL blocks), ragged V zeroing (LAST/ONLY),
    barrier, column shift."""
    if kind in ("FULL", "LAST"):
        # s_nop: the raise mask may have been written by the block's last VALU
        # instruction.
        em.emit("s_nop 4",
                f"s_cmp_lg_u64 {RAISE}, 0",
                f"s_cbranch_scc1 {label}_fixup",
                f"v_add_f32 v{L}, v{L}, v{LA}",
                f"{label}_rescaled:")
    em.emit("s_waitcnt vmcnt(0) lgkmcnt(0)")
    if kind in ("LAST", "ONLY"):
        # Rows >= seq_len of V(j) are zeroed after they land (0 * NaN is NaN):
        # this wave's rows ROWB + 4i. Temporaries: the consumed scores S(sb).
        z = s_reg(sb, 0)
        t_addr, t_row, t_rowb = s_reg(sb, 4), s_reg(sb, 5), s_reg(sb, 6)
        em.emit("s_cmp_eq_u32 %[ragged], 0",
                f"s_cbranch_scc1 {label}_nozero",
                f"s_mul_i32 {ST0}, {SC0}, 128",
                f"s_sub_u32 {ST0}, %[seq], {ST0}",
                f"v_mov_b32 v{z}, 0", f"v_mov_b32 v{z + 1}, 0",
                f"v_mov_b32 v{z + 2}, 0", f"v_mov_b32 v{z + 3}, 0",
                f"s_add_u32 {ST1}, %[m0v], {p * KSLOT}",
                f"v_accvgpr_read_b32 v{t_addr}, a{LANE16}",
                f"v_accvgpr_read_b32 v{t_rowb}, a{ROWB}",
                f"v_add_u32 v{t_addr}, {ST1}, v{t_addr}",
                f"s_mov_b64 {EXSAVE}, exec")
        for i in range(LOADS):
            em.emit(f"v_add_u32 v{t_row}, {4 * i}, v{t_rowb}",
                    f"v_cmp_le_i32 vcc, {ST0}, v{t_row}",
                    "s_and_b64 exec, exec, vcc",
                    f"ds_write_b128 v{t_addr}, v[{z}:{z + 3}] offset:{1024 * i}",
                    f"s_mov_b64 exec, {EXSAVE}")
        em.emit("s_waitcnt lgkmcnt(0)", f"{label}_nozero:")
    em.emit("s_barrier")
    if kind in ("FIRST", "FULL"):
        em.emit(f"s_mov_b32 {SC0}, {SC1}", f"s_mov_b32 {SC1}, {SC2}", f"s_mov_b32 {SC2}, {SCOL}")


def spread(n, lo, hi, total):
    """Cumulative counts placing `total` items evenly after MFMAs lo..hi-1 of
    n (none before lo; all placed by hi)."""
    out = []
    for k in range(1, n + 1):
        if k <= lo:
            out.append(0)
        elif k >= hi:
            out.append(total)
        else:
            out.append(((k - lo) * total) // (hi - lo))
    return out


def dma_quota(n_mfma, n_dma):
    """The block's HBM -> LDS loads are issued over its first half, so they
    have half a block more to land before the block-end wait than if spread
    over the whole block (measured 1-3% faster at cfg3 and cfg4)."""
    return spread(n_mfma, 0, max(1, n_mfma // 2), n_dma)


def gen_block(em, kind, p, label, out_of_line):
    """kind: FIRST (j = 0, n > 1), FULL (0 < j < n - 1), LAST (j = n - 1 > 0),
    ONLY (n = 1). p = j & 1."""
    sc, sn = p, 1 - p
    pn, pp = p, 1 - p
    has_s = kind in ("FIRST", "FULL")
    has_pv = kind in ("FULL", "LAST")
    pre = []
    # K(j + 2) from column SC2 (an empty resource unless j + 2 < n), V(j) from SC0.
    kd = []
    if has_s:
        pre += rsrc_setup("k", SC2, "%[kb_lo]", "%[kb_hi]", "%[krec]", "%[kstep]")
        pre += [f"s_add_u32 {ST1}, {SJ}, 2",
                f"s_cmp_lt_u32 {ST1}, %[n]",
                "s_cselect_b32 s66, s66, 0"]
        kd = dma_lines("k", p)
    pre += rsrc_setup("v", SC0, "%[vb_lo]", "%[vb_hi]", "%[vrec]", "%[vstep]")
    pre += [f"s_sub_u32 {ST1}, %[n], 1"]      # n - 1, the column-load clamp
    if has_s:
        pre += column_load()
    vd = dma_lines("v", p)
    dmas = kd + vd     # each tile's loads together: they share its M0
    sops = s_ops(sn, sn) if has_s else []
    pops = pv_ops(pp, pp) if has_pv else []
    valu = softmax_fast_ops(sc, pn) if has_pv else softmax_ops(sc, pn)
    ops = sops + pops
    dma_at = dma_quota(len(ops), len(dmas)) if ops else None
    if kind in ("LAST", "ONLY"):
        pre += ["s_cmp_eq_u32 %[ragged], 0", f"s_cbranch_scc1 {label}_nomask",
                f"s_mul_i32 {ST0}, {SC0}, 128", f"s_sub_u32 {ST0}, %[seq], {ST0}"]
        pre += mask_ops(sc, pn)
        pre += [f"{label}_nomask:"]
    schedule(em, ops, valu, dmas, pre=pre, dma_at=dma_at)
    if has_s and not has_pv:
        # S(j + 1) is read by the next block's VALU: let the MFMAs drain.
        em.emit("s_nop 15", "s_nop 15", "s_nop 7")
    block_end(em, kind, p, label, sc)
    if has_pv:
        sub = Emitter()
        fixup_code(sub, label, sc, pn)
        out_of_line.extend(sub.lines)


def gen_prologue(em):
    em.emit(f"s_mov_b32 {SM0}, m0",
            f"v_mov_b32 v{M}, {M_INIT}", f"v_mov_b32 v{L}, 0",
            f"s_mov_b32 {SC0}, %[c0]", f"s_mov_b32 {SC1}, %[c1]", f"s_mov_b32 {SC2}, %[c2]",
            "s_mov_b32 s84, %[colp_lo]", "s_mov_b32 s85, %[colp_hi]",
            f"s_mov_b32 {SJ}, 0")
    # Q^T operands from the Q slot: address = K address + qoff. Scores buffer
    # 1 holds the addresses (the FIRST block writes it first).
    for s in range(8):
        em.emit(f"v_add_u32 v{s_reg(1, s)}, %[qoff], v{KA0 + s}")
    for s in range(8):
        em.emit(f"ds_read_b128 {Q(s)}, v{s_reg(1, s)}")
    em.emit("s_waitcnt lgkmcnt(0)")
    # K(1) -> K slot 1 when n > 1
    pre = rsrc_setup("k", SC1, "%[kb_lo]", "%[kb_hi]", "%[krec]", "%[kstep]")
    pre += ["s_cmp_gt_u32 %[n], 1", "s_cselect_b32 s66, s66, 0"]
    zeros = [f"v_accvgpr_write_b32 a{i}, 0" for i in range(64)]
    schedule(em, s_ops(0, 0), zeros, dma_lines("k", 1), pre=pre)
    em.emit("s_nop 15", "s_nop 15", "s_nop 7",
            "s_waitcnt vmcnt(0) lgkmcnt(0)", "s_barrier")


def gen_epilogue(em, p):
    schedule(em, pv_ops(p, p), [], [])


def generate():
    em = Emitter()
    ool = []
    gen_prologue(em)
    em.emit("s_cmp_eq_u32 %[n], 1", "s_cbranch_scc1 L_only_%=")
    gen_block(em, "FIRST", 0, "L_first_%=", ool)
    em.emit(f"s_mov_b32 {SJ}, 1")
    em.emit("L_odd_%=:")
    em.emit(f"s_add_u32 {ST0}, {SJ}, 1", f"s_cmp_eq_u32 {ST0}, %[n]",
            "s_cbranch_scc1 L_last1_%=")
    gen_block(em, "FULL", 1, "L_full1_%=", ool)
    em.emit(f"s_add_u32 {SJ}, {SJ}, 1")
    em.emit(f"s_add_u32 {ST0}, {SJ}, 1", f"s_cmp_eq_u32 {ST0}, %[n]",
            "s_cbranch_scc1 L_last0_%=")
    gen_block(em, "FULL", 0, "L_full0_%=", ool)
    em.emit(f"s_add_u32 {SJ}, {SJ}, 1", "s_branch L_odd_%=")
    em.emit("L_last1_%=:")
    gen_block(em, "LAST", 1, "L_lastb1_%=", ool)
    gen_epilogue(em, 1)
    em.emit("s_branch L_end_%=")
    em.emit("L_last0_%=:")
    gen_block(em, "LAST", 0, "L_lastb0_%=", ool)
    gen_epilogue(em, 0)
    em.emit("s_branch L_end_%=")
    em.emit("L_only_%=:")
    gen_block(em, "ONLY", 0, "L_onlyb_%=", ool)
    gen_epilogue(em, 0)
    em.emit("s_branch L_end_%=")
    em.lines.extend(ool)
    em.emit("L_end_%=:", "s_nop 15", "s_nop 15", "s_nop 7", f"s_mov_b32 m0, {SM0}")
    return em.lines


def clobbers():
    regs = [f"v{i}" for i in range(0, 96)]
    regs += [f"v{i}" for i in range(MX, N_VGPR)]
    regs += [f"a{i}" for i in range(64, RING + 4 * RING_N)]
    regs += [f"s{i}" for i in SGPR_CLOBBERS]
    regs += ["vcc", "scc", "memory"]
    return regs


def render() -> str:
    lines = generate()
    body = "\n".join('  "' + ln.replace('"', '\\"') + '\\n"' for ln in lines)
    cl = ", ".join(f'"{r}"' for r in clobbers())
    n_mfma = sum(1 for ln in lines if ln.startswith("v_mfma"))
    return (
        "// Generated by gen_tile_loop.py -- do not edit; regenerate instead.\n"
        f"// {len(lines)} lines, {n_mfma} MFMAs.\n"
        f"#define H3_TILE_LOOP_WAVES {WAVES}\n"
        f"#define H3_TILE_LOOP_ROWS_PER_WAVE {ROWS_PER_WAVE}\n"
        "#define H3_TILE_LOOP_ASM \\\n" + body.replace("\n", " \\\n") + "\n\n"
        "#define H3_TILE_LOOP_CLOBBERS " + cl + "\n")


def main() -> int:
    text = render()
    if len(sys.argv) > 1 and sys.argv[1] == "--check":
        cur = open(OUT).read() if os.path.exists(OUT) else ""
        return 0 if cur == text else 1
    with open(OUT, "w") as f:
        f.write(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())

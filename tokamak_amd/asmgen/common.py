"""Helpers shared by the attention assembly generators: per-lane integer arithmetic that is
both emitted and evaluated (so every address formula is checked against the HIP kernels'
index formulas at generation time), the LDS chunk swizzle, and the per-lane LDS offsets of
the two operand read patterns used by every attention kernel:

* row reads (ds_read_b128): row l32 of a 32-row block, 8 head-dim elements (ks*16 + hi*8 ..)
  -- the A operand K (forward S^T = K Q^T), Q / dO (dK/dV kernel), K / V (dQ kernel);
* transposed reads (ds_read_b64_tr_b16 pairs): the A operand V^T / dO^T / Q^T / K^T, rows
  ks*16 + tt*8 + hi*4 + trow, columns db*32 + tcol, in the k-slot order of an MFMA
  accumulator used in place as the other operand.

Tiles in LDS are row-major, 256 bytes per row (D = 128), 16-byte chunk c of row r stored at
slot c ^ swz(r).
"""
from __future__ import annotations

import numpy as np

from .gfx950 import Prog, S, V, sr, vr

ROWB = 256


def swz(r):
    return ((r & 3) << 2) | ((r >> 2) & 3)


class Lanes:
    """Emits integer VALU ops on per-lane values and evaluates them over 4 waves x 64 lanes
    (numpy int64 arrays of 256 entries), so the prologue address arithmetic can be checked."""

    def __init__(self, p: Prog, ldb: int):
        self.p = p
        self.val = {}
        tid = np.arange(256, dtype=np.int64)
        self.val[0] = tid  # v0 = workitem id
        self.wave = tid >> 6
        self.ldb = ldb

    def _set(self, d, x):
        self.val[d] = np.asarray(x, dtype=np.int64) & 0xFFFFFFFF

    def op2(self, mnem, d, a, b, fn):
        """d = fn(a, b); a, b are VGPR indices or ('k', const) / ('s', sgpr, value)."""
        def txt(x):
            if isinstance(x, int):
                return vr(x)
            if x[0] == "k":
                return str(x[1])
            return sr(x[1])

        def v(x):
            if isinstance(x, int):
                return self.val[x]
            if x[0] == "k":
                return np.full(256, x[1], dtype=np.int64)
            return x[2]  # per-wave scalar values (array of 256)

        reads = []
        for x in (a, b):
            if isinstance(x, int):
                reads += V(x)
            elif x[0] == "s":
                reads += S(x[1])
        self.p.valu(f"{mnem} {vr(d)}, {txt(a)}, {txt(b)}", reads, V(d))
        self._set(d, fn(v(a), v(b)))

    def and_(self, d, a, b): self.op2("v_and_b32", d, a, b, lambda x, y: x & y)
    def or_(self, d, a, b): self.op2("v_or_b32", d, a, b, lambda x, y: x | y)
    def xor(self, d, a, b): self.op2("v_xor_b32", d, a, b, lambda x, y: x ^ y)
    def add(self, d, a, b): self.op2("v_add_u32", d, a, b, lambda x, y: x + y)
    def shr(self, d, sh, a): self.op2("v_lshrrev_b32", d, sh, a, lambda s_, x: x >> s_)
    def shl(self, d, sh, a): self.op2("v_lshlrev_b32", d, sh, a, lambda s_, x: x << s_)
    def mul(self, d, a, b): self.op2("v_mul_lo_u32", d, a, b, lambda x, y: x * y)

    def k(self, c):
        return ("k", c)

    def s(self, sgpr, per_wave):
        """An SGPR operand whose value is per_wave[wave]."""
        return ("s", sgpr, np.asarray(per_wave, dtype=np.int64)[self.wave])



def row_read_offsets(L: Lanes, koff: int, lanes, scratch):
    """koff[ks] = l32*256 + (((2ks + hi) ^ swz(l32)) << 4), ks = 0..7."""
    LANE, L32, HI = lanes
    TA, TB, TC = scratch
    L.and_(TA, L.k(3), L32)
    L.shl(TA, L.k(2), TA)
    L.shr(TB, L.k(2), L32)
    L.and_(TB, L.k(3), TB)
    L.or_(TA, TA, TB)                               # swz(l32)
    L.shl(TB, L.k(8), L32)                          # l32*256
    for ks in range(8):
        L.add(TC, HI, L.k(2 * ks))
        L.xor(TC, TC, TA)
        L.shl(TC, L.k(4), TC)
        L.add(koff + ks, TC, TB)
    tid = np.arange(256)
    lane = tid & 63
    l32, hi = lane & 31, lane >> 5
    fk = np.vectorize(swz)(l32)
    for ks in range(8):
        ref = l32 * ROWB + (((ks * 2 + hi) ^ fk) << 4)
        assert np.array_equal(L.val[koff + ks], ref), f"row read offset {ks}"


def tr_read_offsets(L: Lanes, voff: int, lanes, scratch):
    """voff[tt*4 + db]: byte offset of the transposed read for rows tt*8 + hi*4 + trow and
    columns db*32 + tcol (trow = (lane&15)>>2, tcol = ((lane>>4)&1)*16 + (lane&3)*4)."""
    LANE, L32, HI = lanes
    TA, TB, TC, TROW, C1, E, RB = scratch
    # row = tt*8 + hi*4 + trow; off = row*256 + (((4db + c1) ^ (4trow + 2tt + hi)) << 4) + e
    # with c1 = ((lane>>4)&1)*2 + ((lane&3)>>1), e = (lane&1)*8
    L.and_(TROW, L.k(15), LANE)
    L.shr(TROW, L.k(2), TROW)
    L.shr(C1, L.k(4), LANE)
    L.and_(C1, L.k(1), C1)
    L.shl(C1, L.k(1), C1)
    L.and_(TC, L.k(3), LANE)
    L.shr(TC, L.k(1), TC)
    L.or_(C1, C1, TC)
    L.and_(E, L.k(1), LANE)
    L.shl(E, L.k(3), E)
    L.shl(TA, L.k(2), HI)
    L.add(RB, TA, TROW)                             # hi*4 + trow
    L.shl(TB, L.k(2), TROW)
    L.add(TB, TB, HI)                               # 4trow + hi
    for tt in range(2):
        for db in range(4):
            L.add(TC, C1, L.k(4 * db))
            L.add(TA, TB, L.k(2 * tt))
            L.xor(TC, TC, TA)
            L.shl(TC, L.k(4), TC)
            L.add(TC, TC, E)
            L.add(TA, RB, L.k(8 * tt))
            L.shl(TA, L.k(8), TA)
            L.add(voff + tt * 4 + db, TC, TA)
    tid = np.arange(256)
    lane = tid & 63
    hi = (lane & 63) >> 5
    trow = (lane & 15) >> 2
    tcol = ((lane >> 4) & 1) * 16 + (lane & 3) * 4
    for tt in range(2):
        row = tt * 8 + hi * 4 + trow
        for db in range(4):
            d = db * 32 + tcol
            ref = row * ROWB + (((d >> 3) ^ np.vectorize(swz)(row)) << 4) + (d & 7) * 2
            assert np.array_equal(L.val[voff + tt * 4 + db], ref), f"tr read offset {tt} {db}"


def lane_basics(L: Lanes, regs):
    """lane = v0 & 63, l32 = v0 & 31, hi = lane >> 5 into regs (LANE, L32, HI)."""
    LANE, L32, HI = regs
    L.and_(LANE, L.k(63), 0)
    L.and_(L32, L.k(31), 0)
    L.shr(HI, L.k(5), LANE)


def xcd_slot(p: Prog, wg: int, nwg: int, t0: int, t1: int):
    """s[wg] := the workgroup's place among the NWG places of a round, dealt XCD by XCD.

    The dispatcher hands workgroups to the 8 XCDs in turn (workgroup w to XCD w % 8), so XCD
    x runs workgroups x, x+8, x+16, ...; they take the places x*q + min(x, r) + 0, 1, ...
    (q = NWG / 8, r = NWG % 8).  Consecutive places then run on one XCD and share its L2: the
    items of a round that read the same rows (the blocks of one head) fetch them from HBM
    once.  The map is a permutation of 0 .. NWG-1 for every NWG."""
    sal = p.salu
    sal(f"s_and_b32 {sr(t0)}, {sr(wg)}, 7", S(wg), S(t0))
    sal(f"s_lshr_b32 {sr(t1)}, {sr(nwg)}, 3", S(nwg), S(t1))
    sal(f"s_mul_i32 {sr(t1)}, {sr(t1)}, {sr(t0)}", S(t1) + S(t0), S(t1))
    sal(f"s_lshr_b32 {sr(wg)}, {sr(wg)}, 3", S(wg), S(wg))
    sal(f"s_add_u32 {sr(wg)}, {sr(wg)}, {sr(t1)}", S(wg) + S(t1), S(wg))
    sal(f"s_and_b32 {sr(t1)}, {sr(nwg)}, 7", S(nwg), S(t1))
    sal(f"s_min_u32 {sr(t1)}, {sr(t1)}, {sr(t0)}", S(t1) + S(t0), S(t1))
    sal(f"s_add_u32 {sr(wg)}, {sr(wg)}, {sr(t1)}", S(wg) + S(t1), S(wg))


def xcd_slots(nwg: int) -> list:
    """The places xcd_slot gives workgroups 0 .. nwg-1."""
    q, r = nwg // 8, nwg % 8
    return [(w % 8) * q + min(w % 8, r) + w // 8 for w in range(nwg)]

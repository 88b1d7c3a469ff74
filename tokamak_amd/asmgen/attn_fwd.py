"""Generator of the gfx950 assembly FlashAttention forward, D = 128, fp16 (causal or not,
optional kv_len).

Contract: identical to fa_fwd_kernel (tokamak_amd/csrc/attn_fwd.hip), which replaces the
reference's k_gqa_flash_attn_tc_fwd<128> (src/tkm_gpu.cu:302-438): packed
qkv [B][S][(Hq+2Hkv)*128] fp16 in; O [B][S][Hq*128] fp16 and LSE [B][Hq][S] fp32 (natural
log of the scaled scores) out; q-head h reads kv-head h/(Hq/Hkv); key j is visible from
query i iff j < kv_len[b] and (!causal || j <= i).

Work decomposition: grid (Hq, B, n_qblk), one workgroup = 4 waves = one (batch, q-head,
block of 256 query rows); one wave per SIMD, so each wave owns 256 VGPRs and 256 AGPRs.
Causal launches walk the query blocks heaviest first (z = 0 is the last block).  A wave keeps
its 64 query rows of Q, prescaled by scale*log2(e) and rounded to fp16, in AGPRs (two 32-row
blocks: every K or V operand read from LDS feeds two MFMAs) and its O accumulators in AGPRs.
K/V tiles of 64 keys move HBM -> LDS by buffer DMA (rows past the valid range read as zero),
double-buffered, row-major with the XOR chunk swizzle chunk' = chunk ^ (4*(row&3) + (row>>2&3)).

Per tile t a wave runs a fixed 64-slot schedule (one v_mfma_f32_32x32x16_f16 per slot):
  slots  0..31   S(t+1) = K(t+1) Q^T into the free score register set;
  slots 32..63   O^T += V(t)^T P(t)^T, V^T read from the row-major tile by ds_read_b64_tr_b16;
and the softmax of S(t) runs between the MFMAs of slots 0..55: P = exp2(S) (the accumulator
starts at -m, m = the row max of the first tile in log2 units), packed to fp16 for the MFMA,
row sums accumulated in fp32 by v_add_f32 (v_dot2c would share the matrix pipe and stall the
MFMA stream).  Operand reads are issued LK / LV slots ahead of their first MFMA; the eight
DMA instructions of K(t+2) and V(t+1) go one every four slots (the vector memory path moves
about 64 B/clk per CU; a burst stalls the wave's issue).  The last active tile of a wave (the only one that can need
a mask: causal diagonal or kv_len edge), the first tile and idle tiles of shorter waves run
unpipelined.  A P that overflows fp16 (the row max grew by more than 2^15 after the first
tile) is detected from the per-tile partial row sums (any P above 65504 makes its lane's
partial sum exceed 65504); the workgroup then computes the exact row max in an extra pass and
repeats the main loop with m fixed to it.

The generated code's per-lane address arithmetic is evaluated here over all 4 x 64 lanes and
checked against the HIP kernel's index formulas before any text is written.
"""
from __future__ import annotations

import numpy as np

from .common import Lanes, lane_basics, row_read_offsets, swz, tr_read_offsets
from .gfx950 import (A, BRANCH, DMA, PERMLANE, Prog, S, V, VALU, ar, kernel_text, sr, vr)

NAME = "tkm_fa_fwd_d128_f16"
D = 128
ROWB = D * 2            # bytes per K/V row in LDS
TILE = 64 * ROWB        # one 64-key tile
LDS_K = (0, TILE)       # K buffers
LDS_V = (2 * TILE, 3 * TILE)
LDS_FLAG = 4 * TILE
LDS_EPI = 4 * TILE + 16     # per wave: 32 rows of 272 B staging O for the store
EPI_ROW = 272               # 256 B + 16 B pad: rows 16 B apart in the banks
EPI_WAVE = 32 * EPI_ROW
LDS_BYTES = LDS_EPI + 4 * EPI_WAVE
LK = 4                  # slots between a K read and its first MFMA
LV = 4
NKB = 4                 # K operand registers in rotation (need 2*NKB > LK + 2)
NVB = 4
MFMA = "v_mfma_f32_32x32x16_f16"

# kernel arguments (byte offsets in the kernarg segment)
ARGS = [(0, 8, "ptr"), (8, 8, "ptr"), (16, 8, "ptr"), (24, 8, "ptr")] + \
       [(32 + 4 * i, 4, "val") for i in range(10)]
KERNARG_BYTES = 72

# ---- SGPRs
S_KARG = 0      # s[0:1]
S_H, S_B, S_Z = 2, 3, 4
S_ARG = 8       # s[8:23]: qkv, out, lse, kvlen, S, Hq, Hkv, sl2, causal, n_qblk, ldb, magic
S_QKV, S_OUT, S_LSE, S_KVLEN = 8, 10, 12, 14
S_SEQ, S_HQ, S_HKV, S_SL2, S_CAUSAL, S_NQBLK, S_LDB, S_MAGIC = 16, 17, 18, 19, 20, 21, 22, 23
S_GRP1, S_LDO = 24, 25
S_QBLK, S_KVH, S_KVL, S_KVEND, S_NT, S_NPLAIN, S_NACT, S_Q0, S_WAVE = 26, 27, 28, 29, 30, 31, 32, 33, 34
S_BQKV = 36     # s[36:37]
S_KB = 38       # s[38:39]
S_VB = 40       # s[40:41]
S_RQ = 44       # s[44:47] Q descriptor, later O
S_RK = 48       # s[48:51]
S_RV = 52       # s[52:55]
S_T = 56
S_PASS = 57
S_LDSW = 58     # this wave's DMA row offset in a tile (bytes)
S_RL = 60       # s[60:63] LSE descriptor
S_TMP = 64      # s64..s79 temporaries
S_EXEC = 80     # s[80:81]
S_C0, S_C1 = 82, 84  # s[82:83], s[84:85] compare results
NEXT_FREE_SGPR = 88

# ---- VGPRs
V_SET = (0, 64)         # score register sets; block (kb, qb) at +(kb*2+qb)*16
V_CINIT = 128           # -m replicated: qb*16 + r
V_P = 160               # P[qb][ks] at 160 + (qb*4+ks)*4
V_KBUF = 192
V_VBUF = V_KBUF + 4 * NKB
V_KOFF = V_VBUF + 4 * NVB   # 8
V_VOFF = V_KOFF + 8         # 8: tt*4 + db
V_DOFF = V_VOFF + 8         # 4
V_LSUM = V_DOFF + 4         # row sums (fp32 P, this lane's half of the keys), per qb
V_LT = V_LSUM + 2           # this tile's partial sums: qb*2 + (0, 1)
V_LMAX = V_LT + 4           # largest per-tile partial sum (fp16 overflow check), per qb
V_NINF = V_LMAX + 2
V_TMP = V_NINF + 1          # 1
V_L32 = V_TMP + 1           # lane & 31
V_HI4 = V_TMP + 2           # 4 * (lane >> 5)
assert V_HI4 < 256
# prologue scratch (score set 1 region, free until the first S(1))
V_PT = 64
# temporaries of the prologue and the epilogue, when P is free
V_T = V_P + 4               # 5 registers

# ---- AGPRs
A_O = 0                 # o[db][qb] at (db*2+qb)*16
A_Q = 128               # q[qb][ks] at 128 + (qb*8+ks)*4


def sblk(J, kb, qb):
    return V_SET[J] + (kb * 2 + qb) * 16


def build(check_ldb: int = 12288) -> str:
    p = Prog()
    # ------------------------------------------------------------------ prologue: scalars
    p.smem(f"s_load_dwordx16 {sr(S_ARG, 16)}, {sr(S_KARG, 2)}, 0x0", S(S_ARG, 16), S(S_KARG, 2))
    p.smem(f"s_load_dwordx2 {sr(S_GRP1, 2)}, {sr(S_KARG, 2)}, 0x40", S(S_GRP1, 2), S(S_KARG, 2))
    L = Lanes(p, check_ldb)
    # wave index (needs only v0)
    L.shr(V_PT + 0, L.k(6), 0)
    p.readlane(f"v_readfirstlane_b32 {sr(S_WAVE)}, {vr(V_PT + 0)}", V(V_PT + 0), S(S_WAVE))
    p.waitcnt(lgkm=0)
    sal = p.salu
    # qblk = causal ? n_qblk - 1 - z : z
    sal(f"s_sub_u32 {sr(S_QBLK)}, {sr(S_NQBLK)}, 1", S(S_NQBLK), S(S_QBLK))
    sal(f"s_sub_u32 {sr(S_QBLK)}, {sr(S_QBLK)}, {sr(S_Z)}", S(S_QBLK) + S(S_Z), S(S_QBLK))
    sal(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(S_QBLK)}, {sr(S_Z)}, {sr(S_QBLK)}", S(S_Z) + S(S_QBLK) + [("scc", 0)], S(S_QBLK))
    # kvh = group == 1 ? h : mulhi(h, magic)
    sal(f"s_mul_hi_u32 {sr(S_KVH)}, {sr(S_H)}, {sr(S_MAGIC)}", S(S_H) + S(S_MAGIC), S(S_KVH))
    sal(f"s_cmp_eq_u32 {sr(S_GRP1)}, 0", S(S_GRP1), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(S_KVH)}, {sr(S_KVH)}, {sr(S_H)}", S(S_KVH) + S(S_H) + [("scc", 0)], S(S_KVH))
    # kvl = clamp(kv_len ? kv_len[b] : S, 0, S)
    sal(f"s_mov_b32 {sr(S_KVL)}, {sr(S_SEQ)}", S(S_SEQ), S(S_KVL))
    sal(f"s_cmp_eq_u64 {sr(S_KVLEN, 2)}, 0", S(S_KVLEN, 2), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lkvl_done", [("scc", 0)])
    sal(f"s_lshl_b32 {sr(S_TMP)}, {sr(S_B)}, 2", S(S_B), S(S_TMP))
    p.smem(f"s_load_dword {sr(S_KVL)}, {sr(S_KVLEN, 2)}, {sr(S_TMP)}", S(S_KVL), S(S_KVLEN, 2) + S(S_TMP))
    p.waitcnt(lgkm=0)
    sal(f"s_max_i32 {sr(S_KVL)}, {sr(S_KVL)}, 0", S(S_KVL), S(S_KVL))
    sal(f"s_min_i32 {sr(S_KVL)}, {sr(S_KVL)}, {sr(S_SEQ)}", S(S_KVL) + S(S_SEQ), S(S_KVL))
    p.label(".Lkvl_done")
    T0, T1, T2, T3 = S_TMP, S_TMP + 1, S_TMP + 2, S_TMP + 3
    # q0 = qblk*256 + wave*64
    sal(f"s_lshl_b32 {sr(S_Q0)}, {sr(S_QBLK)}, 8", S(S_QBLK), S(S_Q0))
    sal(f"s_lshl_b32 {sr(T0)}, {sr(S_WAVE)}, 6", S(S_WAVE), S(T0))
    sal(f"s_add_u32 {sr(S_Q0)}, {sr(S_Q0)}, {sr(T0)}", S(S_Q0) + S(T0), S(S_Q0))
    # kv_end = causal ? min(kvl, qblk*256 + 256) : kvl
    sal(f"s_lshl_b32 {sr(T0)}, {sr(S_QBLK)}, 8", S(S_QBLK), S(T0))
    sal(f"s_add_u32 {sr(T0)}, {sr(T0)}, 0x100", S(T0), S(T0))
    sal(f"s_min_i32 {sr(T0)}, {sr(T0)}, {sr(S_KVL)}", S(T0) + S(S_KVL), S(T0))
    sal(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(S_KVEND)}, {sr(S_KVL)}, {sr(T0)}", S(S_KVL) + S(T0) + [("scc", 0)], S(S_KVEND))
    # ntiles = (kv_end + 63) >> 6
    sal(f"s_add_u32 {sr(T0)}, {sr(S_KVEND)}, 63", S(S_KVEND), S(T0))
    sal(f"s_lshr_b32 {sr(S_NT)}, {sr(T0)}, 6", S(T0), S(S_NT))
    # n_plain = min(kvl >> 6, causal ? q0 >> 6 : ntiles)
    sal(f"s_lshr_b32 {sr(T0)}, {sr(S_KVL)}, 6", S(S_KVL), S(T0))
    sal(f"s_lshr_b32 {sr(T1)}, {sr(S_Q0)}, 6", S(S_Q0), S(T1))
    sal(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(T1)}, {sr(S_NT)}, {sr(T1)}", S(S_NT) + S(T1) + [("scc", 0)], S(T1))
    sal(f"s_min_u32 {sr(S_NPLAIN)}, {sr(T0)}, {sr(T1)}", S(T0) + S(T1), S(S_NPLAIN))
    # n_act = causal ? min(ntiles, (q0 >> 6) + 1) : ntiles
    sal(f"s_lshr_b32 {sr(T0)}, {sr(S_Q0)}, 6", S(S_Q0), S(T0))
    sal(f"s_add_u32 {sr(T0)}, {sr(T0)}, 1", S(T0), S(T0))
    sal(f"s_min_u32 {sr(T0)}, {sr(T0)}, {sr(S_NT)}", S(T0) + S(S_NT), S(T0))
    sal(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(S_NACT)}, {sr(S_NT)}, {sr(T0)}", S(S_NT) + S(T0) + [("scc", 0)], S(S_NACT))
    # bqkv = qkv + b*S*ldb
    sal(f"s_mul_i32 {sr(T0)}, {sr(S_B)}, {sr(S_SEQ)}", S(S_B) + S(S_SEQ), S(T0))
    sal(f"s_mul_i32 {sr(T1)}, {sr(T0)}, {sr(S_LDB)}", S(T0) + S(S_LDB), S(T1))
    sal(f"s_mul_hi_u32 {sr(T2)}, {sr(T0)}, {sr(S_LDB)}", S(T0) + S(S_LDB), S(T2))
    sal(f"s_add_u32 {sr(S_BQKV)}, {sr(S_QKV)}, {sr(T1)}", S(S_QKV) + S(T1), S(S_BQKV) + [("scc", 0)])
    sal(f"s_addc_u32 {sr(S_BQKV + 1)}, {sr(S_QKV + 1)}, {sr(T2)}", S(S_QKV + 1) + S(T2) + [("scc", 0)], S(S_BQKV + 1))
    # K base = bqkv + (Hq + kvh)*256, V base = K base + Hkv*256
    sal(f"s_add_u32 {sr(T0)}, {sr(S_HQ)}, {sr(S_KVH)}", S(S_HQ) + S(S_KVH), S(T0))
    sal(f"s_lshl_b32 {sr(T0)}, {sr(T0)}, 8", S(T0), S(T0))
    sal(f"s_add_u32 {sr(S_KB)}, {sr(S_BQKV)}, {sr(T0)}", S(S_BQKV) + S(T0), S(S_KB) + [("scc", 0)])
    sal(f"s_addc_u32 {sr(S_KB + 1)}, {sr(S_BQKV + 1)}, 0", S(S_BQKV + 1) + [("scc", 0)], S(S_KB + 1))
    sal(f"s_lshl_b32 {sr(T0)}, {sr(S_HKV)}, 8", S(S_HKV), S(T0))
    sal(f"s_add_u32 {sr(S_VB)}, {sr(S_KB)}, {sr(T0)}", S(S_KB) + S(T0), S(S_VB) + [("scc", 0)])
    sal(f"s_addc_u32 {sr(S_VB + 1)}, {sr(S_KB + 1)}, 0", S(S_KB + 1) + [("scc", 0)], S(S_VB + 1))
    # Q descriptor: base bqkv + h*256, S*ldb bytes
    sal(f"s_lshl_b32 {sr(T0)}, {sr(S_H)}, 8", S(S_H), S(T0))
    sal(f"s_add_u32 {sr(S_RQ)}, {sr(S_BQKV)}, {sr(T0)}", S(S_BQKV) + S(T0), S(S_RQ) + [("scc", 0)])
    sal(f"s_addc_u32 {sr(S_RQ + 1)}, {sr(S_BQKV + 1)}, 0", S(S_BQKV + 1) + [("scc", 0)], S(S_RQ + 1))
    sal(f"s_and_b32 {sr(S_RQ + 1)}, {sr(S_RQ + 1)}, 0xffff", S(S_RQ + 1), S(S_RQ + 1))
    sal(f"s_mul_i32 {sr(S_RQ + 2)}, {sr(S_SEQ)}, {sr(S_LDB)}", S(S_SEQ) + S(S_LDB), S(S_RQ + 2))
    sal(f"s_mov_b32 {sr(S_RQ + 3)}, 0x20000", [], S(S_RQ + 3))
    # DMA row offset of this wave inside a tile: wave * 4 instructions * 4 rows * 256 B
    sal(f"s_lshl_b32 {sr(S_LDSW)}, {sr(S_WAVE)}, 12", S(S_WAVE), S(S_LDSW))
    sal(f"s_mov_b32 {sr(S_PASS)}, 0", [], S(S_PASS))

    # ------------------------------------------------------------------ prologue: lane values
    LANE, L32, HI, DR, DP, TA, TB, TC = (V_PT + i for i in range(1, 9))
    lane_basics(L, (LANE, L32, HI))
    L.shr(DR, L.k(4), LANE)
    L.and_(DP, L.k(15), LANE)
    ldb_per_wave = np.full(4, check_ldb)
    wave_vals = np.arange(4)
    # DMA offsets: row = wave*16 + i*4 + dr; off = row*ldb + ((dp ^ (4*dr + i)) << 4)
    L.shl(TA, L.k(2), DR)                          # 4*dr
    T3 = S_TMP + 3
    for i in range(4):
        p.salu(f"s_lshl_b32 {sr(T3)}, {sr(S_WAVE)}, 4", S(S_WAVE), S(T3))
        p.salu(f"s_add_u32 {sr(T3)}, {sr(T3)}, {4 * i}", S(T3), S(T3))
        L.add(TB, DR, L.s(T3, wave_vals * 16 + i * 4))
        L.mul(TB, TB, L.s(S_LDB, ldb_per_wave))
        L.or_(TC, TA, L.k(i))
        L.xor(TC, TC, DP)
        L.shl(TC, L.k(4), TC)
        L.add(V_DOFF + i, TB, TC)
    row_read_offsets(L, V_KOFF, (LANE, L32, HI), (TA, TB, TC))
    tr_read_offsets(L, V_VOFF, (LANE, L32, HI), (TA, TB, TC, V_PT + 9, V_PT + 10, V_PT + 11, V_PT + 12))
    _check_lanes(L, check_ldb)
    return _rest(p, L, (LANE, L32, HI))


def _check_lanes(L: Lanes, ldb: int):
    tid = np.arange(256)
    lane = tid & 63
    wave = tid >> 6
    CPR, RPI, NI = 16, 4, 4
    dma_r, dma_p = lane // CPR, lane % CPR
    for i in range(4):
        row = (wave * NI + i) * RPI + dma_r
        ref = row * ldb + ((dma_p ^ np.vectorize(swz)(row)) << 4)
        assert np.array_equal(L.val[V_DOFF + i], ref & 0xFFFFFFFF), f"dma offset {i}"


class Body:
    """The kernel after the prologue's lane arithmetic: helpers for each stage."""

    def __init__(self, p: Prog):
        self.p = p
        self.L32, self.HI4 = V_L32, V_HI4

    # ---- scalar helpers
    def s(self, text, reads=(), writes=()):
        self.p.salu(text, reads, writes)

    def rsrc_tile(self, dst, base, tsg, tmp):
        """dst[0:3] = descriptor of 64-key tile tsg (SGPR holding t) of the tensor at base
        (s[base:base+1]): rows min(64, kv_end - 64t) (0 when t >= ntiles) x ldb bytes."""
        s = self.s
        k0, rows, lo, hi = tmp, tmp + 1, tmp + 2, tmp + 3
        s(f"s_lshl_b32 {sr(k0)}, {sr(tsg)}, 6", S(tsg), S(k0))
        s(f"s_sub_u32 {sr(rows)}, {sr(S_KVEND)}, {sr(k0)}", S(S_KVEND) + S(k0), S(rows))
        s(f"s_min_i32 {sr(rows)}, {sr(rows)}, 64", S(rows), S(rows))
        s(f"s_cmp_lt_u32 {sr(tsg)}, {sr(S_NT)}", S(tsg) + S(S_NT), [("scc", 0)])
        s(f"s_cselect_b32 {sr(rows)}, {sr(rows)}, 0", S(rows) + [("scc", 0)], S(rows))
        s(f"s_cselect_b32 {sr(k0)}, {sr(k0)}, 0", S(k0) + [("scc", 0)], S(k0))
        s(f"s_mul_i32 {sr(dst + 2)}, {sr(rows)}, {sr(S_LDB)}", S(rows) + S(S_LDB), S(dst + 2))
        s(f"s_mul_i32 {sr(lo)}, {sr(k0)}, {sr(S_LDB)}", S(k0) + S(S_LDB), S(lo))
        s(f"s_mul_hi_u32 {sr(hi)}, {sr(k0)}, {sr(S_LDB)}", S(k0) + S(S_LDB), S(hi))
        s(f"s_add_u32 {sr(dst)}, {sr(base)}, {sr(lo)}", S(base) + S(lo), S(dst) + [("scc", 0)])
        s(f"s_addc_u32 {sr(dst + 1)}, {sr(base + 1)}, {sr(hi)}", S(base + 1) + S(hi) + [("scc", 0)], S(dst + 1))
        s(f"s_and_b32 {sr(dst + 1)}, {sr(dst + 1)}, 0xffff", S(dst + 1), S(dst + 1))
        s(f"s_mov_b32 {sr(dst + 3)}, 0x20000", [], S(dst + 3))

    def dma_m0(self, lds_base, i):
        self.s(f"s_add_u32 m0, {sr(S_LDSW)}, {lds_base + i * 1024}", S(S_LDSW), [("m0", 0)])

    def dma_ld(self, rs, i):
        self.p.dma(f"buffer_load_dwordx4 {vr(V_DOFF + i)}, {sr(rs, 4)}, 0 offen lds",
                   V(V_DOFF + i) + S(rs, 4))

    def initial_dma(self):
        """K(0), V(0) and K(1) into buffers 0, 0 and 1 (tile 0 of the loop reads K(1))."""
        s = self.s
        s(f"s_mov_b32 {sr(S_TMP + 8)}, 0", [], S(S_TMP + 8))
        self.rsrc_tile(S_RK, S_KB, S_TMP + 8, S_TMP + 12)
        self.rsrc_tile(S_RV, S_VB, S_TMP + 8, S_TMP + 12)
        self.dma_tile(S_RK, LDS_K[0])
        self.dma_tile(S_RV, LDS_V[0])
        s(f"s_mov_b32 {sr(S_TMP + 8)}, 1", [], S(S_TMP + 8))
        self.rsrc_tile(S_RK, S_KB, S_TMP + 8, S_TMP + 12)
        self.dma_tile(S_RK, LDS_K[1])

    def dma_tile(self, rs, lds_base):
        for i in range(4):
            self.dma_m0(lds_base, i)
            self.dma_ld(rs, i)

    # ---- LDS operand reads
    def k_read(self, ri, kbase):
        kb, ks = ri // 8, ri % 8
        dst = V_KBUF + (ri % NKB) * 4
        self.p.ds_read(f"ds_read_b128 {vr(dst, 4)}, {vr(V_KOFF + ks)} offset:{kbase + kb * 32 * ROWB}",
                       V(dst, 4), V(V_KOFF + ks))

    def v_read(self, vi, vbase):
        ks, db = vi // 4, vi % 4
        dst = V_VBUF + (vi % NVB) * 4
        off = vbase + ks * 16 * ROWB
        for tt in range(2):
            self.p.ds_read(f"ds_read_b64_tr_b16 {vr(dst + 2 * tt, 2)}, {vr(V_VOFF + tt * 4 + db)} offset:{off}",
                           V(dst + 2 * tt, 2), V(V_VOFF + tt * 4 + db))

    # ---- MFMAs
    def s_mfma(self, i, J, init):
        """S MFMA i of set J: ri = i//2, qb = i%2, kb = ri//8, ks = ri%8.  init for the first
        k-step: 'zero' (accumulate from 0) or 'cinit' (from -m)."""
        ri, qb = i // 2, i % 2
        kb, ks = ri // 8, ri % 8
        dst = sblk(J, kb, qb)
        if ks == 0:
            c = None if init == "zero" else V_CINIT + qb * 16
        else:
            c = dst
        self.p.mfma(MFMA, dst, V_KBUF + (ri % NKB) * 4, A_Q + (qb * 8 + ks) * 4, c, b_acc=True)

    def pv_mfma(self, j):
        vi, qb = j // 2, j % 2
        ks, db = vi // 4, vi % 4
        o = A_O + (db * 2 + qb) * 16
        self.p.mfma(MFMA, o, V_VBUF + (vi % NVB) * 4, V_P + (qb * 4 + ks) * 4, o, dst_acc=True)

    # ---- softmax steps (n = 0..31), k-step major: step n covers P[qb][ks] word w with
    #      ks = n // 8, qb = (n % 8) // 4, w = n % 4, i.e. scores r0 + 2w, r0 + 2w + 1 of block
    #      (kb = ks // 2, qb), r0 = 8 (ks % 2).  The exp half writes exp2 in place; the pack
    #      half packs the pair to fp16 (the MFMA operand) and adds both fp32 values to this
    #      tile's partial sums of the row (two accumulators per block of 32 rows).
    @staticmethod
    def sm_regs(J, n):
        ks, qb, w = n // 8, (n % 8) // 4, n % 4
        kb, r0 = ks // 2, (ks % 2) * 8
        x0 = sblk(J, kb, qb) + r0 + 2 * w
        return x0, qb, ks, w

    def sm_exp(self, J, n):
        x0, _, _, _ = self.sm_regs(J, n)
        for x in (x0, x0 + 1):
            self.p.trans(f"v_exp_f32_e32 {vr(x)}, {vr(x)}", V(x), V(x))

    def sm_pack(self, J, n):
        x0, qb, ks, w = self.sm_regs(J, n)
        pw = V_P + (qb * 4 + ks) * 4 + w
        self.p.valu(f"v_cvt_pk_f16_f32 {vr(pw)}, {vr(x0)}, {vr(x0 + 1)}", V(x0, 2), V(pw))
        for i in range(2):
            lt = V_LT + qb * 2 + i
            if ks == 0 and w == 0:   # first step of this block of rows in the tile
                self.p.valu(f"v_mov_b32_e32 {vr(lt)}, {vr(x0 + i)}", V(x0 + i), V(lt))
            else:
                self.p.valu(f"v_add_f32_e32 {vr(lt)}, {vr(lt)}, {vr(x0 + i)}", V(lt) + V(x0 + i), V(lt))

    def sm_finish(self, qb):
        """Tile done: row sum += partial sum; track the largest partial sum."""
        lt = V_LT + qb * 2
        self.p.valu(f"v_add_f32_e32 {vr(lt)}, {vr(lt)}, {vr(lt + 1)}", V(lt, 2), V(lt))
        self.p.valu(f"v_add_f32_e32 {vr(V_LSUM + qb)}, {vr(V_LSUM + qb)}, {vr(lt)}", V(V_LSUM + qb) + V(lt), V(V_LSUM + qb))
        self.p.valu(f"v_max_f32_e32 {vr(V_LMAX + qb)}, {vr(V_LMAX + qb)}, {vr(lt)}", V(V_LMAX + qb) + V(lt), V(V_LMAX + qb))

    # ---- whole stages (unpipelined)
    def stage_s(self, J, kbase, init):
        """S(J) = K Q^T from the K buffer at kbase; reads run LK slots ahead."""
        reads_issued = 0
        for i in range(32):
            while reads_issued < 16 and reads_issued * 2 - LK <= i:
                self.k_read(reads_issued, kbase)
                reads_issued += 1
            self.s_mfma(i, J, init)

    def stage_softmax(self, J):
        for n in range(33):
            if n < 32:
                self.sm_exp(J, n)
            if n >= 1:
                self.sm_pack(J, n - 1)
        for qb in range(2):
            self.sm_finish(qb)

    def stage_pv(self, vbase):
        issued = 0
        for j in range(32):
            while issued < 16 and issued * 2 - LV <= j:
                self.v_read(issued, vbase)
                issued += 1
            self.pv_mfma(j)

    def stage_mask(self, J, tsg):
        """Scores of set J, tile t (SGPR tsg), set to -inf where key > q (causal) or
        key >= kv_len.  Per lane and 32-row block: thr = min(causal ? q - k0 - 4hi : big,
        kvl - 1 - k0 - 4hi); element key offset c = kb*32 + (r>>2)*8 + (r&3) is masked
        iff c > thr."""
        p, s = self.p, self.s
        t0, t1, t2 = S_TMP + 4, S_TMP + 5, S_TMP + 6
        TH = V_TMP  # one threshold register at a time
        s(f"s_lshl_b32 {sr(t0)}, {sr(tsg)}, 6", S(tsg), S(t0))                 # k0
        s(f"s_sub_u32 {sr(t1)}, {sr(S_KVL)}, {sr(t0)}", S(S_KVL) + S(t0), S(t1))
        s(f"s_sub_u32 {sr(t1)}, {sr(t1)}, 1", S(t1), S(t1))                     # kvl-1-k0
        for qb in range(2):
            # causal part: q0 + 32qb - k0 (scalar), or a large value
            s(f"s_add_u32 {sr(t2)}, {sr(S_Q0)}, {32 * qb}", S(S_Q0), S(t2))
            s(f"s_sub_u32 {sr(t2)}, {sr(t2)}, {sr(t0)}", S(t2) + S(t0), S(t2))
            s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
            s(f"s_cselect_b32 {sr(t2)}, 0x3fffffff, {sr(t2)}", S(t2) + [("scc", 0)], S(t2))
            # thr = min(t2 + l32, t1) - 4hi
            p.valu(f"v_add_u32 {vr(TH)}, {sr(t2)}, {vr(self.L32)}", S(t2) + V(self.L32), V(TH))
            p.valu(f"v_min_i32 {vr(TH)}, {vr(TH)}, {sr(t1)}", V(TH) + S(t1), V(TH))
            p.valu(f"v_sub_u32 {vr(TH)}, {vr(TH)}, {vr(self.HI4)}", V(TH) + V(self.HI4), V(TH))
            for kb in range(2):
                base = sblk(J, kb, qb)
                for r in range(16):
                    c = kb * 32 + (r >> 2) * 8 + (r & 3)
                    p.valu(f"v_cmp_gt_i32_e32 vcc, {c}, {vr(TH)}", V(TH), [("vcc", 0)])
                    p.valu(f"v_cndmask_b32_e32 {vr(base + r)}, {vr(base + r)}, {vr(V_NINF)}, vcc",
                           V(base + r) + V(V_NINF) + [("vcc", 0)], V(base + r))

    def row_max_set_m(self, J):
        """m = row max of set J (0 if -inf); cinit = -m; set J -= m."""
        p = self.p
        for qb in range(2):
            mx = V_P + qb * 2          # P registers are free here
            tmp = mx + 1
            regs = [sblk(J, kb, qb) + r for kb in range(2) for r in range(16)]
            p.valu(f"v_max_f32_e32 {vr(mx)}, {vr(regs[0])}, {vr(regs[1])}", V(regs[0], 2), V(mx))
            for x in regs[2:]:
                p.valu(f"v_max_f32_e32 {vr(mx)}, {vr(mx)}, {vr(x)}", V(mx) + V(x), V(mx))
            p.valu(f"v_mov_b32_e32 {vr(tmp)}, {vr(mx)}", V(mx), V(tmp))
            p.emit(f"v_permlane32_swap_b32_e32 {vr(tmp)}, {vr(mx)}", PERMLANE, V(tmp) + V(mx), V(tmp) + V(mx))
            p.valu(f"v_max_f32_e32 {vr(mx)}, {vr(mx)}, {vr(tmp)}", V(mx) + V(tmp), V(mx))
            p.valu(f"v_cmp_eq_f32_e32 vcc, {vr(V_NINF)}, {vr(mx)}", V(V_NINF) + V(mx), [("vcc", 0)])
            p.valu(f"v_cndmask_b32_e64 {vr(mx)}, {vr(mx)}, 0, vcc", V(mx) + [("vcc", 0)], V(mx))
            ci = V_CINIT + qb * 16
            p.valu(f"v_sub_f32_e32 {vr(ci)}, 0, {vr(mx)}", V(mx), V(ci))
            for r in range(1, 16):
                p.valu(f"v_mov_b32_e32 {vr(ci + r)}, {vr(ci)}", V(ci), V(ci + r))
            for x in regs:
                p.valu(f"v_sub_f32_e32 {vr(x)}, {vr(x)}, {vr(mx)}", V(x) + V(mx), V(x))

    def tile_max_into(self, J, mxs):
        """mxs[qb] = max(mxs[qb], row max of set J) (exact pass)."""
        p = self.p
        for qb in range(2):
            mx, tmp = mxs[qb], V_TMP
            for kb in range(2):
                for r in range(16):
                    x = sblk(J, kb, qb) + r
                    p.valu(f"v_max_f32_e32 {vr(mx)}, {vr(mx)}, {vr(x)}", V(mx) + V(x), V(mx))
            p.valu(f"v_mov_b32_e32 {vr(tmp)}, {vr(mx)}", V(mx), V(tmp))
            p.emit(f"v_permlane32_swap_b32_e32 {vr(tmp)}, {vr(mx)}", PERMLANE, V(tmp) + V(mx), V(tmp) + V(mx))
            p.valu(f"v_max_f32_e32 {vr(mx)}, {vr(mx)}, {vr(tmp)}", V(mx) + V(tmp), V(mx))

    # ---- the pipelined tile
    def tile_pipe(self, J):
        """Iteration t with set J = t & 1: S(t+1) into set J^1 from K buffer J^1, softmax of
        set J, O += V(t) P from V buffer J; DMA K(t+2) -> K buffer J, V(t+1) -> V buffer J^1.
        Slots 0..31 run the S MFMAs, 32..63 the PV MFMAs (k-step major, so PV(ks) starts at
        slot 32 + 8ks).  Softmax step n has its exp half at slot e(n) = floor(7n/4) and its
        pack half one slot later (P[*][ks] is complete at slot e(8ks+7) + 1 <= 32 + 8ks); the
        DMA instructions go one every four slots from slot 2 so the vector memory path never
        backs up into the issue of the MFMA stream."""
        Jn = J ^ 1
        kbase, vbase = LDS_K[Jn], LDS_V[J]
        exp_at = {(7 * n) // 4: n for n in range(32)}
        pack_at = {(7 * n) // 4 + 1: n for n in range(32)}
        dma_at = {2 + 4 * i: i for i in range(8)}
        kissued = 0
        while kissued * 2 - LK < 0:
            self.k_read(kissued, kbase)
            kissued += 1
        vissued = 0
        for s_ in range(64):
            while kissued < 16 and kissued * 2 - LK <= s_:
                self.k_read(kissued, kbase)
                kissued += 1
            while vissued < 16 and 32 + vissued * 2 - LV <= s_:
                self.v_read(vissued, vbase)
                vissued += 1
            if s_ in dma_at:
                i = dma_at[s_]
                self.dma_m0(LDS_K[J] if i < 4 else LDS_V[Jn], i % 4)
            if s_ < 32:
                self.s_mfma(s_, Jn, "cinit")
            else:
                self.pv_mfma(s_ - 32)
            if s_ in exp_at:
                self.sm_exp(J, exp_at[s_])
            if s_ in pack_at:
                self.sm_pack(J, pack_at[s_])
            if s_ in (57, 59):
                self.sm_finish((s_ - 57) // 2)
            if s_ in dma_at:
                i = dma_at[s_]
                self.dma_ld(S_RK if i < 4 else S_RV, i % 4)

    # ---- the per-tile body, both paths
    def body(self, J, n):
        """Tile t (SGPR S_T) with register set J = t & 1; n numbers the labels."""
        p, s = self.p, self.s
        Jn = J ^ 1
        T0, T1, T2 = S_TMP + 8, S_TMP + 9, S_TMP + 10
        p.label(f".Lbody{n}")
        s(f"s_cmp_ge_u32 {sr(S_T)}, {sr(S_NT)}", S(S_T) + S(S_NT), [("scc", 0)])
        p.branch("s_cbranch_scc1 .Lloop_done", [("scc", 0)])
        s(f"s_add_u32 {sr(T0)}, {sr(S_T)}, 2", S(S_T), S(T0))
        self.rsrc_tile(S_RK, S_KB, T0, S_TMP + 12)
        s(f"s_add_u32 {sr(T0)}, {sr(S_T)}, 1", S(S_T), S(T0))
        self.rsrc_tile(S_RV, S_VB, T0, S_TMP + 12)
        # pipelined iff t + 1 < n_act and t < n_plain
        s(f"s_cmp_lt_u32 {sr(T0)}, {sr(S_NACT)}", S(T0) + S(S_NACT), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T1)}, 1, 0", [("scc", 0)], S(T1))
        s(f"s_cmp_lt_u32 {sr(S_T)}, {sr(S_NPLAIN)}", S(S_T) + S(S_NPLAIN), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T2)}, {sr(T1)}, 0", S(T1) + [("scc", 0)], S(T2))
        s(f"s_cmp_eq_u32 {sr(T2)}, 0", S(T2), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lslow{n}", [("scc", 0)])
        self.tile_pipe(J)
        p.branch(f"s_branch .Lend{n}")
        p.label(f".Lslow{n}")
        self.dma_tile(S_RK, LDS_K[J])
        self.dma_tile(S_RV, LDS_V[Jn])
        s(f"s_cmp_lt_u32 {sr(S_T)}, {sr(S_NACT)}", S(S_T) + S(S_NACT), [("scc", 0)])
        p.branch(f"s_cbranch_scc0 .Lend{n}", [("scc", 0)])
        s(f"s_cmp_lt_u32 {sr(S_T)}, {sr(S_NPLAIN)}", S(S_T) + S(S_NPLAIN), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lnomask{n}", [("scc", 0)])
        self.stage_mask(J, S_T)
        p.label(f".Lnomask{n}")
        self.stage_softmax(J)
        self.stage_pv(LDS_V[J])
        s(f"s_add_u32 {sr(T0)}, {sr(S_T)}, 1", S(S_T), S(T0))
        s(f"s_cmp_lt_u32 {sr(T0)}, {sr(S_NACT)}", S(T0) + S(S_NACT), [("scc", 0)])
        p.branch(f"s_cbranch_scc0 .Lend{n}", [("scc", 0)])
        self.stage_s(Jn, LDS_K[Jn], "cinit")
        p.label(f".Lend{n}")
        p.waitcnt(vm=0)
        p.barrier()
        s(f"s_add_u32 {sr(S_T)}, {sr(S_T)}, 1", S(S_T), S(S_T))


def _rest(p: Prog, L, lanes) -> str:
    LANE, L32, HI = lanes
    b = Body(p)
    s = b.s
    # persistent lane values, constants
    p.valu(f"v_mov_b32_e32 {vr(V_L32)}, {vr(L32)}", V(L32), V(V_L32))
    p.valu(f"v_lshlrev_b32_e32 {vr(V_HI4)}, 2, {vr(HI)}", V(HI), V(V_HI4))
    p.valu(f"v_mov_b32_e32 {vr(V_NINF)}, 0xff800000", [], V(V_NINF))
    # first K/V tiles in flight before anything else (their latency overlaps the Q load)
    b.initial_dma()
    # LDS redo flag = 0 (every wave writes it before the first barrier)
    p.valu(f"v_mov_b32_e32 {vr(V_T)}, {LDS_FLAG}", [], V(V_T))
    p.valu(f"v_mov_b32_e32 {vr(V_T + 1)}, 0", [], V(V_T + 1))
    p.ds_write(f"ds_write_b32 {vr(V_T)}, {vr(V_T + 1)}", V(V_T) + V(V_T + 1))
    # ---- Q: 64 rows x 128 of this wave, two 32-row blocks; lane (l32, hi) loads row
    #      q0 + 32qb + l32, bytes hi*16 + 32ks .. +15; prescaled by sl2, rounded to fp16
    QOFF = V_P  # two registers
    p.valu(f"v_lshlrev_b32_e32 {vr(V_T)}, 4, {vr(HI)}", V(HI), V(V_T))
    for qb in range(2):
        p.valu(f"v_add_u32_e32 {vr(QOFF + qb)}, {sr(S_Q0)}, {vr(L32)}", S(S_Q0) + V(L32), V(QOFF + qb))
        if qb:
            p.valu(f"v_add_u32_e32 {vr(QOFF + qb)}, 32, {vr(QOFF + qb)}", V(QOFF + qb), V(QOFF + qb))
        p.valu(f"v_mul_lo_u32 {vr(QOFF + qb)}, {vr(QOFF + qb)}, {sr(S_LDB)}", V(QOFF + qb) + S(S_LDB), V(QOFF + qb))
        p.valu(f"v_add_u32_e32 {vr(QOFF + qb)}, {vr(QOFF + qb)}, {vr(V_T)}", V(QOFF + qb) + V(V_T), V(QOFF + qb))
    for qb in range(2):
        for ks in range(8):
            dst = (qb * 8 + ks) * 4
            p.vmem_load(f"buffer_load_dwordx4 {vr(dst, 4)}, {vr(QOFF + qb)}, {sr(S_RQ, 4)}, 0 offen offset:{ks * 32}",
                        V(dst, 4), V(QOFF + qb) + S(S_RQ, 4))
    # accumulators
    for i in range(128):
        p.valu(f"v_accvgpr_write_b32 {ar(A_O + i)}, 0", [], A(A_O + i))
    for qb in range(2):
        p.valu(f"v_mov_b32_e32 {vr(V_LSUM + qb)}, 0", [], V(V_LSUM + qb))
        p.valu(f"v_mov_b32_e32 {vr(V_LMAX + qb)}, 0", [], V(V_LMAX + qb))
    # prescale: word w of Q fragment -> two f32 (x * sl2) -> fp16 pair -> AGPR
    for i in range(64):
        x = i
        t0, t1 = V_CINIT, V_CINIT + 1
        p.valu(f"v_fma_mix_f32 {vr(t0)}, {vr(x)}, {sr(S_SL2)}, 0 op_sel_hi:[1,0,0]", V(x) + S(S_SL2), V(t0))
        p.valu(f"v_fma_mix_f32 {vr(t1)}, {vr(x)}, {sr(S_SL2)}, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]", V(x) + S(S_SL2), V(t1))
        p.valu(f"v_cvt_pk_f16_f32 {vr(x)}, {vr(t0)}, {vr(t1)}", V(t0, 2), V(x))
        p.valu(f"v_accvgpr_write_b32 {ar(A_Q + i)}, {vr(x)}", V(x), A(A_Q + i))

    # ---- main loop (pass 0 falls through with its first tiles already requested; the
    #      exact redo pass enters at .Lmain_dma)
    p.branch("s_branch .Lmain")
    p.label(".Lmain_dma")
    b.initial_dma()
    p.label(".Lmain")
    s(f"s_mov_b32 {sr(S_T)}, 0", [], S(S_T))
    p.waitcnt(vm=0)
    p.barrier()
    s(f"s_cmp_eq_u32 {sr(S_NACT)}, 0", S(S_NACT), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lpro_end", [("scc", 0)])
    s(f"s_cmp_eq_u32 {sr(S_PASS)}, 0", S(S_PASS), [("scc", 0)])
    p.branch("s_cbranch_scc0 .Lpro_fixed", [("scc", 0)])
    b.stage_s(0, LDS_K[0], "zero")
    p.branch("s_branch .Lpro_s0")
    p.label(".Lpro_fixed")
    b.stage_s(0, LDS_K[0], "cinit")
    p.label(".Lpro_s0")
    s(f"s_cmp_eq_u32 {sr(S_NPLAIN)}, 0", S(S_NPLAIN), [("scc", 0)])
    p.branch("s_cbranch_scc0 .Lpro_nomask", [("scc", 0)])
    b.stage_mask(0, S_T)
    p.label(".Lpro_nomask")
    s(f"s_cmp_eq_u32 {sr(S_PASS)}, 0", S(S_PASS), [("scc", 0)])
    p.branch("s_cbranch_scc0 .Lpro_end", [("scc", 0)])
    b.row_max_set_m(0)
    p.label(".Lpro_end")
    p.barrier()
    p.label(".Lloop")
    b.body(0, 0)
    b.body(1, 1)
    p.branch("s_branch .Lloop")
    p.label(".Lloop_done")

    # ---- overflow check (pass 0): any row sum not finite -> exact pass
    s(f"s_cmp_eq_u32 {sr(S_PASS)}, 0", S(S_PASS), [("scc", 0)])
    p.branch("s_cbranch_scc0 .Lepi", [("scc", 0)])
    # a P above the fp16 range makes its lane's partial sum of that tile exceed 65504
    p.valu(f"v_mov_b32_e32 {vr(V_T + 2)}, 0x477fe000", [], V(V_T + 2))
    for qb, c in ((0, S_C0), (1, S_C1)):
        p.valu(f"v_cmp_gt_f32_e64 {sr(c, 2)}, {vr(V_T + 2)}, {vr(V_LMAX + qb)}", V(V_T + 2) + V(V_LMAX + qb), S(c, 2))
    s(f"s_and_b64 {sr(S_C0, 2)}, {sr(S_C0, 2)}, {sr(S_C1, 2)}", S(S_C0, 2) + S(S_C1, 2), S(S_C0, 2))
    s(f"s_andn2_b64 {sr(S_C0, 2)}, exec, {sr(S_C0, 2)}", S(S_C0, 2) + [("exec", 0)], S(S_C0, 2))
    s(f"s_cmp_lg_u64 {sr(S_C0, 2)}, 0", S(S_C0, 2), [("scc", 0)])
    p.branch("s_cbranch_scc0 .Lnobad", [("scc", 0)])
    p.valu(f"v_mov_b32_e32 {vr(V_T)}, {LDS_FLAG}", [], V(V_T))
    p.valu(f"v_mov_b32_e32 {vr(V_T + 1)}, 1", [], V(V_T + 1))
    p.ds_write(f"ds_write_b32 {vr(V_T)}, {vr(V_T + 1)}", V(V_T) + V(V_T + 1))
    p.label(".Lnobad")
    p.waitcnt(lgkm=0)
    p.barrier()
    p.valu(f"v_mov_b32_e32 {vr(V_T)}, {LDS_FLAG}", [], V(V_T))
    p.ds_read(f"ds_read_b32 {vr(V_T + 1)}, {vr(V_T)}", V(V_T + 1), V(V_T))
    p.readlane(f"v_readfirstlane_b32 {sr(S_TMP)}, {vr(V_T + 1)}", V(V_T + 1), S(S_TMP))
    s(f"s_cmp_eq_u32 {sr(S_TMP)}, 0", S(S_TMP), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lepi", [("scc", 0)])
    # exact row max over all visible keys
    MX = (V_P, V_P + 1)
    for m_ in MX:
        p.valu(f"v_mov_b32_e32 {vr(m_)}, {vr(V_NINF)}", V(V_NINF), V(m_))
    s(f"s_mov_b32 {sr(S_T)}, 0", [], S(S_T))
    p.label(".Lxloop")
    s(f"s_cmp_ge_u32 {sr(S_T)}, {sr(S_NT)}", S(S_T) + S(S_NT), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lxdone", [("scc", 0)])
    b.rsrc_tile(S_RK, S_KB, S_T, S_TMP + 12)
    b.dma_tile(S_RK, LDS_K[0])
    p.waitcnt(vm=0)
    p.barrier()
    s(f"s_cmp_lt_u32 {sr(S_T)}, {sr(S_NACT)}", S(S_T) + S(S_NACT), [("scc", 0)])
    p.branch("s_cbranch_scc0 .Lxskip", [("scc", 0)])
    b.stage_s(0, LDS_K[0], "zero")
    s(f"s_cmp_lt_u32 {sr(S_T)}, {sr(S_NPLAIN)}", S(S_T) + S(S_NPLAIN), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lxnomask", [("scc", 0)])
    b.stage_mask(0, S_T)
    p.label(".Lxnomask")
    b.tile_max_into(0, MX)
    p.label(".Lxskip")
    p.barrier()
    s(f"s_add_u32 {sr(S_T)}, {sr(S_T)}, 1", S(S_T), S(S_T))
    p.branch("s_branch .Lxloop")
    p.label(".Lxdone")
    for qb in range(2):
        mx = MX[qb]
        p.valu(f"v_cmp_eq_f32_e32 vcc, {vr(V_NINF)}, {vr(mx)}", V(V_NINF) + V(mx), [("vcc", 0)])
        p.valu(f"v_cndmask_b32_e64 {vr(mx)}, {vr(mx)}, 0, vcc", V(mx) + [("vcc", 0)], V(mx))
        ci = V_CINIT + qb * 16
        p.valu(f"v_sub_f32_e32 {vr(ci)}, 0, {vr(mx)}", V(mx), V(ci))
        for r in range(1, 16):
            p.valu(f"v_mov_b32_e32 {vr(ci + r)}, {vr(ci)}", V(ci), V(ci + r))
        p.valu(f"v_mov_b32_e32 {vr(V_LSUM + qb)}, 0", [], V(V_LSUM + qb))
        p.valu(f"v_mov_b32_e32 {vr(V_LMAX + qb)}, 0", [], V(V_LMAX + qb))
    for i in range(128):
        p.valu(f"v_accvgpr_write_b32 {ar(A_O + i)}, 0", [], A(A_O + i))
    s(f"s_mov_b32 {sr(S_PASS)}, 1", [], S(S_PASS))
    p.branch("s_branch .Lmain_dma")

    # ---- epilogue: O = acc / l (fp16), LSE = (m + log2 l) ln 2
    p.label(".Lepi")
    T0, T1, T2 = S_TMP, S_TMP + 1, S_TMP + 2
    # O descriptor: base out + b*S*ldo, S*ldo bytes
    s(f"s_mul_i32 {sr(T0)}, {sr(S_B)}, {sr(S_SEQ)}", S(S_B) + S(S_SEQ), S(T0))
    s(f"s_mul_i32 {sr(T1)}, {sr(T0)}, {sr(S_LDO)}", S(T0) + S(S_LDO), S(T1))
    s(f"s_mul_hi_u32 {sr(T2)}, {sr(T0)}, {sr(S_LDO)}", S(T0) + S(S_LDO), S(T2))
    s(f"s_add_u32 {sr(S_RQ)}, {sr(S_OUT)}, {sr(T1)}", S(S_OUT) + S(T1), S(S_RQ) + [("scc", 0)])
    s(f"s_addc_u32 {sr(S_RQ + 1)}, {sr(S_OUT + 1)}, {sr(T2)}", S(S_OUT + 1) + S(T2) + [("scc", 0)], S(S_RQ + 1))
    s(f"s_and_b32 {sr(S_RQ + 1)}, {sr(S_RQ + 1)}, 0xffff", S(S_RQ + 1), S(S_RQ + 1))
    s(f"s_mul_i32 {sr(S_RQ + 2)}, {sr(S_SEQ)}, {sr(S_LDO)}", S(S_SEQ) + S(S_LDO), S(S_RQ + 2))
    s(f"s_mov_b32 {sr(S_RQ + 3)}, 0x20000", [], S(S_RQ + 3))
    # LSE descriptor: base lse + (b*Hq + h)*S*4, S*4 bytes (none when lse is null)
    s(f"s_mul_i32 {sr(T0)}, {sr(S_B)}, {sr(S_HQ)}", S(S_B) + S(S_HQ), S(T0))
    s(f"s_add_u32 {sr(T0)}, {sr(T0)}, {sr(S_H)}", S(T0) + S(S_H), S(T0))
    s(f"s_mul_i32 {sr(T0)}, {sr(T0)}, {sr(S_SEQ)}", S(T0) + S(S_SEQ), S(T0))
    s(f"s_mul_hi_u32 {sr(T2)}, {sr(T0)}, 4", S(T0), S(T2))
    s(f"s_lshl_b32 {sr(T1)}, {sr(T0)}, 2", S(T0), S(T1))
    s(f"s_add_u32 {sr(S_RL)}, {sr(S_LSE)}, {sr(T1)}", S(S_LSE) + S(T1), S(S_RL) + [("scc", 0)])
    s(f"s_addc_u32 {sr(S_RL + 1)}, {sr(S_LSE + 1)}, {sr(T2)}", S(S_LSE + 1) + S(T2) + [("scc", 0)], S(S_RL + 1))
    s(f"s_and_b32 {sr(S_RL + 1)}, {sr(S_RL + 1)}, 0xffff", S(S_RL + 1), S(S_RL + 1))
    s(f"s_lshl_b32 {sr(S_RL + 2)}, {sr(S_SEQ)}, 2", S(S_SEQ), S(S_RL + 2))
    s(f"s_cmp_eq_u64 {sr(S_LSE, 2)}, 0", S(S_LSE, 2), [("scc", 0)])
    s(f"s_cselect_b32 {sr(S_RL + 2)}, 0, {sr(S_RL + 2)}", S(S_RL + 2) + [("scc", 0)], S(S_RL + 2))
    s(f"s_mov_b32 {sr(S_RL + 3)}, 0x20000", [], S(S_RL + 3))
    s(f"s_lshl_b32 {sr(T0)}, {sr(S_H)}, 8", S(S_H), S(T0))
    Q, LO, L_, INV, LG = 0, 2, 3, 4, 5           # registers in the free score region
    W = 8                                        # 4 values + 2 packed words
    # O leaves through the wave's LDS staging rows (row = query, 16-byte chunk db*4 + g4) so
    # that each store instruction writes four whole 256-byte rows; write address
    # EPW + l32*272 + hi*8, read address EPW + (lane>>4)*272 + (lane&15)*16
    BW, BR, TA, TB, RBUF, OOS = 24, 25, 26, 27, 28, 44
    EPW, ROW4 = S_TMP + 4, S_TMP + 5
    s(f"s_mul_i32 {sr(EPW)}, {sr(S_WAVE)}, {EPI_WAVE}", S(S_WAVE), S(EPW))
    s(f"s_add_u32 {sr(EPW)}, {sr(EPW)}, {LDS_EPI}", S(EPW), S(EPW))
    s(f"s_lshl_b32 {sr(ROW4)}, {sr(S_LDO)}, 2", S(S_LDO), S(ROW4))
    p.valu(f"v_mul_u32_u24_e32 {vr(BW)}, {EPI_ROW}, {vr(V_L32)}", V(V_L32), V(BW))
    p.valu(f"v_add_u32_e32 {vr(BW)}, {sr(EPW)}, {vr(BW)}", S(EPW) + V(BW), V(BW))
    p.valu(f"v_lshl_add_u32 {vr(BW)}, {vr(V_HI4)}, 1, {vr(BW)}", V(V_HI4) + V(BW), V(BW))
    p.valu(f"v_lshrrev_b32_e32 {vr(TA)}, 4, {vr(V_L32)}", V(V_L32), V(TA))
    p.valu(f"v_lshrrev_b32_e32 {vr(TB)}, 1, {vr(V_HI4)}", V(V_HI4), V(TB))
    p.valu(f"v_add_u32_e32 {vr(TA)}, {vr(TA)}, {vr(TB)}", V(TA) + V(TB), V(TA))        # lane >> 4
    p.valu(f"v_and_b32_e32 {vr(TB)}, 15, {vr(V_L32)}", V(V_L32), V(TB))                 # lane & 15
    p.valu(f"v_mul_u32_u24_e32 {vr(BR)}, {EPI_ROW}, {vr(TA)}", V(TA), V(BR))
    p.valu(f"v_lshl_add_u32 {vr(BR)}, {vr(TB)}, 4, {vr(BR)}", V(TB) + V(BR), V(BR))
    p.valu(f"v_add_u32_e32 {vr(BR)}, {sr(EPW)}, {vr(BR)}", S(EPW) + V(BR), V(BR))
    # global offset of row q0 + (lane >> 4), chunk lane & 15 of this head; +4 rows per read
    p.valu(f"v_add_u32_e32 {vr(TA)}, {sr(S_Q0)}, {vr(TA)}", S(S_Q0) + V(TA), V(TA))
    p.valu(f"v_mul_lo_u32 {vr(TA)}, {vr(TA)}, {sr(S_LDO)}", V(TA) + S(S_LDO), V(TA))
    p.valu(f"v_lshl_add_u32 {vr(OOS)}, {vr(TB)}, 4, {vr(TA)}", V(TB) + V(TA), V(OOS))
    p.valu(f"v_add_u32_e32 {vr(OOS)}, {sr(T0)}, {vr(OOS)}", S(T0) + V(OOS), V(OOS))
    for i in range(1, 16):
        p.valu(f"v_add_u32_e32 {vr(OOS + i)}, {sr(ROW4)}, {vr(OOS + i - 1)}", S(ROW4) + V(OOS + i - 1), V(OOS + i))
    for qb in range(2):
        # q and LSE offsets
        p.valu(f"v_add_u32_e32 {vr(Q)}, {sr(S_Q0)}, {vr(V_L32)}", S(S_Q0) + V(V_L32), V(Q))
        if qb:
            p.valu(f"v_add_u32_e32 {vr(Q)}, 32, {vr(Q)}", V(Q), V(Q))
        p.valu(f"v_lshlrev_b32_e32 {vr(LO)}, 2, {vr(Q)}", V(Q), V(LO))
        p.valu(f"v_cmp_eq_u32_e32 vcc, 0, {vr(V_HI4)}", V(V_HI4), [("vcc", 0)])
        p.valu(f"v_mov_b32_e32 {vr(V_T)}, 0x7ffffff0", [], V(V_T))
        p.valu(f"v_cndmask_b32_e32 {vr(LO)}, {vr(V_T)}, {vr(LO)}, vcc", V(V_T) + V(LO) + [("vcc", 0)], V(LO))
        # l = both lane halves' sums
        p.valu(f"v_mov_b32_e32 {vr(L_)}, {vr(V_LSUM + qb)}", V(V_LSUM + qb), V(L_))
        p.valu(f"v_mov_b32_e32 {vr(V_T)}, {vr(V_LSUM + qb)}", V(V_LSUM + qb), V(V_T))
        p.emit(f"v_permlane32_swap_b32_e32 {vr(L_)}, {vr(V_T)}", PERMLANE, V(L_) + V(V_T), V(L_) + V(V_T))
        p.valu(f"v_add_f32_e32 {vr(L_)}, {vr(L_)}, {vr(V_T)}", V(L_) + V(V_T), V(L_))
        p.trans(f"v_rcp_f32_e32 {vr(INV)}, {vr(L_)}", V(L_), V(INV))
        p.trans(f"v_log_f32_e32 {vr(LG)}, {vr(L_)}", V(L_), V(LG))
        p.valu(f"v_cmp_lt_f32_e32 vcc, 0, {vr(L_)}", V(L_), [("vcc", 0)])
        p.valu(f"v_cndmask_b32_e64 {vr(INV)}, 0, {vr(INV)}, vcc", V(INV) + [("vcc", 0)], V(INV))
        p.valu(f"v_sub_f32_e32 {vr(LG)}, {vr(LG)}, {vr(V_CINIT + qb * 16)}", V(LG) + V(V_CINIT + qb * 16), V(LG))
        p.valu(f"v_mul_f32_e32 {vr(LG)}, 0x3f317218, {vr(LG)}", V(LG), V(LG))
        p.valu(f"v_cndmask_b32_e32 {vr(LG)}, {vr(V_NINF)}, {vr(LG)}, vcc", V(V_NINF) + V(LG) + [("vcc", 0)], V(LG))
        p.vmem_store(f"buffer_store_dword {vr(LG)}, {vr(LO)}, {sr(S_RL, 4)}, 0 offen", V(LG) + V(LO) + S(S_RL, 4))
        for db in range(4):
            for g4 in range(4):
                o = A_O + (db * 2 + qb) * 16 + g4 * 4
                for j in range(4):
                    p.valu(f"v_accvgpr_read_b32 {vr(W + j)}, {ar(o + j)}", A(o + j), V(W + j))
                for j in range(4):
                    p.valu(f"v_mul_f32_e32 {vr(W + j)}, {vr(W + j)}, {vr(INV)}", V(W + j) + V(INV), V(W + j))
                p.valu(f"v_cvt_pk_f16_f32 {vr(W + 4)}, {vr(W)}, {vr(W + 1)}", V(W, 2), V(W + 4))
                p.valu(f"v_cvt_pk_f16_f32 {vr(W + 5)}, {vr(W + 2)}, {vr(W + 3)}", V(W + 2, 2), V(W + 5))
                p.ds_write(f"ds_write_b64 {vr(BW)}, {vr(W + 4, 2)} offset:{(db * 4 + g4) * 16}", V(BW) + V(W + 4, 2))
                W = 8 if W == 16 else 16   # alternate register sets
        for i in range(8):   # LDS operations of a wave complete in order: reads see the rows
            R = RBUF + 4 * (i % 4)
            p.ds_read(f"ds_read_b128 {vr(R, 4)}, {vr(BR)} offset:{i * 4 * EPI_ROW}", V(R, 4), V(BR))
            p.vmem_store(f"buffer_store_dwordx4 {vr(R, 4)}, {vr(OOS + qb * 8 + i)}, {sr(S_RQ, 4)}, 0 offen",
                         V(R, 4) + V(OOS + qb * 8 + i) + S(S_RQ, 4))
    p.emit("s_endpgm", BRANCH)
    body_lines = p.finalize()
    return kernel_text(NAME, body_lines, lds_bytes=LDS_BYTES, kernarg_bytes=KERNARG_BYTES,
                       next_free_sgpr=NEXT_FREE_SGPR, args=ARGS)


def main(path: str) -> None:
    with open(path, "w") as f:
        f.write(build())


if __name__ == "__main__":
    import sys
    main(sys.argv[1])

"""Generator of the gfx950 assembly FlashAttention backward dK/dV kernel, D = 128, fp16.

Contract: identical to fa_bwd_dkdv_kernel (tokamak_amd/csrc/attn_bwd.hip), the true-gradient
replacement of the reference's k_gqa_flash_attn_tc_bwd dK/dV (src/tkm_gpu.cu:440-598, which
writes copies of dQ/dO at 588-596 instead):
    P_ij = exp(s_ij - LSE_i),  dS_ij = P_ij (<dO_i, v_j> - D_i)
    dK_j = scale sum_i dS_ij q_i,  dV_j = sum_i P_ij dO_i
over every query row i of every q-head of key j's kv group, key j visible from row i iff
j < kv_len[b] and (!causal || j <= i); dK and dV are written (not accumulated) into dqkv.

Work decomposition: grid (Hkv, B, n_kblk), one workgroup = 4 waves = one (batch, kv head,
block of 128 keys); one wave per SIMD.  A wave owns 32 keys: K (prescaled by
scale*log2(e)) and V of those keys sit in AGPRs as the B operands of S = Q K^T and
dP = dO V^T, and the accumulators dV^T, dK^T (C[m = head dim][n = key]) in AGPRs.  The
workgroup walks the query tiles (32 rows) of every q-head of the group (causal: from its own
key block on); each tile's Q, dO, LSE and D rows go HBM -> LDS by buffer DMA into one of four
buffers (tile t in buffer t % 4, requested three tiles ahead).  Per tile:
    S  = Q K'^T  + (-LSE*log2e)   8 MFMAs, C[m = query][n = key]: lane = key
    dP = dO V^T  + (-D)           8 MFMAs (the offsets enter as the accumulators' start value)
    P = exp2(S), dS = P * dP      masked to 0 where the key is hidden
    dV^T += dO^T P, dK^T += Q^T dS 16 MFMAs, P and dS packed to fp16 in place as B operands,
                                  dO^T and Q^T read transposed (ds_read_b64_tr_b16)
Each iteration runs 32 MFMA slots: S/dP of the next tile with the elementwise work of this
tile between them, one workgroup barrier, then dV/dK of this tile, with the next-but-one
tile's LSE/D offsets loaded and the tile three ahead requested in between.
"""
from __future__ import annotations

import numpy as np

from .common import Lanes, lane_basics, row_read_offsets, swz, tr_read_offsets
from .gfx950 import A, BRANCH, Prog, S, V, ar, kernel_text, sr, vr

NAME = "tkm_fa_bwd_dkdv_d128_f16"
MFMA = "v_mfma_f32_32x32x16_f16"
ROWB = 256
NBUF = 4
TILE = 32 * ROWB                    # 8 KB: one 32-row tile of Q or dO
BUFB = 2 * TILE                     # Q then dO
LDS_LD = NBUF * BUFB                # LSE / D area, 1 KB per buffer: LSE at +0, D at +256;
LDB = 1024                          # +512, +768: zero rows from the waves that load neither
LDS_BYTES = LDS_LD + NBUF * LDB
LK = 4                              # slots between a row read and its MFMA
LV = 4                              # slots between a transposed read pair and its MFMA
NRB = 6                             # row-read registers in rotation (x4)
NTB = 6                             # transposed-read registers in rotation (x4)
NEG_LOG2E = "0xbfb8aa3b"

ARGS = [(0, 8, "ptr"), (8, 8, "ptr"), (16, 8, "ptr"), (24, 8, "ptr"), (32, 8, "ptr"), (40, 8, "ptr")] + \
       [(48 + 4 * i, 4, "val") for i in range(12)]
KERNARG_BYTES = 96

# ---- SGPRs
S_H, S_B, S_Z = 2, 3, 4                 # kv head, batch, key block
S_QKV, S_DOUT, S_LSE, S_DELTA, S_DQKV, S_KVLEN = 8, 10, 12, 14, 16, 18
S_SEQ, S_HQ, S_HKV, S_SL2 = 20, 21, 22, 23
S_CAUSAL, S_LDB, S_LDO, S_G, S_SCALE, S_NKBLK = 24, 25, 26, 27, 28, 29
S_WAVE, S_KVL, S_KB0, S_KW0, S_QTB, S_QTE, S_ITERS, S_IT = 32, 33, 34, 35, 36, 37, 38, 39
S_BQKV, S_BDO, S_BLSE, S_BDEL = 40, 42, 44, 46     # 64-bit bases (batch, head-group start)
S_RQ, S_RO, S_RL = 48, 52, 56                      # DMA descriptors of the requested tile
S_QT0, S_QT1, S_QT3, S_H3 = 60, 61, 62, 63         # q-tile of tiles it, it+1; (head, q-tile) of it+3
S_LDSW, S_LDSL = 64, 65                            # wave's DMA offset in a tile; LDS target of its LSE/D DMA
S_SMALLSEL = 66                                    # 0: LSE, 1: D, 2: nothing
S_KWACT = 67                                       # 1 if the wave has a visible key at all
S_KWMASK = 68                                      # 1 if some key of the wave is >= kv_len
S_TMP = 72                                         # s72..s87
NEXT_FREE_SGPR = 88

# ---- VGPRs
V_SD = (0, 32)          # set J: S at +0..15, dP at +16..31
V_P, V_DS = 64, 72      # packed P[ks][w], dS[ks][w]
V_CS, V_CD = 80, 96     # accumulator start values: -LSE*log2e, -D (per register row)
V_RB = 112              # row-read buffers
V_TB = V_RB + 4 * NRB   # transposed-read buffers
V_KOFF = V_TB + 4 * NTB
V_VOFF = V_KOFF + 8
V_DOFF = V_VOFF + 8     # Q rows (2), dO rows (2)
V_LOFF = V_DOFF + 4     # lane*4 (LSE/D DMA)
V_LDR = V_LOFF + 1      # LSE/D read base: LDS_LD + hi*16
V_L32 = V_LDR + 1
V_HI4 = V_L32 + 1
V_TK = V_HI4 + 1        # mask threshold of the current tile
V_T = V_TK + 1          # temporaries
V_PT = V_T + 8          # prologue lane scratch (13 registers)
assert V_PT + 13 <= 256

# ---- AGPRs
A_DV, A_DK, A_K, A_V = 0, 64, 128, 160


def mask_c(r):
    """Query-row offset (within the tile, lane half aside) of accumulator register r."""
    return (r // 4) * 8 + (r % 4)


class Body:
    def __init__(self, p: Prog):
        self.p = p

    def s(self, text, reads=(), writes=()):
        self.p.salu(text, reads, writes)

    # ---------------------------------------------------------------- descriptors
    def rsrc(self, dst, base_lo, off_rows_sgpr, stride_sgpr, rows_sgpr, extra_sgpr=None):
        """dst = buffer descriptor for base + off_rows*stride (+ extra), rows*stride bytes."""
        s, T = self.s, S_TMP + 12
        s(f"s_mul_i32 {sr(T)}, {sr(off_rows_sgpr)}, {sr(stride_sgpr)}", S(off_rows_sgpr) + S(stride_sgpr), S(T))
        s(f"s_mul_hi_u32 {sr(T + 1)}, {sr(off_rows_sgpr)}, {sr(stride_sgpr)}", S(off_rows_sgpr) + S(stride_sgpr), S(T + 1))
        if extra_sgpr is not None:
            s(f"s_add_u32 {sr(T)}, {sr(T)}, {sr(extra_sgpr)}", S(T) + S(extra_sgpr), S(T) + [("scc", 0)])
            s(f"s_addc_u32 {sr(T + 1)}, {sr(T + 1)}, 0", S(T + 1) + [("scc", 0)], S(T + 1))
        s(f"s_add_u32 {sr(dst)}, {sr(base_lo)}, {sr(T)}", S(base_lo) + S(T), S(dst) + [("scc", 0)])
        s(f"s_addc_u32 {sr(dst + 1)}, {sr(base_lo + 1)}, {sr(T + 1)}", S(base_lo + 1) + S(T + 1) + [("scc", 0)], S(dst + 1))
        s(f"s_and_b32 {sr(dst + 1)}, {sr(dst + 1)}, 0xffff", S(dst + 1), S(dst + 1))
        s(f"s_mul_i32 {sr(dst + 2)}, {sr(rows_sgpr)}, {sr(stride_sgpr)}", S(rows_sgpr) + S(stride_sgpr), S(dst + 2))
        s(f"s_mov_b32 {sr(dst + 3)}, 0x20000", [], S(dst + 3))

    def tile_rsrcs(self, it_sgpr, h_sgpr, qt_sgpr):
        """Descriptors of tile (head offset h, q-tile qt) for DMA; empty when it >= iters."""
        s = self.s
        T0, T1, T2, T3, T4 = S_TMP, S_TMP + 1, S_TMP + 2, S_TMP + 3, S_TMP + 4
        # rows = it < iters ? min(32, S - qt*32) : 0 ; r0 = qt*32
        s(f"s_lshl_b32 {sr(T0)}, {sr(qt_sgpr)}, 5", S(qt_sgpr), S(T0))
        s(f"s_sub_u32 {sr(T1)}, {sr(S_SEQ)}, {sr(T0)}", S(S_SEQ) + S(T0), S(T1))
        s(f"s_min_i32 {sr(T1)}, {sr(T1)}, 32", S(T1), S(T1))
        s(f"s_cmp_lt_u32 {sr(it_sgpr)}, {sr(S_ITERS)}", S(it_sgpr) + S(S_ITERS), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T1)}, {sr(T1)}, 0", S(T1) + [("scc", 0)], S(T1))
        # head column offset h*256 (bytes) for Q / dO; LSE/D row offset (h*S + r0)
        s(f"s_lshl_b32 {sr(T2)}, {sr(h_sgpr)}, 8", S(h_sgpr), S(T2))
        self.rsrc(S_RQ, S_BQKV, T0, S_LDB, T1, T2)
        self.rsrc(S_RO, S_BDO, T0, S_LDO, T1, T2)
        s(f"s_mul_i32 {sr(T3)}, {sr(h_sgpr)}, {sr(S_SEQ)}", S(h_sgpr) + S(S_SEQ), S(T3))
        s(f"s_add_u32 {sr(T3)}, {sr(T3)}, {sr(T0)}", S(T3) + S(T0), S(T3))
        s(f"s_mov_b32 {sr(T4)}, 4", [], S(T4))
        # LSE for wave 0, D for wave 1, nothing for waves 2, 3
        TB = S_TMP + 14
        s(f"s_cmp_eq_u32 {sr(S_SMALLSEL)}, 1", S(S_SMALLSEL), [("scc", 0)])
        s(f"s_cselect_b64 {sr(TB, 2)}, {sr(S_BDEL, 2)}, {sr(S_BLSE, 2)}", S(S_BDEL, 2) + S(S_BLSE, 2) + [("scc", 0)], S(TB, 2))
        s(f"s_cmp_lt_u32 {sr(S_SMALLSEL)}, 2", S(S_SMALLSEL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T1)}, {sr(T1)}, 0", S(T1) + [("scc", 0)], S(T1))
        self.rsrc(S_RL, TB, T3, T4, T1)

    # ---------------------------------------------------------------- DMA
    def dma_m0(self, which, jb, i=0):
        s = self.s
        if which == "q":
            s(f"s_add_u32 m0, {sr(S_LDSW)}, {jb * BUFB + i * 1024}", S(S_LDSW), [("m0", 0)])
        elif which == "o":
            s(f"s_add_u32 m0, {sr(S_LDSW)}, {jb * BUFB + TILE + i * 1024}", S(S_LDSW), [("m0", 0)])
        else:
            s(f"s_add_u32 m0, {sr(S_LDSL)}, {jb * LDB}", S(S_LDSL), [("m0", 0)])

    def dma_ld(self, which, i=0):
        if which == "q":
            self.p.dma(f"buffer_load_dwordx4 {vr(V_DOFF + i)}, {sr(S_RQ, 4)}, 0 offen lds", V(V_DOFF + i) + S(S_RQ, 4))
        elif which == "o":
            self.p.dma(f"buffer_load_dwordx4 {vr(V_DOFF + 2 + i)}, {sr(S_RO, 4)}, 0 offen lds", V(V_DOFF + 2 + i) + S(S_RO, 4))
        else:
            self.p.dma(f"buffer_load_dword {vr(V_LOFF)}, {sr(S_RL, 4)}, 0 offen lds", V(V_LOFF) + S(S_RL, 4))

    DMA_ORDER = (("q", 0), ("q", 1), ("o", 0), ("o", 1), ("l", 0))

    def dma_all(self, jb):
        for which, i in self.DMA_ORDER:
            self.dma_m0(which, jb, i)
            self.dma_ld(which, i)

    # ---------------------------------------------------------------- LDS reads
    def row_read(self, i, jb):
        """Read for S/dP MFMA i (ks = i // 2; even: Q row, odd: dO row) of tile buffer jb."""
        ks, which = i // 2, i % 2
        dst = V_RB + (i % NRB) * 4
        off = jb * BUFB + which * TILE
        self.p.ds_read(f"ds_read_b128 {vr(dst, 4)}, {vr(V_KOFF + ks)} offset:{off}", V(dst, 4), V(V_KOFF + ks))

    def tr_read(self, j, jb):
        """Reads for dV/dK MFMA j (ks = j // 8; j % 8 < 4: dO^T for dV, else Q^T for dK,
        db = j % 4) of tile buffer jb."""
        ks, k8 = j // 8, j % 8
        db = k8 % 4
        which = 1 if k8 < 4 else 0
        dst = V_TB + (j % NTB) * 4
        off = jb * BUFB + which * TILE + ks * 16 * ROWB
        for tt in range(2):
            self.p.ds_read(f"ds_read_b64_tr_b16 {vr(dst + 2 * tt, 2)}, {vr(V_VOFF + tt * 4 + db)} offset:{off}",
                           V(dst + 2 * tt, 2), V(V_VOFF + tt * 4 + db))

    def cinit_reads(self, jb, part):
        """LSE (part 0) or D (part 1) of the tile in buffer jb into the start values."""
        base = V_CS if part == 0 else V_CD
        for g4 in range(4):
            self.p.ds_read(f"ds_read_b128 {vr(base + 4 * g4, 4)}, {vr(V_LDR)} offset:{jb * LDB + part * 256 + g4 * 32}",
                           V(base + 4 * g4, 4), V(V_LDR))

    def cinit_fix(self, k):
        """Start values 4k..4k+3 of both sets: -LSE*log2e and -D."""
        for r in range(4 * k, 4 * k + 4):
            self.p.valu(f"v_mul_f32_e32 {vr(V_CS + r)}, {NEG_LOG2E}, {vr(V_CS + r)}", V(V_CS + r), V(V_CS + r))
            self.p.valu(f"v_sub_f32_e32 {vr(V_CD + r)}, 0, {vr(V_CD + r)}", V(V_CD + r), V(V_CD + r))

    # ---------------------------------------------------------------- MFMAs
    def sdp_mfma(self, i, J):
        ks, which = i // 2, i % 2
        dst = V_SD[J] + 16 * which
        c = (V_CS if which == 0 else V_CD) if ks == 0 else dst
        b = (A_K if which == 0 else A_V) + ks * 4
        self.p.mfma(MFMA, dst, V_RB + (i % NRB) * 4, b, c, b_acc=True)

    def dvdk_mfma(self, j):
        ks, k8 = j // 8, j % 8
        db = k8 % 4
        if k8 < 4:
            acc, b = A_DV + db * 16, V_P + ks * 4
        else:
            acc, b = A_DK + db * 16, V_DS + ks * 4
        self.p.mfma(MFMA, acc, V_TB + (j % NTB) * 4, b, acc, dst_acc=True)

    # ---------------------------------------------------------------- elementwise (set J)
    def ew_exp(self, J, n):
        for r in (2 * n, 2 * n + 1):
            x = V_SD[J] + r
            self.p.trans(f"v_exp_f32_e32 {vr(x)}, {vr(x)}", V(x), V(x))

    def ew_rest(self, J, n, masked):
        p = self.p
        g4 = n // 2
        ks, w = g4 >> 1, (g4 & 1) * 2 + (n & 1)
        for r in (2 * n, 2 * n + 1):
            x, dp = V_SD[J] + r, V_SD[J] + 16 + r
            if masked:
                p.valu(f"v_cmp_lt_i32_e32 vcc, {mask_c(r)}, {vr(V_TK)}", V(V_TK), [("vcc", 0)])
                p.valu(f"v_cndmask_b32_e64 {vr(x)}, {vr(x)}, 0, vcc", V(x) + [("vcc", 0)], V(x))
            p.valu(f"v_mul_f32_e32 {vr(dp)}, {vr(x)}, {vr(dp)}", V(x) + V(dp), V(dp))
        x, dp = V_SD[J] + 2 * n, V_SD[J] + 16 + 2 * n
        p.valu(f"v_cvt_pk_f16_f32 {vr(V_P + ks * 4 + w)}, {vr(x)}, {vr(x + 1)}", V(x, 2), V(V_P + ks * 4 + w))
        p.valu(f"v_cvt_pk_f16_f32 {vr(V_DS + ks * 4 + w)}, {vr(dp)}, {vr(dp + 1)}", V(dp, 2), V(V_DS + ks * 4 + w))

    def mask_threshold(self, qt_sgpr):
        """tk = key >= kv_len ? 32 : (causal ? kw0 - qr0 + l32 - 4hi : -32); an element of
        register r is hidden iff mask_c(r) < tk."""
        s, p = self.s, self.p
        T0, T1 = S_TMP + 5, S_TMP + 6
        s(f"s_lshl_b32 {sr(T0)}, {sr(qt_sgpr)}, 5", S(qt_sgpr), S(T0))
        s(f"s_sub_u32 {sr(T0)}, {sr(S_KW0)}, {sr(T0)}", S(S_KW0) + S(T0), S(T0))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T0)}, 0xffffffa0, {sr(T0)}", S(T0) + [("scc", 0)], S(T0))  # -96: no causal mask
        p.valu(f"v_add_u32_e32 {vr(V_TK)}, {sr(T0)}, {vr(V_L32)}", S(T0) + V(V_L32), V(V_TK))
        p.valu(f"v_sub_u32_e32 {vr(V_TK)}, {vr(V_TK)}, {vr(V_HI4)}", V(V_TK) + V(V_HI4), V(V_TK))
        # keys at or past kv_len: hide everything
        s(f"s_sub_u32 {sr(T1)}, {sr(S_KVL)}, {sr(S_KW0)}", S(S_KVL) + S(S_KW0), S(T1))
        p.valu(f"v_cmp_le_i32_e32 vcc, {sr(T1)}, {vr(V_L32)}", S(T1) + V(V_L32), [("vcc", 0)])
        p.valu(f"v_cndmask_b32_e64 {vr(V_TK)}, {vr(V_TK)}, 32, vcc", V(V_TK) + [("vcc", 0)], V(V_TK))

    # ---------------------------------------------------------------- iteration bodies
    def body(self, u, sdp, ew, masked):
        """Iteration it with it % 4 == u: S/dP of tile it+1 (sdp), elementwise + dV/dK of tile
        it (ew), barrier, LSE/D of tile it+2, DMA of tile it+3."""
        p = self.p
        J0, J1 = u % 2, (u + 1) % 2
        jb0, jb1, jb2, jb3 = u, (u + 1) % 4, (u + 2) % 4, (u + 3) % 4
        # --- first half: S/dP(it+1) with elementwise(it) between the MFMAs; the first LK row
        # reads of tile it+1 were issued at the end of the previous body
        rissued = LK
        tissued = 0
        if ew and masked:
            self.mask_threshold(S_QT0)
        nslots = 16 if sdp else 0
        half_steps = list(range(16)) if ew else []
        for s_ in range(nslots):
            while rissued < 16 and rissued - LK <= s_:
                self.row_read(rissued, jb1)
                rissued += 1
            if ew:
                while tissued < 16 and 16 + tissued - LV <= s_:
                    self.tr_read(tissued, jb0)
                    tissued += 1
            self.sdp_mfma(s_, J1)
            if ew:
                h = half_steps[s_]
                if h % 2 == 0:
                    self.ew_exp(J0, h // 2)
                else:
                    self.ew_rest(J0, h // 2, masked)
        if ew and not sdp:
            for n in range(9):
                if n < 8:
                    self.ew_exp(J0, n)
                if n >= 1:
                    self.ew_rest(J0, n - 1, masked)
        # --- barrier: every wave is past the reads of tile it-1; tile it+2 is in LDS
        p.waitcnt(vm=0)
        p.barrier()
        # --- second half: dV/dK(it); LSE/D of tile it+2; DMA of tile it+3
        dma_at = {18: 0, 21: 1, 24: 2, 27: 3, 30: 4}
        for s_ in range(16, 32):
            if ew:
                while tissued < 16 and 16 + tissued - LV <= s_:
                    self.tr_read(tissued, jb0)
                    tissued += 1
            if s_ in (16, 17):
                self.cinit_reads(jb2, s_ - 16)
            if s_ in dma_at:
                which, i = self.DMA_ORDER[dma_at[s_]]
                self.dma_m0(which, jb3, i)
            if ew:
                self.dvdk_mfma(s_ - 16)
            if 20 <= s_ < 24:
                self.cinit_fix(s_ - 20)
            if s_ in dma_at:
                which, i = self.DMA_ORDER[dma_at[s_]]
                self.dma_ld(which, i)
            if s_ >= 32 - LK:   # first row reads of tile it+2 for the next body
                self.row_read(s_ - (32 - LK), jb2)


def build(check_ldb: int = 12288, check_ldo: int = 4096) -> str:
    p = Prog()
    sal = p.salu
    # ---------------------------------------------------------------- scalars
    p.smem(f"s_load_dwordx16 {sr(8, 16)}, {sr(0, 2)}, 0x0", S(8, 16), S(0, 2))
    p.smem(f"s_load_dwordx8 {sr(24, 8)}, {sr(0, 2)}, 0x40", S(24, 8), S(0, 2))
    L = Lanes(p, check_ldb)
    L.shr(V_PT + 0, L.k(6), 0)
    p.readlane(f"v_readfirstlane_b32 {sr(S_WAVE)}, {vr(V_PT + 0)}", V(V_PT + 0), S(S_WAVE))
    p.waitcnt(lgkm=0)
    T0, T1, T2, T3 = S_TMP, S_TMP + 1, S_TMP + 2, S_TMP + 3
    # kv_len
    sal(f"s_mov_b32 {sr(S_KVL)}, {sr(S_SEQ)}", S(S_SEQ), S(S_KVL))
    sal(f"s_cmp_eq_u64 {sr(S_KVLEN, 2)}, 0", S(S_KVLEN, 2), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lkvl_done", [("scc", 0)])
    sal(f"s_lshl_b32 {sr(T0)}, {sr(S_B)}, 2", S(S_B), S(T0))
    p.smem(f"s_load_dword {sr(S_KVL)}, {sr(S_KVLEN, 2)}, {sr(T0)}", S(S_KVL), S(S_KVLEN, 2) + S(T0))
    p.waitcnt(lgkm=0)
    sal(f"s_max_i32 {sr(S_KVL)}, {sr(S_KVL)}, 0", S(S_KVL), S(S_KVL))
    sal(f"s_min_i32 {sr(S_KVL)}, {sr(S_KVL)}, {sr(S_SEQ)}", S(S_KVL) + S(S_SEQ), S(S_KVL))
    p.label(".Lkvl_done")
    # key block, this wave's keys
    sal(f"s_lshl_b32 {sr(S_KB0)}, {sr(S_Z)}, 7", S(S_Z), S(S_KB0))
    sal(f"s_lshl_b32 {sr(T0)}, {sr(S_WAVE)}, 5", S(S_WAVE), S(T0))
    sal(f"s_add_u32 {sr(S_KW0)}, {sr(S_KB0)}, {sr(T0)}", S(S_KB0) + S(T0), S(S_KW0))
    sal(f"s_cmp_lt_u32 {sr(S_KW0)}, {sr(S_KVL)}", S(S_KW0) + S(S_KVL), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(S_KWACT)}, 1, 0", [("scc", 0)], S(S_KWACT))
    sal(f"s_add_u32 {sr(T0)}, {sr(S_KW0)}, 32", S(S_KW0), S(T0))
    sal(f"s_cmp_gt_u32 {sr(T0)}, {sr(S_KVL)}", S(T0) + S(S_KVL), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(S_KWMASK)}, 1, 0", [("scc", 0)], S(S_KWMASK))
    # q-tiles: [qt_begin, qt_end) per head; iters = g * (qt_end - qt_begin)
    sal(f"s_add_u32 {sr(T0)}, {sr(S_SEQ)}, 31", S(S_SEQ), S(T0))
    sal(f"s_lshr_b32 {sr(S_QTE)}, {sr(T0)}, 5", S(T0), S(S_QTE))
    sal(f"s_lshr_b32 {sr(T0)}, {sr(S_KB0)}, 5", S(S_KB0), S(T0))
    sal(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(S_QTB)}, 0, {sr(T0)}", S(T0) + [("scc", 0)], S(S_QTB))
    sal(f"s_sub_u32 {sr(T0)}, {sr(S_QTE)}, {sr(S_QTB)}", S(S_QTE) + S(S_QTB), S(T0))
    sal(f"s_mul_i32 {sr(S_ITERS)}, {sr(T0)}, {sr(S_G)}", S(T0) + S(S_G), S(S_ITERS))
    # batch bases: qkv + b*S*ldb (Q columns of the group's first head at + kvh*g*256);
    # dout + b*S*ldo + kvh*g*256; lse/delta + (b*Hq + kvh*g)*S*4
    sal(f"s_mul_i32 {sr(T0)}, {sr(S_B)}, {sr(S_SEQ)}", S(S_B) + S(S_SEQ), S(T0))
    sal(f"s_mul_i32 {sr(T1)}, {sr(S_H)}, {sr(S_G)}", S(S_H) + S(S_G), S(T1))           # first q-head
    sal(f"s_lshl_b32 {sr(T2)}, {sr(T1)}, 8", S(T1), S(T2))
    for base, src, stride in ((S_BQKV, S_QKV, S_LDB), (S_BDO, S_DOUT, S_LDO)):
        sal(f"s_mul_i32 {sr(T3)}, {sr(T0)}, {sr(stride)}", S(T0) + S(stride), S(T3))
        sal(f"s_mul_hi_u32 {sr(S_TMP + 4)}, {sr(T0)}, {sr(stride)}", S(T0) + S(stride), S(S_TMP + 4))
        sal(f"s_add_u32 {sr(T3)}, {sr(T3)}, {sr(T2)}", S(T3) + S(T2), S(T3) + [("scc", 0)])
        sal(f"s_addc_u32 {sr(S_TMP + 4)}, {sr(S_TMP + 4)}, 0", S(S_TMP + 4) + [("scc", 0)], S(S_TMP + 4))
        sal(f"s_add_u32 {sr(base)}, {sr(src)}, {sr(T3)}", S(src) + S(T3), S(base) + [("scc", 0)])
        sal(f"s_addc_u32 {sr(base + 1)}, {sr(src + 1)}, {sr(S_TMP + 4)}", S(src + 1) + S(S_TMP + 4) + [("scc", 0)], S(base + 1))
    sal(f"s_mul_i32 {sr(T3)}, {sr(S_B)}, {sr(S_HQ)}", S(S_B) + S(S_HQ), S(T3))
    sal(f"s_add_u32 {sr(T3)}, {sr(T3)}, {sr(T1)}", S(T3) + S(T1), S(T3))
    sal(f"s_mul_i32 {sr(T3)}, {sr(T3)}, {sr(S_SEQ)}", S(T3) + S(S_SEQ), S(T3))
    sal(f"s_mul_hi_u32 {sr(S_TMP + 4)}, {sr(T3)}, 4", S(T3), S(S_TMP + 4))
    sal(f"s_lshl_b32 {sr(T3)}, {sr(T3)}, 2", S(T3), S(T3))
    for base, src in ((S_BLSE, S_LSE), (S_BDEL, S_DELTA)):
        sal(f"s_add_u32 {sr(base)}, {sr(src)}, {sr(T3)}", S(src) + S(T3), S(base) + [("scc", 0)])
        sal(f"s_addc_u32 {sr(base + 1)}, {sr(src + 1)}, {sr(S_TMP + 4)}", S(src + 1) + S(S_TMP + 4) + [("scc", 0)], S(base + 1))
    # the Q base above points at the group's first q-head columns: the K and V columns of the
    # kv head are at + (Hq - kvh*g + kvh)*256 and + (Hq + Hkv - kvh*g + kvh)*256 from it
    # (handled with the batch base below)
    # DMA placement
    sal(f"s_lshl_b32 {sr(S_LDSW)}, {sr(S_WAVE)}, 11", S(S_WAVE), S(S_LDSW))          # wave * 2 KB
    sal(f"s_min_u32 {sr(S_SMALLSEL)}, {sr(S_WAVE)}, 2", S(S_WAVE), S(S_SMALLSEL))
    sal(f"s_lshl_b32 {sr(S_LDSL)}, {sr(S_WAVE)}, 8", S(S_WAVE), S(S_LDSL))
    sal(f"s_add_u32 {sr(S_LDSL)}, {sr(S_LDSL)}, {LDS_LD}", S(S_LDSL), S(S_LDSL))
    # a workgroup whose keys all lie at or past kv_len only writes zero gradients
    sal(f"s_cmp_ge_u32 {sr(S_KB0)}, {sr(S_KVL)}", S(S_KB0) + S(S_KVL), [("scc", 0)])
    sal(f"s_cselect_b32 {sr(S_ITERS)}, 0, {sr(S_ITERS)}", S(S_ITERS) + [("scc", 0)], S(S_ITERS))

    # ---------------------------------------------------------------- lane values
    LANE, L32, HI = V_PT + 1, V_PT + 2, V_PT + 3
    DR, DP, TA, TB, TC = V_PT + 4, V_PT + 5, V_PT + 6, V_PT + 7, V_PT + 8
    lane_basics(L, (LANE, L32, HI))
    L.shr(DR, L.k(4), LANE)
    L.and_(DP, L.k(15), LANE)
    # DMA: wave w, instruction i moves rows w*8 + i*4 + dr: chunk dp ^ swz(row) of row
    # -> LDS slot dp; swz(row) = 4*dr + ((2w + i) & 3)
    wave_vals = np.arange(4)
    L.shl(TA, L.k(2), DR)
    T3 = S_TMP + 3
    for i in range(2):
        sal(f"s_lshl_b32 {sr(T3)}, {sr(S_WAVE)}, 1", S(S_WAVE), S(T3))
        sal(f"s_add_u32 {sr(T3)}, {sr(T3)}, {i}", S(T3), S(T3))
        sal(f"s_and_b32 {sr(T3)}, {sr(T3)}, 3", S(T3), S(T3))
        L.or_(TC, TA, L.s(T3, (2 * wave_vals + i) & 3))
        L.xor(TC, TC, DP)
        L.shl(TC, L.k(4), TC)
        sal(f"s_lshl_b32 {sr(T3)}, {sr(S_WAVE)}, 3", S(S_WAVE), S(T3))
        sal(f"s_add_u32 {sr(T3)}, {sr(T3)}, {4 * i}", S(T3), S(T3))
        L.add(TB, DR, L.s(T3, wave_vals * 8 + 4 * i))
        L.mul(V_DOFF + i, TB, L.s(S_LDB, np.full(4, check_ldb)))
        L.add(V_DOFF + i, V_DOFF + i, TC)
        L.mul(V_DOFF + 2 + i, TB, L.s(S_LDO, np.full(4, check_ldo)))
        L.add(V_DOFF + 2 + i, V_DOFF + 2 + i, TC)
    L.shl(V_LOFF, L.k(2), LANE)
    row_read_offsets(L, V_KOFF, (LANE, L32, HI), (TA, TB, TC))
    tr_read_offsets(L, V_VOFF, (LANE, L32, HI), (TA, TB, TC, V_PT + 9, V_PT + 10, V_PT + 11, V_PT + 12))
    _check_dma(L, check_ldb, check_ldo)
    p.valu(f"v_mov_b32_e32 {vr(V_L32)}, {vr(L32)}", V(L32), V(V_L32))
    p.valu(f"v_lshlrev_b32_e32 {vr(V_HI4)}, 2, {vr(HI)}", V(HI), V(V_HI4))
    p.valu(f"v_lshlrev_b32_e32 {vr(V_LDR)}, 4, {vr(HI)}", V(HI), V(V_LDR))
    p.valu(f"v_add_u32_e32 {vr(V_LDR)}, {LDS_LD}, {vr(V_LDR)}", V(V_LDR), V(V_LDR))
    return _rest(p)


def _check_dma(L: Lanes, ldb, ldo):
    tid = np.arange(256)
    lane, wave = tid & 63, tid >> 6
    dr, dp = lane // 16, lane % 16
    for i in range(2):
        row = wave * 8 + i * 4 + dr
        chunk = (dp ^ np.vectorize(swz)(row)) << 4
        assert np.array_equal(L.val[V_DOFF + i], (row * ldb + chunk) & 0xFFFFFFFF), f"Q dma {i}"
        assert np.array_equal(L.val[V_DOFF + 2 + i], (row * ldo + chunk) & 0xFFFFFFFF), f"dO dma {i}"
    assert np.array_equal(L.val[V_LOFF], lane * 4)


def _rest(p: Prog) -> str:
    b = Body(p)
    s = b.s
    T0, T1, T2, T3 = S_TMP, S_TMP + 1, S_TMP + 2, S_TMP + 3
    # ---------------------------------------------------------------- first tiles in flight
    s(f"s_mov_b32 {sr(S_IT)}, 0", [], S(S_IT))
    s(f"s_mov_b32 {sr(S_H3)}, 0", [], S(S_H3))
    s(f"s_mov_b32 {sr(S_QT3)}, {sr(S_QTB)}", S(S_QTB), S(S_QT3))
    for t in range(3):
        s(f"s_mov_b32 {sr(S_TMP + 8)}, {t}", [], S(S_TMP + 8))
        b.tile_rsrcs(S_TMP + 8, S_H3, S_QT3)
        b.dma_all(t)
        _advance(b, S_H3, S_QT3)
    # ---------------------------------------------------------------- K, V of the wave's keys
    # lane (l32, hi): key kw0 + l32, head-dim elements ks*16 + hi*8 .. +7
    RK, RV = S_RQ, S_RO    # reuse: the tile descriptors are rebuilt per tile afterwards
    # K base = batch base + (Hq + kvh)*256 ; rows = clamp(kv_len - kw0, 0, 32) ; start row kw0
    s(f"s_sub_u32 {sr(T1)}, {sr(S_KVL)}, {sr(S_KW0)}", S(S_KVL) + S(S_KW0), S(T1))
    s(f"s_max_i32 {sr(T1)}, {sr(T1)}, 0", S(T1), S(T1))
    s(f"s_min_i32 {sr(T1)}, {sr(T1)}, 32", S(T1), S(T1))
    # S_BQKV points at the group's first q-head columns (kvh*g*256): K columns are at
    # (Hq + kvh)*256 - kvh*g*256 from it, V columns Hkv*256 further
    s(f"s_mul_i32 {sr(T2)}, {sr(S_H)}, {sr(S_G)}", S(S_H) + S(S_G), S(T2))
    s(f"s_sub_u32 {sr(T2)}, {sr(S_H)}, {sr(T2)}", S(S_H) + S(T2), S(T2))
    s(f"s_add_u32 {sr(T2)}, {sr(T2)}, {sr(S_HQ)}", S(T2) + S(S_HQ), S(T2))
    s(f"s_lshl_b32 {sr(T2)}, {sr(T2)}, 8", S(T2), S(T2))
    b.rsrc(RK, S_BQKV, S_KW0, S_LDB, T1, T2)
    s(f"s_lshl_b32 {sr(T3)}, {sr(S_HKV)}, 8", S(S_HKV), S(T3))
    s(f"s_add_u32 {sr(T2)}, {sr(T2)}, {sr(T3)}", S(T2) + S(T3), S(T2))
    b.rsrc(RV, S_BQKV, S_KW0, S_LDB, T1, T2)
    KO = V_T   # row offset l32*ldb + hi*16
    p.valu(f"v_mul_lo_u32 {vr(KO)}, {vr(V_L32)}, {sr(S_LDB)}", V(V_L32) + S(S_LDB), V(KO))
    p.valu(f"v_lshl_add_u32 {vr(KO)}, {vr(V_HI4)}, 2, {vr(KO)}", V(V_HI4) + V(KO), V(KO))
    for ks in range(8):
        p.vmem_load(f"buffer_load_dwordx4 {vr(ks * 4, 4)}, {vr(KO)}, {sr(RK, 4)}, 0 offen offset:{ks * 32}",
                    V(ks * 4, 4), V(KO) + S(RK, 4))
    for ks in range(8):
        p.vmem_load(f"buffer_load_dwordx4 {vr(32 + ks * 4, 4)}, {vr(KO)}, {sr(RV, 4)}, 0 offen offset:{ks * 32}",
                    V(32 + ks * 4, 4), V(KO) + S(RV, 4))
    for i in range(128):
        p.valu(f"v_accvgpr_write_b32 {ar(A_DV + i)}, 0", [], A(A_DV + i))
    t0, t1 = V_T + 1, V_T + 2
    for i in range(32):   # K * scale*log2e, rounded to fp16
        p.valu(f"v_fma_mix_f32 {vr(t0)}, {vr(i)}, {sr(S_SL2)}, 0 op_sel_hi:[1,0,0]", V(i) + S(S_SL2), V(t0))
        p.valu(f"v_fma_mix_f32 {vr(t1)}, {vr(i)}, {sr(S_SL2)}, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]", V(i) + S(S_SL2), V(t1))
        p.valu(f"v_cvt_pk_f16_f32 {vr(i)}, {vr(t0)}, {vr(t1)}", V(t0, 2), V(i))
        p.valu(f"v_accvgpr_write_b32 {ar(A_K + i)}, {vr(i)}", V(i), A(A_K + i))
    for i in range(32):
        p.valu(f"v_accvgpr_write_b32 {ar(A_V + i)}, {vr(32 + i)}", V(32 + i), A(A_V + i))
    # ---------------------------------------------------------------- tile 0
    p.waitcnt(vm=0)
    p.barrier()
    s(f"s_mov_b32 {sr(S_QT0)}, {sr(S_QTB)}", S(S_QTB), S(S_QT0))
    s(f"s_mov_b32 {sr(S_QT1)}, {sr(S_QTB)}", S(S_QTB), S(S_QT1))
    b.cinit_reads(0, 0)
    b.cinit_reads(0, 1)
    for k in range(4):
        b.cinit_fix(k)
    # S/dP(0) if tile 0 is active for this wave
    _active(b, S_QT0, T0)
    s(f"s_cmp_eq_u32 {sr(T0)}, 0", S(T0), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lpro_skip", [("scc", 0)])
    rissued = 0
    for i in range(16):
        while rissued < 16 and rissued - LK <= i:
            b.row_read(rissued, 0)
            rissued += 1
        b.sdp_mfma(i, 0)
    p.label(".Lpro_skip")
    _advance_qt(b, S_QT1)
    b.cinit_reads(1, 0)
    b.cinit_reads(1, 1)
    for k in range(4):
        b.cinit_fix(k)
    for i in range(LK):
        b.row_read(i, 1)
    # ---------------------------------------------------------------- tile loop
    p.label(".Lloop")
    for u in range(4):
        _loop_body(b, u)
    p.branch("s_branch .Lloop")
    p.label(".Lloop_done")
    p.waitcnt(vm=0)   # the last (empty) tile requests still write LDS
    # ---------------------------------------------------------------- epilogue
    # dK^T * scale, dV^T: lane holds key kw0 + l32, d = db*32 + g4*8 + hi*4 + 0..3
    s(f"s_mov_b32 {sr(T1)}, {sr(S_SEQ)}", S(S_SEQ), S(T1))
    s(f"s_mov_b32 {sr(T3)}, 0", [], S(T3))
    s(f"s_add_u32 {sr(T2)}, {sr(S_HQ)}, {sr(S_H)}", S(S_HQ) + S(S_H), S(T2))
    s(f"s_lshl_b32 {sr(T2)}, {sr(T2)}, 8", S(T2), S(T2))
    # base: dqkv + b*S*ldb + column; rows [0, S)
    s(f"s_mul_i32 {sr(T0)}, {sr(S_B)}, {sr(S_SEQ)}", S(S_B) + S(S_SEQ), S(T0))
    b.rsrc(S_RQ, S_DQKV, T0, S_LDB, T1, T2)
    s(f"s_lshl_b32 {sr(T3)}, {sr(S_HKV)}, 8", S(S_HKV), S(T3))
    s(f"s_add_u32 {sr(T2)}, {sr(T2)}, {sr(T3)}", S(T2) + S(T3), S(T2))
    b.rsrc(S_RO, S_DQKV, T0, S_LDB, T1, T2)
    OO = V_T
    p.valu(f"v_add_u32_e32 {vr(OO)}, {sr(S_KW0)}, {vr(V_L32)}", S(S_KW0) + V(V_L32), V(OO))
    p.valu(f"v_mul_lo_u32 {vr(OO)}, {vr(OO)}, {sr(S_LDB)}", V(OO) + S(S_LDB), V(OO))
    p.valu(f"v_lshl_add_u32 {vr(OO)}, {vr(V_HI4)}, 1, {vr(OO)}", V(V_HI4) + V(OO), V(OO))
    W = 0
    for acc, rs, scale in ((A_DK, S_RQ, True), (A_DV, S_RO, False)):
        for db in range(4):
            for g4 in range(4):
                a0 = acc + db * 16 + g4 * 4
                for j in range(4):
                    p.valu(f"v_accvgpr_read_b32 {vr(W + j)}, {ar(a0 + j)}", A(a0 + j), V(W + j))
                if scale:
                    for j in range(4):
                        p.valu(f"v_mul_f32_e32 {vr(W + j)}, {sr(S_SCALE)}, {vr(W + j)}", V(W + j) + S(S_SCALE), V(W + j))
                p.valu(f"v_cvt_pk_f16_f32 {vr(W + 4)}, {vr(W)}, {vr(W + 1)}", V(W, 2), V(W + 4))
                p.valu(f"v_cvt_pk_f16_f32 {vr(W + 5)}, {vr(W + 2)}, {vr(W + 3)}", V(W + 2, 2), V(W + 5))
                p.vmem_store(f"buffer_store_dwordx2 {vr(W + 4, 2)}, {vr(OO)}, {sr(rs, 4)}, 0 offen offset:{db * 64 + g4 * 16}",
                             V(W + 4, 2) + V(OO) + S(rs, 4))
                W = 8 if W == 0 else 0
    p.emit("s_endpgm", BRANCH)
    return kernel_text(NAME, p.finalize(), lds_bytes=LDS_BYTES, kernarg_bytes=KERNARG_BYTES,
                       next_free_sgpr=NEXT_FREE_SGPR, args=ARGS)


def _advance_qt(b: Body, qt):
    """qt := qt + 1, wrapping to qt_begin at qt_end."""
    s = b.s
    s(f"s_add_u32 {sr(qt)}, {sr(qt)}, 1", S(qt), S(qt))
    s(f"s_cmp_ge_u32 {sr(qt)}, {sr(S_QTE)}", S(qt) + S(S_QTE), [("scc", 0)])
    s(f"s_cselect_b32 {sr(qt)}, {sr(S_QTB)}, {sr(qt)}", S(S_QTB) + S(qt) + [("scc", 0)], S(qt))


def _advance(b: Body, h, qt):
    """(h, qt) := next tile: qt + 1, or (h + 1, qt_begin) at qt_end."""
    s = b.s
    s(f"s_add_u32 {sr(qt)}, {sr(qt)}, 1", S(qt), S(qt))
    s(f"s_cmp_ge_u32 {sr(qt)}, {sr(S_QTE)}", S(qt) + S(S_QTE), [("scc", 0)])
    s(f"s_cselect_b32 {sr(qt)}, {sr(S_QTB)}, {sr(qt)}", S(S_QTB) + S(qt) + [("scc", 0)], S(qt))
    s(f"s_addc_u32 {sr(h)}, {sr(h)}, 0", S(h) + [("scc", 0)], S(h))


def _active(b: Body, qt, dst):
    """dst = 1 if q-tile qt holds a row that sees a key of this wave: the wave has a key
    below kv_len and (not causal, or qt*32 + 31 >= kw0, i.e. qt*32 >= kw0)."""
    s = b.s
    T = S_TMP + 7
    s(f"s_lshl_b32 {sr(T)}, {sr(qt)}, 5", S(qt), S(T))
    s(f"s_cmp_ge_u32 {sr(T)}, {sr(S_KW0)}", S(T) + S(S_KW0), [("scc", 0)])
    s(f"s_cselect_b32 {sr(dst)}, 1, 0", [("scc", 0)], S(dst))
    s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
    s(f"s_cselect_b32 {sr(dst)}, 1, {sr(dst)}", S(dst) + [("scc", 0)], S(dst))
    s(f"s_and_b32 {sr(dst)}, {sr(dst)}, {sr(S_KWACT)}", S(dst) + S(S_KWACT), S(dst))


def _loop_body(b: Body, u: int):
    p, s = b.p, b.s
    A0, A1, MK = S_TMP + 8, S_TMP + 9, S_TMP + 10
    p.label(f".Lb{u}")
    s(f"s_cmp_ge_u32 {sr(S_IT)}, {sr(S_ITERS)}", S(S_IT) + S(S_ITERS), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lloop_done", [("scc", 0)])
    # descriptors of tile it+3
    s(f"s_add_u32 {sr(S_TMP + 11)}, {sr(S_IT)}, 3", S(S_IT), S(S_TMP + 11))
    b.tile_rsrcs(S_TMP + 11, S_H3, S_QT3)
    # flags: act0 (tile it), act1 (tile it+1 exists and is active), masked (tile it)
    _active(b, S_QT0, A0)
    _active(b, S_QT1, A1)
    s(f"s_add_u32 {sr(S_TMP + 11)}, {sr(S_IT)}, 1", S(S_IT), S(S_TMP + 11))
    s(f"s_cmp_lt_u32 {sr(S_TMP + 11)}, {sr(S_ITERS)}", S(S_TMP + 11) + S(S_ITERS), [("scc", 0)])
    s(f"s_cselect_b32 {sr(A1)}, {sr(A1)}, 0", S(A1) + [("scc", 0)], S(A1))
    # masked: causal and qt0*32 == kw0 (the diagonal tile), or a key of the wave is >= kv_len
    s(f"s_lshl_b32 {sr(MK)}, {sr(S_QT0)}, 5", S(S_QT0), S(MK))
    s(f"s_cmp_eq_u32 {sr(MK)}, {sr(S_KW0)}", S(MK) + S(S_KW0), [("scc", 0)])
    s(f"s_cselect_b32 {sr(MK)}, {sr(S_CAUSAL)}, 0", S(S_CAUSAL) + [("scc", 0)], S(MK))
    s(f"s_or_b32 {sr(MK)}, {sr(MK)}, {sr(S_KWMASK)}", S(MK) + S(S_KWMASK), S(MK))
    # variant = 4*act1 + 2*act0 + masked
    s(f"s_lshl_b32 {sr(A1)}, {sr(A1)}, 2", S(A1), S(A1))
    s(f"s_lshl_b32 {sr(A0)}, {sr(A0)}, 1", S(A0), S(A0))
    s(f"s_or_b32 {sr(A1)}, {sr(A1)}, {sr(A0)}", S(A1) + S(A0), S(A1))
    s(f"s_or_b32 {sr(A1)}, {sr(A1)}, {sr(MK)}", S(A1) + S(MK), S(A1))
    variants = [  # (label, sdp, ew, masked, codes)
        ("full", True, True, False, (6,)),
        ("fullm", True, True, True, (7,)),
        ("sdp", True, False, False, (4, 5)),
        ("last", False, True, False, (2,)),
        ("lastm", False, True, True, (3,)),
    ]
    for lab, _, _, _, codes in variants:
        for c in codes:
            s(f"s_cmp_eq_u32 {sr(A1)}, {c}", S(A1), [("scc", 0)])
            p.branch(f"s_cbranch_scc1 .L{lab}{u}", [("scc", 0)])
    # idle (codes 0, 1)
    b.body(u, sdp=False, ew=False, masked=False)
    p.branch(f"s_branch .Le{u}")
    for lab, sdp, ew, masked, _ in variants:
        p.label(f".L{lab}{u}")
        b.body(u, sdp=sdp, ew=ew, masked=masked)
        p.branch(f"s_branch .Le{u}")
    p.label(f".Le{u}")
    _advance_qt(b, S_QT0)
    _advance_qt(b, S_QT1)
    _advance(b, S_H3, S_QT3)
    s(f"s_add_u32 {sr(S_IT)}, {sr(S_IT)}, 1", S(S_IT), S(S_IT))


def main(path: str) -> None:
    with open(path, "w") as f:
        f.write(build())


if __name__ == "__main__":
    import sys
    main(sys.argv[1])

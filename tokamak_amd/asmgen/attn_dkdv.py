"""Generator of the gfx950 assembly FlashAttention backward dK/dV kernel, D = 128, fp16.

Contract: identical to fa_bwd_dkdv_kernel (tokamak_amd/csrc/attn_bwd.hip), the true-gradient
replacement of the reference's k_gqa_flash_attn_tc_bwd dK/dV (src/tkm_gpu.cu:440-598, which
writes copies of dQ/dO at 588-596 instead):
    P_ij = exp(s_ij - LSE_i),  dS_ij = P_ij (<dO_i, v_j> - D_i)
    dK_j = scale sum_i dS_ij q_i,  dV_j = sum_i P_ij dO_i
over every query row i of every q-head of key j's kv group, key j visible from row i iff
j < kv_len[b] and (!causal || j <= i); dK and dV are written (not accumulated) into dqkv.
Instead of LSE and D it reads the workspace's row values -LSE*log2(e) and -D, stored per
(batch, head) in tiles of 32 rows (the 32 values -LSE*log2e, then the 32 values -D; rows
padded to a multiple of 32 with zeros), which the pass that computes D writes.

Work decomposition: persistent, one workgroup (4 waves, one per SIMD) per compute unit walks
items (batch, kv head, block of 128 keys), the key blocks of a head together on one XCD.  A wave owns 32 keys: K and V of those keys
(fp16, as loaded) sit in AGPRs as the B operands of S = Q K^T and
dP = dO V^T, and the accumulators dV^T, dK^T (C[m = head dim][n = key]) in AGPRs.  The
workgroup walks the query tiles (32 rows) of every q-head of the group from the last one down
(causal: to its own key block's first); each tile's Q and dO rows go HBM -> LDS by buffer DMA into one of four buffers
(tile t in buffer t % 4, requested three tiles ahead); each wave also copies the tile's 256
bytes of row values into its own slot.  The DMA descriptors are fixed for the kernel (whole batch, so rows
past S read as zero); a tile's position enters as an offset added to the lane offsets.
Per tile:
    S  = Q K^T                    8 MFMAs, C[m = query][n = key]: lane = key (unscaled
                                  scores, exact products summed in fp32)
    dP = dO V^T  + (-D)           8 MFMAs (-D: the accumulators' start values)
    P = exp2(fma(S, scale*log2e, -LSE*log2e)), dS = P * dP
                                  masked to 0 where the key is hidden; the scale is applied
                                  in fp32, as the reference's kernel does (a scale folded into
                                  K and rounded to fp16 moves a score s by up to |s|*2^-12)
    (the row values -LSE*log2e and -D: four consecutive rows per register group, read by each
     half-wave as one 16-byte broadcast LDS read)
    dV^T += dO^T P, dK^T += Q^T dS 16 MFMAs, P and dS packed to fp16 in place as B operands,
                                  dO^T and Q^T read transposed (ds_read_b64_tr_b16)
Each loop body runs 32 MFMA slots: S/dP of the next tile with the elementwise work of this
tile between them, one workgroup barrier, then dV/dK of this tile with the next tile's
-LSE*log2e, the next-but-one tile's -D and the request of the tile three ahead in between.  The scalar
bookkeeping (descriptors of the requested tile, the next body's variant) is spread between
the MFMAs; a body ends by jumping straight into the next body's common variant.
"""
from __future__ import annotations

import numpy as np

from .common import Lanes, lane_basics, row_read_offsets, swz, tr_read_offsets, xcd_slot
from .gfx950 import A, BRANCH, Prog, S, V, ar, kernel_text, sr, vr

NAME = "tkm_fa_bwd_dkdv_d128_f16"
MFMA = "v_mfma_f32_32x32x16_f16"
MFMA_OF = {"f16": MFMA, "bf16": "v_mfma_f32_32x32x16_bf16"}
PACK_OF = {"f16": "v_cvt_pk_f16_f32", "bf16": "v_cvt_pk_bf16_f32"}
# bf16 (build(dt="bf16"), tkm_fa_bwd_dkdv_d128_bf16): P and dS go to the dV / dK MFMAs as two
# bf16 halves each, hi = bf16(x) and lo = bf16(x - hi) (about 16 significant bits), so each
# transposed read feeds two MFMAs and a body has 48 slots: S/dP in 0..15, dV/dK in 16..47.
ROWB = 256
NBUF = 4
TILE = 32 * ROWB                    # 8 KB: one 32-row tile of Q or dO
BUFB = 2 * TILE                     # Q then dO
LDS_LD = NBUF * BUFB                # row values: per buffer 4 waves x 256 B
LDB = 1024
LDS_EPI = LDS_LD + NBUF * LDB       # per wave: 32 key rows of 272 B staging dK, dV for the store
EPI_ROW = 272                       # 256 B + 16 B pad: rows 16 B apart in the banks
EPI_WAVE = 32 * EPI_ROW
LDS_BYTES = LDS_EPI + 4 * EPI_WAVE
LK = 4                              # slots between a row read and its MFMA
LV = 4                              # slots between a transposed read pair and its MFMA
NRB = 6                             # row-read registers in rotation (x4)
NTB = 6                             # transposed-read registers in rotation (x4)
assert LK <= NRB                    # the first LK row reads of a tile are in flight across bodies
EW_SPLIT = False                    # elementwise pairs 4..7 in the dV/dK half (measured slower)

ARGS = [(0, 8, "ptr"), (8, 8, "ptr"), (16, 8, "ptr"), (24, 8, "ptr"), (32, 8, "ptr")] + \
       [(40 + 4 * i, 4, "val") for i in range(16)]
KERNARG_BYTES = 104

# ---- SGPRs
S_WG = 2                               # workgroup index, then its place in a round (xcd_slot)
S_KA, S_KD = 3, 4                      # round of the current item / of the DMA stream's item
S_QKV, S_DOUT, S_PAIRS, S_DQKV, S_KVLEN = 8, 10, 12, 14, 16
S_SEQ, S_HQ, S_HKV, S_SL2, S_CAUSAL, S_LDB = 18, 19, 20, 21, 22, 23
S_LDO, S_G, S_SCALE, S_NKBLK, S_SP, S_NWG, S_NI, S_BH = 24, 25, 26, 27, 28, 29, 30, 31
S_TQ, S_TO, S_TL = 5, 6, 7             # offsets of the requested tile (Q, dO, row values)
S_LDB32, S_LDO32 = 88, 89              # 32 rows of qkv / dO in bytes
S_MAGNK, S_MAGHKV = 90, 91             # ceil(2^32 / n_kblk), ceil(2^32 / Hkv) (0 for 1)
S_BA, S_KVHA, S_ITERSD, S_QTBD = 92, 93, 94, 95   # current item's batch, kv head; DMA item's tiles
S_WAVE, S_KVL, S_KB0, S_KW0, S_QTB, S_QTL, S_ITERS, S_IT = 32, 33, 34, 35, 36, 37, 38, 39
S_BQKV, S_BDO, S_BLD = 40, 42, 44      # 64-bit bases of the DMA stream's item
S_CODE, S_KWACT = 46, 47               # variant of the current body; wave has a key < kv_len
S_RQ, S_RO, S_RL = 48, 52, 56          # DMA descriptors of the DMA stream's item
S_QT0, S_QT1, S_QT3, S_H3 = 60, 61, 62, 63
S_LDSW, S_LDSL, S_KWMASK = 64, 65, 66  # DMA offsets; 1 if a key of the wave is >= kv_len
S_ITD = 67                             # tiles of the DMA stream's item already requested
S_KWEFF, S_KWDIAG = 68, 69             # causal ? kw0 : 0;  causal ? kw0 : -1
S_TMP = 70                             # s70..s87
NEXT_FREE_SGPR = 96

# ---- VGPRs
V_SD = (0, 32)          # set J: S at +0..15, dP at +16..31
V_P, V_DS = 64, 72      # packed P[ks][w], dS[ks][w]
V_CS, V_CD = 80, 96     # accumulator start values: -LSE*log2e, -D (per register row)
V_RB = 112              # row-read buffers
V_TB = V_RB + 4 * NRB   # transposed-read buffers
V_KOFF = V_TB + 4 * NTB
V_VOFF = V_KOFF + 8
V_DOFF = V_VOFF + 8     # Q rows (2), dO rows (2)
V_LOFF = V_DOFF + 4     # lane*4 (row-quad DMA)
V_LDR = V_LOFF + 1      # row-value read address: the wave's slot + 16*hi (see the lane check)
V_DA = V_LDR + 1        # (5) DMA addresses of the requested tile
V_L32 = V_DA + 5
V_HI4 = V_L32 + 1
V_TK = V_HI4 + 1        # mask threshold of the current tile
V_T = V_TK + 1          # temporaries
V_PT = V_T + 8          # prologue lane scratch (13 registers)
assert V_PT + 13 <= 256
V_PL, V_DSL = 212, 220  # bf16: lo halves of P[ks][w], dS[ks][w]
V_SPL = 228             # bf16: split temporaries (4)
assert V_PT + 13 <= V_PL and V_SPL + 4 <= 256

# ---- AGPRs
A_DV, A_DK, A_K, A_V = 0, 64, 128, 160
A_NK, A_NV = 192, 224     # the next item's K and V rows as loaded
ACC = set(A(A_DV, 128))

# variants of a body: (label, S/dP of the next tile, elementwise + dV/dK of this tile, masked)
VARIANTS = [("full", True, True, False), ("fullm", True, True, True), ("sdp", True, False, False),
            ("last", False, True, False), ("lastm", False, True, True), ("idle", False, False, False)]
# code = 8 (done) or 4*act(next tile) + 2*act(this tile) + masked(this tile)
CODES = {"full": (6,), "fullm": (7,), "sdp": (4, 5), "last": (2,), "lastm": (3,), "idle": (0, 1)}

_SCC_W = ("s_add_", "s_sub_", "s_addc", "s_subb", "s_and_", "s_or_", "s_xor_", "s_lshl", "s_lshr",
          "s_ashr", "s_min_", "s_max_", "s_cmp", "s_bfe", "s_not", "s_andn2", "s_orn2", "s_nand",
          "s_nor", "s_xnor", "s_abs", "s_bcnt")
_SCC_R = ("s_cselect", "s_addc", "s_subb", "s_cbranch_scc", "s_cmov")


def _scc(ins):
    op = ins.text.split()[0] if ins.text else ""
    return op.startswith(_SCC_R), op.startswith(_SCC_W)


def split_scalar(ins, n):
    """Split a scalar instruction list into n consecutive chunks, cutting only where SCC is dead
    (so other instructions, including SCC-writing M0 updates, can go between chunks)."""
    safe = [True] * (len(ins) + 1)
    nxt = "dead"
    for k in range(len(ins) - 1, -1, -1):
        r, w = _scc(ins[k])
        if r:
            nxt = "live"
        elif w:
            nxt = "dead"
        safe[k] = nxt == "dead"
    cuts = [0]
    for c in range(1, n):
        want = round(c * len(ins) / n)
        k = max(want, cuts[-1])
        while k < len(ins) and not safe[k]:
            k += 1
        cuts.append(k)
    cuts.append(len(ins))
    return [ins[cuts[i]:cuts[i + 1]] for i in range(n)]


def mask_c(r):
    """Query-row offset (within the tile, lane half aside) of accumulator register r."""
    return (r // 4) * 8 + (r % 4)


class Body:
    def __init__(self, p: Prog, dt: str = "f16"):
        self.p = p
        self.dt = dt
        self.mfma_op = MFMA_OF[dt]
        self.pack_op = PACK_OF[dt]
        self.split = dt == "bf16"

    def s(self, text, reads=(), writes=()):
        self.p.salu(text, reads, writes)

    def capture(self, fn, *args):
        """Instructions fn emits, without emitting them."""
        saved = self.p
        self.p = Prog()
        try:
            fn(*args)
            return self.p.ins
        finally:
            self.p = saved

    # ---------------------------------------------------------------- descriptors
    def nrec_rows(self, dst, rows, stride, width_sgpr=None):
        """dst = bytes of a descriptor over `rows` rows of `stride` bytes whose lanes touch
        the first `width` bytes of each row (256, or the SGPR width_sgpr): (rows-1)*stride +
        width, 0 without rows.  It ends at the last row's last touched byte, so no request
        reaches past the tensor's end."""
        s = self.s
        s(f"s_mul_i32 {sr(dst)}, {sr(rows)}, {sr(stride)}", S(rows) + S(stride), S(dst))
        s(f"s_sub_u32 {sr(dst)}, {sr(dst)}, {sr(stride)}", S(dst) + S(stride), S(dst))
        if width_sgpr is None:
            s(f"s_add_u32 {sr(dst)}, {sr(dst)}, 0x100", S(dst), S(dst))
        else:
            s(f"s_add_u32 {sr(dst)}, {sr(dst)}, {sr(width_sgpr)}", S(dst) + S(width_sgpr), S(dst))
        s(f"s_max_i32 {sr(dst)}, {sr(dst)}, 0", S(dst), S(dst))

    def tile_offsets(self, h_sgpr, qt_sgpr):
        """Byte offsets of tile (head offset h, q-tile qt) from the fixed descriptors:
        TQ = qt*32*ldb + h*256, TO = qt*32*ldo + h*256, TL = (h*SP + qt*32)*8."""
        s = self.s
        T0, T1 = S_TMP, S_TMP + 1
        s(f"s_lshl_b32 {sr(T0)}, {sr(h_sgpr)}, 8", S(h_sgpr), S(T0))
        s(f"s_mul_i32 {sr(S_TQ)}, {sr(qt_sgpr)}, {sr(S_LDB32)}", S(qt_sgpr) + S(S_LDB32), S(S_TQ))
        s(f"s_add_u32 {sr(S_TQ)}, {sr(S_TQ)}, {sr(T0)}", S(S_TQ) + S(T0), S(S_TQ))
        s(f"s_mul_i32 {sr(S_TO)}, {sr(qt_sgpr)}, {sr(S_LDO32)}", S(qt_sgpr) + S(S_LDO32), S(S_TO))
        s(f"s_add_u32 {sr(S_TO)}, {sr(S_TO)}, {sr(T0)}", S(S_TO) + S(T0), S(S_TO))
        s(f"s_mul_i32 {sr(S_TL)}, {sr(h_sgpr)}, {sr(S_SP)}", S(h_sgpr) + S(S_SP), S(S_TL))
        s(f"s_lshl_b32 {sr(T1)}, {sr(qt_sgpr)}, 5", S(qt_sgpr), S(T1))
        s(f"s_add_u32 {sr(S_TL)}, {sr(S_TL)}, {sr(T1)}", S(S_TL) + S(T1), S(S_TL))
        s(f"s_lshl_b32 {sr(S_TL)}, {sr(S_TL)}, 3", S(S_TL), S(S_TL))

    # ---------------------------------------------------------------- DMA
    def dma_m0(self, which, jb, i=0):
        """M0 (LDS target) of one DMA instruction and its lane addresses in V_DA."""
        s, p = self.s, self.p
        k = {"q": i, "o": 2 + i, "l": 4}[which]
        if which == "q":
            s(f"s_add_u32 m0, {sr(S_LDSW)}, {jb * BUFB + i * 1024}", S(S_LDSW), [("m0", 0)])
            p.valu(f"v_add_u32_e32 {vr(V_DA + k)}, {sr(S_TQ)}, {vr(V_DOFF + i)}", S(S_TQ) + V(V_DOFF + i), V(V_DA + k))
        elif which == "o":
            s(f"s_add_u32 m0, {sr(S_LDSW)}, {jb * BUFB + TILE + i * 1024}", S(S_LDSW), [("m0", 0)])
            p.valu(f"v_add_u32_e32 {vr(V_DA + k)}, {sr(S_TO)}, {vr(V_DOFF + 2 + i)}", S(S_TO) + V(V_DOFF + 2 + i), V(V_DA + k))
        else:
            s(f"s_add_u32 m0, {sr(S_LDSL)}, {jb * LDB}", S(S_LDSL), [("m0", 0)])
            p.valu(f"v_add_u32_e32 {vr(V_DA + k)}, {sr(S_TL)}, {vr(V_LOFF)}", S(S_TL) + V(V_LOFF), V(V_DA + k))

    def dma_ld(self, which, i=0):
        k = {"q": i, "o": 2 + i, "l": 4}[which]
        rs = {"q": S_RQ, "o": S_RO, "l": S_RL}[which]
        op = "buffer_load_dword" if which == "l" else "buffer_load_dwordx4"
        self.p.dma(f"{op} {vr(V_DA + k)}, {sr(rs, 4)}, 0 offen lds", V(V_DA + k) + S(rs, 4))

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

    def prefetch_regs(self):
        return [V(V_RB + (i % NRB) * 4, 4) for i in range(LK)]

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

    def cinit_read(self, jb, k):
        """Row values of accumulator registers 4g .. 4g+3 (g = k % 4): k < 4, -LSE*log2e (the
        exps' offset of S); k >= 4, -D (dP's start values): query rows 8g + 4hi .. +3 of the
        tile in buffer jb, the same for every lane of a half-wave (one 16-byte broadcast read
        per half)."""
        g, which = k % 4, k // 4
        base = (V_CS if which == 0 else V_CD) + 4 * g
        self.p.ds_read(f"ds_read_b128 {vr(base, 4)}, {vr(V_LDR)} offset:{jb * LDB + 128 * which + 32 * g}",
                       V(base, 4), V(V_LDR))

    def cinit(self, jb, ks=range(8)):
        for k in ks:
            self.cinit_read(jb, k)

    # ---------------------------------------------------------------- MFMAs
    def sdp_mfma(self, i, J):
        """S (unscaled scores, from 0) or dP (from -D), k-step i // 2."""
        ks, which = i // 2, i % 2
        dst = V_SD[J] + 16 * which
        c = (None if which == 0 else V_CD) if ks == 0 else dst
        b = (A_K if which == 0 else A_V) + ks * 4
        self.p.mfma(self.mfma_op, dst, V_RB + (i % NRB) * 4, b, c, b_acc=True)

    def dvdk_mfma(self, j, lo=False):
        """dV or dK MFMA j (the operand of transposed read j); lo: the bf16 residual half."""
        ks, k8 = j // 8, j % 8
        db = k8 % 4
        if k8 < 4:
            acc, b = A_DV + db * 16, (V_PL if lo else V_P) + ks * 4
        else:
            acc, b = A_DK + db * 16, (V_DSL if lo else V_DS) + ks * 4
        self.p.mfma(self.mfma_op, acc, V_TB + (j % NTB) * 4, b, acc, dst_acc=True)

    def dvdk_slots(self):
        """(transposed read j, lo) of each dV/dK slot: j in order for fp16; bf16: for each
        pair of reads (2a, 2a+1), hi 2a, hi 2a+1, lo 2a, lo 2a+1 (one MFMA between the two
        into one accumulator)."""
        if not self.split:
            return [(j, False) for j in range(16)]
        return [(4 * (k // 4) // 2 + k % 2, (k // 2) % 2 == 1) for k in range(32)]

    def tr_first_use(self):
        """Slot offset (from the first dV/dK slot) of each transposed read's first MFMA."""
        first = {}
        for k, (j, _) in enumerate(self.dvdk_slots()):
            first.setdefault(j, k)
        return [first[j] for j in range(16)]

    # ---------------------------------------------------------------- elementwise (set J)
    def ew_exp(self, J, n):
        """P = exp2(fma(S, scale*log2e, -LSE*log2e)) of registers 2n, 2n+1 of set J: the scale
        applied in fp32 to the exact scores (the row values of the same tile are in V_CS)."""
        for r in (2 * n, 2 * n + 1):
            x = V_SD[J] + r
            self.p.valu(f"v_fma_f32 {vr(x)}, {vr(x)}, {sr(S_SL2)}, {vr(V_CS + r)}", V(x) + S(S_SL2) + V(V_CS + r),
                        V(x))
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
        for src, hi, lo, t in ((x, V_P, V_PL, V_SPL), (dp, V_DS, V_DSL, V_SPL + 2)):
            hw = hi + ks * 4 + w
            p.valu(f"{self.pack_op} {vr(hw)}, {vr(src)}, {vr(src + 1)}", V(src, 2), V(hw))
            if self.split:
                # lo = bf16(x - hi): hi's halves as fp32 are its word shifted up / masked
                p.valu(f"v_lshlrev_b32_e32 {vr(t)}, 16, {vr(hw)}", V(hw), V(t))
                p.valu(f"v_and_b32_e32 {vr(t + 1)}, 0xffff0000, {vr(hw)}", V(hw), V(t + 1))
                p.valu(f"v_sub_f32_e32 {vr(src)}, {vr(src)}, {vr(t)}", V(src) + V(t), V(src))
                p.valu(f"v_sub_f32_e32 {vr(src + 1)}, {vr(src + 1)}, {vr(t + 1)}", V(src + 1) + V(t + 1), V(src + 1))
                lw = lo + ks * 4 + w
                p.valu(f"v_cvt_pk_bf16_f32 {vr(lw)}, {vr(src)}, {vr(src + 1)}", V(src, 2), V(lw))

    def mask_threshold(self, qt_sgpr):
        """tk = key >= kv_len ? 32 : (causal ? kw0 - qr0 + l32 - 4hi : -96); an element of
        register r is hidden iff mask_c(r) < tk."""
        s, p = self.s, self.p
        T0, T1 = S_TMP + 12, S_TMP + 13
        s(f"s_lshl_b32 {sr(T0)}, {sr(qt_sgpr)}, 5", S(qt_sgpr), S(T0))
        s(f"s_sub_u32 {sr(T0)}, {sr(S_KW0)}, {sr(T0)}", S(S_KW0) + S(T0), S(T0))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T0)}, 0xffffffa0, {sr(T0)}", S(T0) + [("scc", 0)], S(T0))
        p.valu(f"v_add_u32_e32 {vr(V_TK)}, {sr(T0)}, {vr(V_L32)}", S(T0) + V(V_L32), V(V_TK))
        p.valu(f"v_sub_u32_e32 {vr(V_TK)}, {vr(V_TK)}, {vr(V_HI4)}", V(V_TK) + V(V_HI4), V(V_TK))
        s(f"s_sub_u32 {sr(T1)}, {sr(S_KVL)}, {sr(S_KW0)}", S(S_KVL) + S(S_KW0), S(T1))
        p.valu(f"v_cmp_le_i32_e32 vcc, {sr(T1)}, {vr(V_L32)}", S(T1) + V(V_L32), [("vcc", 0)])
        p.valu(f"v_cndmask_b32_e64 {vr(V_TK)}, {vr(V_TK)}, 32, vcc", V(V_TK) + [("vcc", 0)], V(V_TK))

    # ---------------------------------------------------------------- scalar bookkeeping
    def active(self, qt, dst):
        """dst = KWACT if q-tile qt holds a row that sees a key of this wave (causal: qt*32 >= kw0)."""
        T = S_TMP + 14
        self.s(f"s_lshl_b32 {sr(T)}, {sr(qt)}, 5", S(qt), S(T))
        self.s(f"s_cmp_ge_u32 {sr(T)}, {sr(S_KWEFF)}", S(T) + S(S_KWEFF), [("scc", 0)])
        self.s(f"s_cselect_b32 {sr(dst)}, {sr(S_KWACT)}, 0", S(S_KWACT) + [("scc", 0)], S(dst))

    # Query tiles are walked from the last (S_QTL) down to the item's first visible one, so
    # that the items of one (batch, kv head) that run at the same time on one XCD (key blocks
    # z, z+1, ... of a round) read the same Q / dO tiles together and share them in its L2;
    # walked upwards, they start at their own diagonals and read each tile at different times.
    def advance_qt(self, qt):
        s = self.s
        s(f"s_sub_u32 {sr(qt)}, {sr(qt)}, 1", S(qt), S(qt))
        s(f"s_cmp_lt_i32 {sr(qt)}, {sr(S_QTB)}", S(qt) + S(S_QTB), [("scc", 0)])
        s(f"s_cselect_b32 {sr(qt)}, {sr(S_QTL)}, {sr(qt)}", S(S_QTL) + S(qt) + [("scc", 0)], S(qt))

    def advance_h(self, h, qt, qtb=S_QTBD):
        """(h, qt) := (h, qt - 1), or (h + 1, last tile) below the first visible query tile."""
        s = self.s
        s(f"s_sub_u32 {sr(qt)}, {sr(qt)}, 1", S(qt), S(qt))
        s(f"s_cmp_lt_i32 {sr(qt)}, {sr(qtb)}", S(qt) + S(qtb), [("scc", 0)])
        s(f"s_cselect_b32 {sr(qt)}, {sr(S_QTL)}, {sr(qt)}", S(S_QTL) + S(qt) + [("scc", 0)], S(qt))
        s(f"s_addc_u32 {sr(h)}, {sr(h)}, 0", S(h) + [("scc", 0)], S(h))

    def code(self):
        """S_CODE for body S_IT with tiles S_QT0 (this) and S_QT1 (next)."""
        s = self.s
        A0, A1, T = S_TMP + 15, S_TMP + 16, S_TMP + 17
        self.active(S_QT0, A0)
        self.active(S_QT1, A1)
        s(f"s_add_u32 {sr(T)}, {sr(S_IT)}, 1", S(S_IT), S(T))
        s(f"s_cmp_lt_u32 {sr(T)}, {sr(S_ITERS)}", S(T) + S(S_ITERS), [("scc", 0)])
        s(f"s_cselect_b32 {sr(A1)}, {sr(A1)}, 0", S(A1) + [("scc", 0)], S(A1))
        s(f"s_lshl_b32 {sr(T)}, {sr(S_QT0)}, 5", S(S_QT0), S(T))
        s(f"s_cmp_eq_u32 {sr(T)}, {sr(S_KWDIAG)}", S(T) + S(S_KWDIAG), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T)}, 1, {sr(S_KWMASK)}", S(S_KWMASK) + [("scc", 0)], S(T))
        s(f"s_lshl2_add_u32 {sr(A1)}, {sr(A1)}, {sr(T)}", S(A1) + S(T), S(A1))
        s(f"s_lshl1_add_u32 {sr(S_CODE)}, {sr(A0)}, {sr(A1)}", S(A0) + S(A1), S(S_CODE))
        s(f"s_cmp_ge_u32 {sr(S_IT)}, {sr(S_ITERS)}", S(S_IT) + S(S_ITERS), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_CODE)}, 8, {sr(S_CODE)}", S(S_CODE) + [("scc", 0)], S(S_CODE))

    def advance_and_code(self):
        """Next body's tiles: this item's next query tile, the DMA stream's next tile (bit 16 of
        the code when that starts a new item); the next body's variant."""
        s = self.s
        s(f"s_mov_b32 {sr(S_QT0)}, {sr(S_QT1)}", S(S_QT1), S(S_QT0))
        self.advance_qt(S_QT1)
        self.advance_h(S_H3, S_QT3)
        s(f"s_add_u32 {sr(S_ITD)}, {sr(S_ITD)}, 1", S(S_ITD), S(S_ITD))
        s(f"s_add_u32 {sr(S_IT)}, {sr(S_IT)}, 1", S(S_IT), S(S_IT))
        self.code()
        T = S_TMP + 17
        s(f"s_cmp_ge_u32 {sr(S_ITD)}, {sr(S_ITERSD)}", S(S_ITD) + S(S_ITERSD), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T)}, 16, 0", [("scc", 0)], S(T))
        s(f"s_or_b32 {sr(S_CODE)}, {sr(S_CODE)}, {sr(T)}", S(S_CODE) + S(T), S(S_CODE))

    # ---------------------------------------------------------------- items
    # A workgroup walks items i = (b*Hkv + kvh)*n_kblk + z (z = key block, fastest) in rounds
    # of NWG: round k takes item k*NWG + v, or k*NWG + NWG-1-v for odd k, v the workgroup's
    # place (xcd_slot: consecutive places share an XCD).  The key blocks of a head then run
    # together on one XCD and share its L2 for the head's Q / dO rows, and for causal the
    # long and short blocks of consecutive rounds pair up (z with n_kblk-1-z).  An item has
    # g*(QTE - QTB) query tiles, or one tile that no wave uses when its keys all lie past
    # kv_len.  Two roles follow the item sequence: the current item (tile it: its keys, masks,
    # accumulators) and the DMA stream (tile it+3), which runs ahead across item boundaries.
    def item_index(self, k_sgpr, dst):
        s, T = self.s, S_TMP + 12
        s(f"s_mul_i32 {sr(dst)}, {sr(k_sgpr)}, {sr(S_NWG)}", S(k_sgpr) + S(S_NWG), S(dst))
        s(f"s_sub_u32 {sr(T)}, {sr(S_NWG)}, 1", S(S_NWG), S(T))
        s(f"s_sub_u32 {sr(T)}, {sr(T)}, {sr(S_WG)}", S(T) + S(S_WG), S(T))
        s(f"s_bitcmp1_b32 {sr(k_sgpr)}, 0", S(k_sgpr), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T)}, {sr(T)}, {sr(S_WG)}", S(T) + S(S_WG) + [("scc", 0)], S(T))
        s(f"s_add_u32 {sr(dst)}, {sr(dst)}, {sr(T)}", S(dst) + S(T), S(dst))

    def decode(self, i, z, b, kvh):
        """R = i / n_kblk, z = i % n_kblk, b = R / Hkv, kvh = R % Hkv (multiply-high by the
        host's reciprocals, checked exact on the host for every index that occurs)."""
        s, R = self.s, S_TMP + 13
        s(f"s_mul_hi_u32 {sr(R)}, {sr(i)}, {sr(S_MAGNK)}", S(i) + S(S_MAGNK), S(R))
        s(f"s_cmp_eq_u32 {sr(S_NKBLK)}, 1", S(S_NKBLK), [("scc", 0)])
        s(f"s_cselect_b32 {sr(R)}, {sr(i)}, {sr(R)}", S(i) + S(R) + [("scc", 0)], S(R))
        s(f"s_mul_i32 {sr(z)}, {sr(R)}, {sr(S_NKBLK)}", S(R) + S(S_NKBLK), S(z))
        s(f"s_sub_u32 {sr(z)}, {sr(i)}, {sr(z)}", S(i) + S(z), S(z))
        s(f"s_mul_hi_u32 {sr(b)}, {sr(R)}, {sr(S_MAGHKV)}", S(R) + S(S_MAGHKV), S(b))
        s(f"s_cmp_eq_u32 {sr(S_HKV)}, 1", S(S_HKV), [("scc", 0)])
        s(f"s_cselect_b32 {sr(b)}, {sr(R)}, {sr(b)}", S(R) + S(b) + [("scc", 0)], S(b))
        s(f"s_mul_i32 {sr(kvh)}, {sr(b)}, {sr(S_HKV)}", S(b) + S(S_HKV), S(kvh))
        s(f"s_sub_u32 {sr(kvh)}, {sr(R)}, {sr(kvh)}", S(R) + S(kvh), S(kvh))

    def kvl_of(self, b, dst, label):
        """dst = clamp(kv_len[b], 0, S), or S without kv_len.  No LDS read may be in flight."""
        p, s, T = self.p, self.s, S_TMP + 12
        s(f"s_mov_b32 {sr(dst)}, {sr(S_SEQ)}", S(S_SEQ), S(dst))
        s(f"s_cmp_eq_u64 {sr(S_KVLEN, 2)}, 0", S(S_KVLEN, 2), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 {label}", [("scc", 0)], skip_xdl=ACC)
        s(f"s_lshl_b32 {sr(T)}, {sr(b)}, 2", S(b), S(T))
        p.smem(f"s_load_dword {sr(dst)}, {sr(S_KVLEN, 2)}, {sr(T)}", S(dst), S(S_KVLEN, 2) + S(T))
        p.waitcnt(lgkm=0)
        s(f"s_max_i32 {sr(dst)}, {sr(dst)}, 0", S(dst), S(dst))
        s(f"s_min_i32 {sr(dst)}, {sr(dst)}, {sr(S_SEQ)}", S(dst) + S(S_SEQ), S(dst))
        p.label(label)

    def tiles_of(self, kb0, kvl, qtb, iters):
        """qtb = causal ? kb0/32 : 0; iters = kb0 >= kvl ? 1 : g*(QTL + 1 - qtb)."""
        s = self.s
        s(f"s_lshr_b32 {sr(qtb)}, {sr(kb0)}, 5", S(kb0), S(qtb))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(qtb)}, 0, {sr(qtb)}", S(qtb) + [("scc", 0)], S(qtb))
        s(f"s_sub_u32 {sr(iters)}, {sr(S_QTL)}, {sr(qtb)}", S(S_QTL) + S(qtb), S(iters))
        s(f"s_add_u32 {sr(iters)}, {sr(iters)}, 1", S(iters), S(iters))
        s(f"s_mul_i32 {sr(iters)}, {sr(iters)}, {sr(S_G)}", S(iters) + S(S_G), S(iters))
        s(f"s_cmp_ge_u32 {sr(kb0)}, {sr(kvl)}", S(kb0) + S(kvl), [("scc", 0)])
        s(f"s_cselect_b32 {sr(iters)}, 1, {sr(iters)}", S(iters) + [("scc", 0)], S(iters))

    def decode_d(self, sfx):
        """DMA stream: item of round S_KD -> bases, descriptors, QTBD, ITERSD; tile (0, QTL).
        Past the last item the stream re-reads its last item's tile (0, QTL) at every request
        (in bounds, never used): one tile per decode, so that the next request decodes again
        instead of advancing.  Advancing, it would walk on past the group's last head (one head
        per request where a head has one visible query tile) and, for the last batch and kv
        head, read past the end of dO."""
        p, s = self.p, self.s
        I, Z, B, KVH, KVL, KB0 = (S_TMP + k for k in range(6))
        T0, T1, T2 = S_TMP + 6, S_TMP + 7, S_TMP + 8
        self.item_index(S_KD, I)
        s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
        p.branch(f"s_cbranch_scc0 .Ldd_{sfx}", [("scc", 0)], skip_xdl=ACC)
        s(f"s_mov_b32 {sr(S_ITERSD)}, 1", [], S(S_ITERSD))
        s(f"s_mov_b32 {sr(S_ITD)}, 0", [], S(S_ITD))
        s(f"s_mov_b32 {sr(S_H3)}, 0", [], S(S_H3))
        s(f"s_mov_b32 {sr(S_QT3)}, {sr(S_QTL)}", S(S_QTL), S(S_QT3))
        p.branch(f"s_branch .Lde_{sfx}", skip_xdl=ACC)
        p.label(f".Ldd_{sfx}")
        self.decode(I, Z, B, KVH)
        self.kvl_of(B, KVL, f".Ldk_{sfx}")
        s(f"s_lshl_b32 {sr(KB0)}, {sr(Z)}, 7", S(Z), S(KB0))
        self.tiles_of(KB0, KVL, S_QTBD, S_ITERSD)
        s(f"s_mov_b32 {sr(S_ITD)}, 0", [], S(S_ITD))
        s(f"s_mov_b32 {sr(S_H3)}, 0", [], S(S_H3))
        s(f"s_mov_b32 {sr(S_QT3)}, {sr(S_QTL)}", S(S_QTL), S(S_QT3))
        # bases: qkv + b*S*ldb + kvh*g*256; dout + b*S*ldo + kvh*g*256; pairs + (b*Hq + kvh*g)*SP*8
        s(f"s_mul_i32 {sr(T0)}, {sr(B)}, {sr(S_SEQ)}", S(B) + S(S_SEQ), S(T0))
        s(f"s_mul_i32 {sr(T1)}, {sr(KVH)}, {sr(S_G)}", S(KVH) + S(S_G), S(T1))
        s(f"s_lshl_b32 {sr(T2)}, {sr(T1)}, 8", S(T1), S(T2))
        for base, src, stride in ((S_BQKV, S_QKV, S_LDB), (S_BDO, S_DOUT, S_LDO)):
            self.add64(base, src, T0, stride, T2)
        s(f"s_mul_i32 {sr(T0)}, {sr(B)}, {sr(S_HQ)}", S(B) + S(S_HQ), S(T0))
        s(f"s_add_u32 {sr(T0)}, {sr(T0)}, {sr(T1)}", S(T0) + S(T1), S(T0))
        s(f"s_mul_i32 {sr(T0)}, {sr(T0)}, {sr(S_SP)}", S(T0) + S(S_SP), S(T0))
        s(f"s_mov_b32 {sr(T1)}, 8", [], S(T1))
        self.add64(S_BLD, S_PAIRS, T0, T1, None)
        for dst, base in ((S_RQ, S_BQKV), (S_RO, S_BDO), (S_RL, S_BLD)):
            s(f"s_mov_b32 {sr(dst)}, {sr(base)}", S(base), S(dst))
            s(f"s_and_b32 {sr(dst + 1)}, {sr(base + 1)}, 0xffff", S(base + 1), S(dst + 1))
        p.label(f".Lde_{sfx}")

    def add64(self, dst, src, rows, stride, extra):
        """s[dst:dst+1] = s[src:src+1] + rows*stride (+ extra)."""
        s, lo, hi = self.s, S_TMP + 14, S_TMP + 15
        s(f"s_mul_i32 {sr(lo)}, {sr(rows)}, {sr(stride)}", S(rows) + S(stride), S(lo))
        s(f"s_mul_hi_u32 {sr(hi)}, {sr(rows)}, {sr(stride)}", S(rows) + S(stride), S(hi))
        if extra is not None:
            s(f"s_add_u32 {sr(lo)}, {sr(lo)}, {sr(extra)}", S(lo) + S(extra), S(lo) + [("scc", 0)])
            s(f"s_addc_u32 {sr(hi)}, {sr(hi)}, 0", S(hi) + [("scc", 0)], S(hi))
        s(f"s_add_u32 {sr(dst)}, {sr(src)}, {sr(lo)}", S(src) + S(lo), S(dst) + [("scc", 0)])
        s(f"s_addc_u32 {sr(dst + 1)}, {sr(src + 1)}, {sr(hi)}", S(src + 1) + S(hi) + [("scc", 0)], S(dst + 1))

    def d_advance(self, sfx):
        """DMA stream to its next tile (outside the loop bodies)."""
        p, s = self.p, self.s
        self.advance_h(S_H3, S_QT3)
        s(f"s_add_u32 {sr(S_ITD)}, {sr(S_ITD)}, 1", S(S_ITD), S(S_ITD))
        s(f"s_cmp_lt_u32 {sr(S_ITD)}, {sr(S_ITERSD)}", S(S_ITD) + S(S_ITERSD), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lda_{sfx}", [("scc", 0)], skip_xdl=ACC)
        s(f"s_add_u32 {sr(S_KD)}, {sr(S_KD)}, 1", S(S_KD), S(S_KD))
        self.decode_d(sfx)
        p.label(f".Lda_{sfx}")

    def decode_a(self, i, sfx):
        """Current item i: its keys, masks and tiles; tile it = its first tile."""
        s = self.s
        Z = S_TMP
        self.decode(i, Z, S_BA, S_KVHA)
        self.kvl_of(S_BA, S_KVL, f".Lak_{sfx}")
        s(f"s_lshl_b32 {sr(S_KB0)}, {sr(Z)}, 7", S(Z), S(S_KB0))
        T0 = S_TMP + 1
        s(f"s_lshl_b32 {sr(T0)}, {sr(S_WAVE)}, 5", S(S_WAVE), S(T0))
        s(f"s_add_u32 {sr(S_KW0)}, {sr(S_KB0)}, {sr(T0)}", S(S_KB0) + S(T0), S(S_KW0))
        s(f"s_cmp_lt_u32 {sr(S_KW0)}, {sr(S_KVL)}", S(S_KW0) + S(S_KVL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_KWACT)}, 1, 0", [("scc", 0)], S(S_KWACT))
        s(f"s_add_u32 {sr(T0)}, {sr(S_KW0)}, 32", S(S_KW0), S(T0))
        s(f"s_cmp_gt_u32 {sr(T0)}, {sr(S_KVL)}", S(T0) + S(S_KVL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_KWMASK)}, 1, 0", [("scc", 0)], S(S_KWMASK))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_KWEFF)}, 0, {sr(S_KW0)}", S(S_KW0) + [("scc", 0)], S(S_KWEFF))
        s(f"s_cselect_b32 {sr(S_KWDIAG)}, -1, {sr(S_KW0)}", S(S_KW0) + [("scc", 0)], S(S_KWDIAG))
        self.tiles_of(S_KB0, S_KVL, S_QTB, S_ITERS)
        s(f"s_mov_b32 {sr(S_IT)}, 0", [], S(S_IT))
        s(f"s_mov_b32 {sr(S_QT0)}, {sr(S_QTL)}", S(S_QTL), S(S_QT0))
        s(f"s_mov_b32 {sr(S_QT1)}, {sr(S_QTL)}", S(S_QTL), S(S_QT1))
        self.advance_qt(S_QT1)

    def kv_load(self):
        """K (into VGPRs 0..31) and V (into its AGPRs) of the current item's
        wave keys: lane (l32, hi) loads key kw0 + l32, bytes hi*16 + 32ks .. +15."""
        p, s = self.p, self.s
        RK, RV = S_TMP + 6, S_TMP + 10   # 4-aligned
        ROWS, COL, T0 = S_TMP, S_TMP + 1, S_TMP + 2
        s(f"s_sub_u32 {sr(ROWS)}, {sr(S_KVL)}, {sr(S_KW0)}", S(S_KVL) + S(S_KW0), S(ROWS))
        s(f"s_max_i32 {sr(ROWS)}, {sr(ROWS)}, 0", S(ROWS), S(ROWS))
        s(f"s_min_i32 {sr(ROWS)}, {sr(ROWS)}, 32", S(ROWS), S(ROWS))
        s(f"s_mul_i32 {sr(T0)}, {sr(S_BA)}, {sr(S_SEQ)}", S(S_BA) + S(S_SEQ), S(T0))
        s(f"s_add_u32 {sr(T0)}, {sr(T0)}, {sr(S_KW0)}", S(T0) + S(S_KW0), S(T0))      # first key row
        s(f"s_add_u32 {sr(COL)}, {sr(S_HQ)}, {sr(S_KVHA)}", S(S_HQ) + S(S_KVHA), S(COL))
        s(f"s_lshl_b32 {sr(COL)}, {sr(COL)}, 8", S(COL), S(COL))
        for rs, more in ((RK, False), (RV, True)):
            if more:
                s(f"s_lshl_b32 {sr(S_TMP + 3)}, {sr(S_HKV)}, 8", S(S_HKV), S(S_TMP + 3))
                s(f"s_add_u32 {sr(COL)}, {sr(COL)}, {sr(S_TMP + 3)}", S(COL) + S(S_TMP + 3), S(COL))
            self.add64(rs, S_QKV, T0, S_LDB, COL)
            s(f"s_and_b32 {sr(rs + 1)}, {sr(rs + 1)}, 0xffff", S(rs + 1), S(rs + 1))
            self.nrec_rows(rs + 2, ROWS, S_LDB)
            s(f"s_mov_b32 {sr(rs + 3)}, 0x20000", [], S(rs + 3))
        KO = V_T
        p.valu(f"v_mul_lo_u32 {vr(KO)}, {vr(V_L32)}, {sr(S_LDB)}", V(V_L32) + S(S_LDB), V(KO))
        p.valu(f"v_lshl_add_u32 {vr(KO)}, {vr(V_HI4)}, 2, {vr(KO)}", V(V_HI4) + V(KO), V(KO))
        for ks in range(8):
            p.vmem_load(f"buffer_load_dwordx4 {vr(ks * 4, 4)}, {vr(KO)}, {sr(RK, 4)}, 0 offen offset:{ks * 32}",
                        V(ks * 4, 4), V(KO) + S(RK, 4))
        for ks in range(8):
            p.vmem_load(f"buffer_load_dwordx4 {ar(A_V + ks * 4, 4)}, {vr(KO)}, {sr(RV, 4)}, 0 offen offset:{ks * 32}",
                        A(A_V + ks * 4, 4), V(KO) + S(RV, 4))

    def kv_prefetch(self, i, sfx):
        """Loads of item i's K and V rows of this wave's keys (z*128 + 32*wave + l32; rows past
        kv_len read as zero) into the spare AGPRs, untracked: they are issued before the
        current item's epilogue, whose time covers their latency; kv_take waits for them.
        Touches no state of the current item."""
        p, s = self.p, self.s
        Z, B, KVH, KVL, KW0, ROWS = (S_TMP + k for k in range(6))
        RK, RV, T0 = S_TMP + 6, S_TMP + 10, S_TMP + 17
        assert i not in (Z, B, KVH, KVL, KW0, ROWS, T0) and i not in range(RK, RV + 4)
        self.decode(i, Z, B, KVH)
        self.kvl_of(B, KVL, f".Lpk_{sfx}")
        s(f"s_lshl_b32 {sr(KW0)}, {sr(Z)}, 7", S(Z), S(KW0))
        s(f"s_lshl_b32 {sr(T0)}, {sr(S_WAVE)}, 5", S(S_WAVE), S(T0))
        s(f"s_add_u32 {sr(KW0)}, {sr(KW0)}, {sr(T0)}", S(KW0) + S(T0), S(KW0))
        s(f"s_sub_u32 {sr(ROWS)}, {sr(KVL)}, {sr(KW0)}", S(KVL) + S(KW0), S(ROWS))
        s(f"s_max_i32 {sr(ROWS)}, {sr(ROWS)}, 0", S(ROWS), S(ROWS))
        s(f"s_min_i32 {sr(ROWS)}, {sr(ROWS)}, 32", S(ROWS), S(ROWS))
        s(f"s_mul_i32 {sr(T0)}, {sr(B)}, {sr(S_SEQ)}", S(B) + S(S_SEQ), S(T0))
        s(f"s_add_u32 {sr(T0)}, {sr(T0)}, {sr(KW0)}", S(T0) + S(KW0), S(T0))      # first key row
        COL = Z
        s(f"s_add_u32 {sr(COL)}, {sr(S_HQ)}, {sr(KVH)}", S(S_HQ) + S(KVH), S(COL))
        s(f"s_lshl_b32 {sr(COL)}, {sr(COL)}, 8", S(COL), S(COL))
        for rs, more in ((RK, False), (RV, True)):
            if more:
                s(f"s_lshl_b32 {sr(B)}, {sr(S_HKV)}, 8", S(S_HKV), S(B))
                s(f"s_add_u32 {sr(COL)}, {sr(COL)}, {sr(B)}", S(COL) + S(B), S(COL))
            self.add64(rs, S_QKV, T0, S_LDB, COL)
            s(f"s_and_b32 {sr(rs + 1)}, {sr(rs + 1)}, 0xffff", S(rs + 1), S(rs + 1))
            self.nrec_rows(rs + 2, ROWS, S_LDB)
            s(f"s_mov_b32 {sr(rs + 3)}, 0x20000", [], S(rs + 3))
        KO = V_T
        p.valu(f"v_mul_lo_u32 {vr(KO)}, {vr(V_L32)}, {sr(S_LDB)}", V(V_L32) + S(S_LDB), V(KO))
        p.valu(f"v_lshl_add_u32 {vr(KO)}, {vr(V_HI4)}, 2, {vr(KO)}", V(V_HI4) + V(KO), V(KO))
        for base, rs in ((A_NK, RK), (A_NV, RV)):
            for ks in range(8):
                p.vmem_load(f"buffer_load_dwordx4 {ar(base + ks * 4, 4)}, {vr(KO)}, {sr(rs, 4)}, 0 offen offset:{ks * 32}",
                            A(base + ks * 4, 4), V(KO) + S(rs, 4), untracked=True)

    def kv_take(self):
        """The prefetched K and V into place, as loaded."""
        p = self.p
        p.waitcnt(vm=0)
        for i in range(32):
            p.valu(f"v_accvgpr_mov_b32 {ar(A_V + i)}, {ar(A_NV + i)}", A(A_NV + i), A(A_V + i))
        for i in range(32):
            p.valu(f"v_accvgpr_mov_b32 {ar(A_K + i)}, {ar(A_NK + i)}", A(A_NK + i), A(A_K + i))

    def zero_acc(self):
        p = self.p
        for i in range(4):
            p.valu(f"v_mov_b32_e32 {vr(V_TB + i)}, 0", [], V(V_TB + i))
        for i in range(8):   # dV, dK := 0 with eight MFMAs of zero operands
            p.mfma(MFMA, A_DV + 16 * i, V_TB, V_TB, None, dst_acc=True)

    def take_k(self):
        """K as loaded (VGPRs 0..31) into its AGPRs."""
        for i in range(32):
            self.p.valu(f"v_accvgpr_write_b32 {ar(A_K + i)}, {vr(i)}", V(i), A(A_K + i))

    def epilogue(self):
        """dK^T * scale and dV^T of the current item into dqkv.  A lane holds key kw0 + l32,
        d = db*32 + g4*8 + hi*4 + 0..3; the values go to fp16, through the wave's LDS staging
        rows (row = key, 16-byte chunk db*4 + g4), and back out 16 bytes per lane so that every
        store instruction writes four whole 256-byte rows.  Keys past S are dropped by the
        descriptors."""
        p, s = self.p, self.s
        p.comment("epilogue")
        RK, RV = S_TMP + 6, S_TMP + 10   # 4-aligned
        T0, COL, T2, EPW = S_TMP, S_TMP + 1, S_TMP + 2, S_TMP + 3
        s(f"s_mul_i32 {sr(T0)}, {sr(S_BA)}, {sr(S_SEQ)}", S(S_BA) + S(S_SEQ), S(T0))
        s(f"s_add_u32 {sr(COL)}, {sr(S_HQ)}, {sr(S_KVHA)}", S(S_HQ) + S(S_KVHA), S(COL))
        s(f"s_lshl_b32 {sr(COL)}, {sr(COL)}, 8", S(COL), S(COL))
        for rs, more in ((RK, False), (RV, True)):
            if more:
                s(f"s_lshl_b32 {sr(T2)}, {sr(S_HKV)}, 8", S(S_HKV), S(T2))
                s(f"s_add_u32 {sr(COL)}, {sr(COL)}, {sr(T2)}", S(COL) + S(T2), S(COL))
            self.add64(rs, S_DQKV, T0, S_LDB, COL)
            s(f"s_and_b32 {sr(rs + 1)}, {sr(rs + 1)}, 0xffff", S(rs + 1), S(rs + 1))
            self.nrec_rows(rs + 2, S_SEQ, S_LDB)
            s(f"s_mov_b32 {sr(rs + 3)}, 0x20000", [], S(rs + 3))
        s(f"s_mul_i32 {sr(EPW)}, {sr(S_WAVE)}, {EPI_WAVE}", S(S_WAVE), S(EPW))
        s(f"s_add_u32 {sr(EPW)}, {sr(EPW)}, {LDS_EPI}", S(EPW), S(EPW))
        s(f"s_lshl_b32 {sr(T2)}, {sr(S_LDB)}, 2", S(S_LDB), S(T2))              # 4 rows
        BW, BR, TA, TB = 16, 17, 18, 19
        OO = 40
        # write address: EPW + l32*272 + hi*8;  read address: EPW + (lane>>4)*272 + (lane&15)*16
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
        # global offsets of rows kw0 + 4i + (lane >> 4), chunk lane & 15
        p.valu(f"v_add_u32_e32 {vr(TA)}, {sr(S_KW0)}, {vr(TA)}", S(S_KW0) + V(TA), V(TA))
        p.valu(f"v_mul_lo_u32 {vr(TA)}, {vr(TA)}, {sr(S_LDB)}", V(TA) + S(S_LDB), V(TA))
        p.valu(f"v_lshl_add_u32 {vr(OO)}, {vr(TB)}, 4, {vr(TA)}", V(TB) + V(TA), V(OO))
        for i in range(1, 8):
            p.valu(f"v_add_u32_e32 {vr(OO + i)}, {sr(T2)}, {vr(OO + i - 1)}", S(T2) + V(OO + i - 1), V(OO + i))
        W = 0
        for acc, rs, scale in ((A_DK, RK, True), (A_DV, RV, False)):
            for db in range(4):
                for g4 in range(4):
                    a0 = acc + db * 16 + g4 * 4
                    for j in range(4):
                        p.valu(f"v_accvgpr_read_b32 {vr(W + j)}, {ar(a0 + j)}", A(a0 + j), V(W + j))
                    if scale:
                        for j in range(4):
                            p.valu(f"v_mul_f32_e32 {vr(W + j)}, {sr(S_SCALE)}, {vr(W + j)}", V(W + j) + S(S_SCALE), V(W + j))
                    p.valu(f"{self.pack_op} {vr(W + 4)}, {vr(W)}, {vr(W + 1)}", V(W, 2), V(W + 4))
                    p.valu(f"{self.pack_op} {vr(W + 5)}, {vr(W + 2)}, {vr(W + 3)}", V(W + 2, 2), V(W + 5))
                    p.ds_write(f"ds_write_b64 {vr(BW)}, {vr(W + 4, 2)} offset:{(db * 4 + g4) * 16}", V(BW) + V(W + 4, 2))
                    W = 8 if W == 0 else 0
            for i in range(8):   # LDS operations of a wave complete in order: reads see the rows
                R = 20 + 4 * (i % 4)
                p.ds_read(f"ds_read_b128 {vr(R, 4)}, {vr(BR)} offset:{i * 4 * EPI_ROW}", V(R, 4), V(BR))
                p.vmem_store(f"buffer_store_dwordx4 {vr(R, 4)}, {vr(OO + i)}, {sr(rs, 4)}, 0 offen nt",
                             V(R, 4) + V(OO + i) + S(rs, 4))

    def start_item(self, u, sfx):
        """The current item's tile it (in buffer u, score set u % 2) after its K, V are loaded:
        start values, S/dP of tile it when active, the body's variant, start values and first
        row reads of tile it+1."""
        p, s = self.p, self.s
        T0 = S_TMP
        self.cinit(u)
        self.active(S_QT0, T0)
        s(f"s_cmp_eq_u32 {sr(T0)}, 0", S(T0), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lss_{sfx}", [("scc", 0)], skip_xdl=ACC)
        rissued = 0
        for i in range(16):
            while rissued < 16 and rissued - LK <= i:
                self.row_read(rissued, u)
                rissued += 1
            self.sdp_mfma(i, u % 2)
        p.label(f".Lss_{sfx}")
        self.code()
        self.cinit((u + 1) % 4, range(4, 8))   # -D of tile it+1 (its exps' row values come in body it)
        for i in range(LK):
            self.row_read(i, (u + 1) % 4)
        p.branch(f"s_branch .Ldisp{u}", keep_lgkm=True, skip_xdl=ACC)

    # ---------------------------------------------------------------- iteration bodies
    def body(self, u, sdp, ew, masked):
        """Body of iteration it (it % 4 == u): S/dP of tile it+1 (sdp), elementwise + dV/dK of
        tile it (ew), barrier, start values of tile it+2, request of tile it+3.  Enters with
        the first LK row reads of tile it+1 in flight; leaves with those of tile it+2."""
        p = self.p
        J0, J1 = u % 2, (u + 1) % 2
        jb0, jb1, jb2, jb3 = u, (u + 1) % 4, (u + 2) % 4, (u + 3) % 4
        h1 = split_scalar(self.capture(self.tile_offsets, S_H3, S_QT3), 16)
        h2 = split_scalar(self.capture(self.advance_and_code), 16)
        # --- first half: S/dP(it+1) with elementwise(it) between the MFMAs
        rissued = LK
        tissued = 0
        if ew and masked:
            self.mask_threshold(S_QT0)
        slots = self.dvdk_slots()
        first = self.tr_first_use()
        end = 16 + len(slots)
        if sdp:
            for s_ in range(16):
                while rissued < 16 and rissued - LK <= s_:
                    self.row_read(rissued, jb1)
                    rissued += 1
                if ew:
                    while tissued < 16 and 16 + first[tissued] - LV <= s_:
                        self.tr_read(tissued, jb0)
                        tissued += 1
                self.sdp_mfma(s_, J1)
                p.ins.extend(h1[s_])
                if ew and EW_SPLIT:   # pairs n = 0..3 (first query k-step) here
                    if s_ % 4 == 0:
                        self.ew_exp(J0, s_ // 4)
                    elif s_ % 4 == 2:
                        self.ew_rest(J0, s_ // 4, masked)
                elif ew:
                    if s_ % 2 == 0:
                        self.ew_exp(J0, s_ // 2)
                    else:
                        self.ew_rest(J0, s_ // 2, masked)
        else:
            for c in h1:
                p.ins.extend(c)
            if ew:
                nn = 4 if EW_SPLIT else 8
                for n in range(nn + 1):
                    if n < nn:
                        self.ew_exp(J0, n)
                    if n >= 1:
                        self.ew_rest(J0, n - 1, masked)
        # --- barrier: every wave is past the reads of tile it-1; tile it+2 is in LDS
        p.waitcnt(vm=0)
        p.barrier()
        # --- second half: dV/dK(it); start values of tile it+2; DMA of tile it+3
        dma_at = {17: 0, 20: 1, 23: 2, 26: 3, 29: 4}
        for s_ in range(16, end):
            if ew:
                while tissued < 16 and 16 + first[tissued] - LV <= s_:
                    self.tr_read(tissued, jb0)
                    tissued += 1
            if 16 <= s_ < 24:   # -LSE*log2e of tile it+1 (its exps, next body), -D of tile it+2
                self.cinit_read(jb1 if s_ < 20 else jb2, s_ - 16)
            if s_ - 16 < len(h2):
                p.ins.extend(h2[s_ - 16])
            if s_ in dma_at:
                which, i = self.DMA_ORDER[dma_at[s_]]
                self.dma_m0(which, jb3, i)
            if ew:
                self.dvdk_mfma(*slots[s_ - 16])
                if EW_SPLIT and s_ < 24:   # pairs n = 4..7, ready for dV/dK MFMA 8 on
                    n = 4 + (s_ - 16) // 2
                    if s_ % 2 == 0:
                        self.ew_exp(J0, n)
                    else:
                        self.ew_rest(J0, n, masked)
            if s_ in dma_at:
                which, i = self.DMA_ORDER[dma_at[s_]]
                self.dma_ld(which, i)
            if s_ >= end - LK:   # first row reads of tile it+2 for the next body
                self.row_read(s_ - (end - LK), jb2)
        # --- into the next body: the common variant directly, else the dispatcher
        un = (u + 1) % 4
        p.salu(f"s_cmp_eq_u32 {sr(S_CODE)}, 6", S(S_CODE), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lfull{un}", [("scc", 0)], keep_lgkm=True, skip_xdl=ACC)
        p.branch(f"s_branch .Ldisp{un}", keep_lgkm=True, skip_xdl=ACC)


def build(check_ldb: int = 12288, check_ldo: int = 4096, dt: str = "f16") -> str:
    """The kernel's assembly text: tkm_fa_bwd_dkdv_d128_f16 (dt "f16") or _bf16."""
    p = Prog(coalesce_lgkm=True)
    sal = p.salu
    b = Body(p, dt)
    # ---------------------------------------------------------------- scalars
    p.smem(f"s_load_dwordx16 {sr(8, 16)}, {sr(0, 2)}, 0x0", S(8, 16), S(0, 2))
    p.smem(f"s_load_dwordx8 {sr(24, 8)}, {sr(0, 2)}, 0x40", S(24, 8), S(0, 2))
    p.smem(f"s_load_dwordx2 {sr(S_MAGNK, 2)}, {sr(0, 2)}, 0x60", S(S_MAGNK, 2), S(0, 2))
    L = Lanes(p, check_ldb)
    L.shr(V_PT + 0, L.k(6), 0)
    p.readlane(f"v_readfirstlane_b32 {sr(S_WAVE)}, {vr(V_PT + 0)}", V(V_PT + 0), S(S_WAVE))
    p.waitcnt(lgkm=0)
    xcd_slot(p, S_WG, S_NWG, S_TMP, S_TMP + 1)
    T0, T3 = S_TMP, S_TMP + 3
    sal(f"s_add_u32 {sr(T0)}, {sr(S_SEQ)}, 31", S(S_SEQ), S(T0))
    sal(f"s_lshr_b32 {sr(S_QTL)}, {sr(T0)}, 5", S(T0), S(S_QTL))
    sal(f"s_sub_u32 {sr(S_QTL)}, {sr(S_QTL)}, 1", S(S_QTL), S(S_QTL))          # the last query tile
    sal(f"s_lshl_b32 {sr(S_LDB32)}, {sr(S_LDB)}, 5", S(S_LDB), S(S_LDB32))
    sal(f"s_lshl_b32 {sr(S_LDO32)}, {sr(S_LDO)}, 5", S(S_LDO), S(S_LDO32))
    sal(f"s_lshl_b32 {sr(S_LDSW)}, {sr(S_WAVE)}, 11", S(S_WAVE), S(S_LDSW))       # Q/dO rows wave*8..
    sal(f"s_lshl_b32 {sr(S_LDSL)}, {sr(S_WAVE)}, 8", S(S_WAVE), S(S_LDSL))        # the wave's quad slot
    sal(f"s_add_u32 {sr(S_LDSL)}, {sr(S_LDSL)}, {LDS_LD}", S(S_LDSL), S(S_LDSL))
    # ---------------------------------------------------------------- DMA lane offsets
    LANE, L32, HI = V_PT + 1, V_PT + 2, V_PT + 3
    DR, DP, TA, TB, TC = V_PT + 4, V_PT + 5, V_PT + 6, V_PT + 7, V_PT + 8
    lane_basics(L, (LANE, L32, HI))
    L.shr(DR, L.k(4), LANE)
    L.and_(DP, L.k(15), LANE)
    # DMA: wave w, instruction i moves rows w*8 + i*4 + dr: chunk dp ^ swz(row) of row
    # -> LDS slot dp; swz(row) = 4*dr + ((2w + i) & 3)
    wave_vals = np.arange(4)
    L.shl(TA, L.k(2), DR)
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
    p.valu(f"v_mov_b32_e32 {vr(V_L32)}, {vr(L32)}", V(L32), V(V_L32))
    p.valu(f"v_lshlrev_b32_e32 {vr(V_HI4)}, 2, {vr(HI)}", V(HI), V(V_HI4))
    # ---------------------------------------------------------------- DMA descriptor sizes
    # (the same for every item: a batch's Q / dO rows up to the last row's last head of the
    # kv group, a kv group's row values)
    sal(f"s_lshl_b32 {sr(T0)}, {sr(S_G)}, 8", S(S_G), S(T0))
    b.nrec_rows(S_RQ + 2, S_SEQ, S_LDB, T0)
    b.nrec_rows(S_RO + 2, S_SEQ, S_LDO, T0)
    sal(f"s_mul_i32 {sr(S_RL + 2)}, {sr(S_G)}, {sr(S_SP)}", S(S_G) + S(S_SP), S(S_RL + 2))
    sal(f"s_lshl_b32 {sr(S_RL + 2)}, {sr(S_RL + 2)}, 3", S(S_RL + 2), S(S_RL + 2))
    for dst in (S_RQ, S_RO, S_RL):
        sal(f"s_mov_b32 {sr(dst + 3)}, 0x20000", [], S(dst + 3))
    # ---------------------------------------------------------------- first items, tiles 0, 1
    sal(f"s_mov_b32 {sr(S_KA)}, 0", [], S(S_KA))
    sal(f"s_mov_b32 {sr(S_KD)}, 0", [], S(S_KD))
    b.decode_d("p0")
    for t in range(2):
        b.tile_offsets(S_H3, S_QT3)
        b.dma_all(t)
        b.d_advance(f"p{t + 1}")
    b.item_index(S_KA, S_TMP + 16)
    b.decode_a(S_TMP + 16, "p")
    b.kv_load()
    b.tile_offsets(S_H3, S_QT3)
    b.dma_all(2)
    b.d_advance("p3")
    # ---------------------------------------------------------------- LDS read offsets
    # row values: the half-wave hi reads rows 8g + 4hi .. +3 of its wave's slot (+32g, +128)
    L.shl(TA, L.k(4), HI)
    L.add(V_LDR, TA, L.s(S_LDSL, LDS_LD + wave_vals * 256))
    row_read_offsets(L, V_KOFF, (LANE, L32, HI), (TA, TB, TC))
    tr_read_offsets(L, V_VOFF, (LANE, L32, HI), (TA, TB, TC, V_PT + 9, V_PT + 10, V_PT + 11, V_PT + 12))
    _check_lanes(L, check_ldb, check_ldo)
    b.zero_acc()
    b.take_k()
    p.waitcnt(vm=0)
    p.barrier()
    b.start_item(0, "p")
    # ---------------------------------------------------------------- bodies, boundaries
    for u in range(4):
        _dispatch(b, u)
    for u in range(4):
        _boundary(b, u)
    p.label(".Lexit")
    p.waitcnt(vm=0, lgkm=0)   # DMA requests past the last item still write LDS
    p.emit("s_endpgm", BRANCH)
    return kernel_text(f"tkm_fa_bwd_dkdv_d128_{dt}", p.finalize(), lds_bytes=LDS_BYTES, kernarg_bytes=KERNARG_BYTES,
                       next_free_sgpr=NEXT_FREE_SGPR, args=ARGS, wg_ids=(1, 0, 0))


def _check_lanes(L: Lanes, ldb, ldo):
    tid = np.arange(256)
    lane, wave = tid & 63, tid >> 6
    dr, dp = lane // 16, lane % 16
    for i in range(2):
        row = wave * 8 + i * 4 + dr
        chunk = (dp ^ np.vectorize(swz)(row)) << 4
        assert np.array_equal(L.val[V_DOFF + i], (row * ldb + chunk) & 0xFFFFFFFF), f"Q dma {i}"
        assert np.array_equal(L.val[V_DOFF + 2 + i], (row * ldo + chunk) & 0xFFFFFFFF), f"dO dma {i}"
    assert np.array_equal(L.val[V_LOFF], lane * 4)
    # accumulator register r of a lane holds query row mask_c(r) + 4hi; its start value sits at
    # byte 4*(row) of the tile's 128-byte -LSE*log2e run (-D: +128) in the wave's slot, so the
    # read of registers 4g .. 4g+3 at V_LDR + 32g covers rows mask_c(4g) + 4hi .. +3
    hi = lane >> 5
    for g in range(4):
        rows = np.array([mask_c(4 * g + j) for j in range(4)])
        assert np.array_equal(rows, rows[0] + np.arange(4)) and rows[0] == 8 * g
    assert np.array_equal(L.val[V_LDR], LDS_LD + wave * 256 + 16 * hi), "row-value read offsets"


def _dispatch(b: Body, u: int):
    """Dispatcher and the six body variants of residue u: first a DMA stream that moved on to
    its next item (code bit 16), then the end of the current item (code 8), then the variant."""
    p, s = b.p, b.s
    pend = b.prefetch_regs()
    p.label(f".Ldisp{u}")
    p.assume_lgkm(pend)
    s(f"s_bitcmp1_b32 {sr(S_CODE)}, 4", S(S_CODE), [("scc", 0)])
    p.branch(f"s_cbranch_scc0 .Lnod{u}", [("scc", 0)], keep_lgkm=True, skip_xdl=ACC)
    p.waitcnt(lgkm=0)
    s(f"s_add_u32 {sr(S_KD)}, {sr(S_KD)}, 1", S(S_KD), S(S_KD))
    b.decode_d(f"d{u}")
    s(f"s_andn2_b32 {sr(S_CODE)}, {sr(S_CODE)}, 16", S(S_CODE), S(S_CODE))
    p.label(f".Lnod{u}")
    p.assume_lgkm(pend)
    s(f"s_bitcmp1_b32 {sr(S_CODE)}, 3", S(S_CODE), [("scc", 0)])
    p.branch(f"s_cbranch_scc1 .Lbnd{u}", [("scc", 0)], keep_lgkm=True, skip_xdl=ACC)
    for lab, _, _, _ in VARIANTS[:-1]:
        for c in CODES[lab]:
            s(f"s_cmp_eq_u32 {sr(S_CODE)}, {c}", S(S_CODE), [("scc", 0)])
            p.branch(f"s_cbranch_scc1 .L{lab}{u}", [("scc", 0)], keep_lgkm=True, skip_xdl=ACC)
    for lab, sdp, ew, masked in VARIANTS[::-1]:     # idle falls through from the dispatcher
        p.label(f".L{lab}{u}")
        p.assume_lgkm(pend)
        b.body(u, sdp=sdp, ew=ew, masked=masked)


def _boundary(b: Body, u: int):
    """End of the current item before body residue u: request the next item's K, V rows (their
    latency hides behind the epilogue), store the current dK, dV; then the next item (or stop):
    K, V into place, start on tile it (buffer u), whose data the DMA stream has already
    delivered."""
    p, s = b.p, b.s
    I = S_TMP + 16
    p.label(f".Lbnd{u}")
    p.nop(16)                 # MFMA results of the last body before the accumulator reads
    p.waitcnt(lgkm=0)
    K1 = S_TMP
    s(f"s_add_u32 {sr(K1)}, {sr(S_KA)}, 1", S(S_KA), S(K1))
    b.item_index(K1, I)
    s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
    p.branch(f"s_cbranch_scc1 .Lnopf{u}", [("scc", 0)], skip_xdl=ACC)
    b.kv_prefetch(I, f"b{u}")
    p.label(f".Lnopf{u}")
    b.epilogue()
    s(f"s_add_u32 {sr(S_KA)}, {sr(S_KA)}, 1", S(S_KA), S(S_KA))
    s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lexit", [("scc", 0)], skip_xdl=ACC)
    p.comment("next kv")
    b.decode_a(I, f"b{u}")
    p.comment("item")
    b.zero_acc()
    b.kv_take()
    b.start_item(u, f"b{u}")


def main(path: str) -> None:
    with open(path, "w") as f:
        f.write(build())


if __name__ == "__main__":
    import sys
    main(sys.argv[1])

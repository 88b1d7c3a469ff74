"""Generator of the gfx950 assembly FlashAttention backward dQ kernel, D = 128, fp16.

Contract: identical to fa_bwd_dq_kernel (tokamak_amd/csrc/attn_bwd.hip), which replaces the
dQ part of the reference's k_gqa_flash_attn_tc_bwd (src/tkm_gpu.cu:440-598):
    P_ij = exp(s_ij - LSE_i),  dS_ij = P_ij (<dO_i, v_j> - D_i),  dQ_i = scale sum_j dS_ij k_j
over the keys j visible from query row i (j < kv_len[b] and, causal, j <= i); dQ is written
(not accumulated) into dqkv.  With compute_d set it also computes D_i = <O_i, dO_i> in fp32
and writes it to delta and, with -LSE_i*log2(e), to the workspace's row values (per 32-row
tile: the 32 values -LSE*log2e, then the 32 values -D; rows past S zero) that the dK/dV
kernel reads; otherwise it reads D from delta.

Work decomposition: persistent, one workgroup (4 waves, one per SIMD) per compute unit walks
items (batch, q-head, block of 256 query rows; block fastest) in snake order over rounds of
NWG items, consecutive items of a round on one XCD (xcd_slot), so that the blocks of a head
share K/V tiles in its L2 and, for causal, long and short blocks of consecutive rounds pair up.  A wave owns 64 query rows (two blocks of 32): Q and dO of its rows (fp16,
as loaded) sit in AGPRs as the B operands of S^T = K Q^T and
dP^T = V dO^T, dQ^T (C[m = head dim][n = query]) accumulates in AGPRs.  K and V tiles of 32
keys go HBM -> LDS by buffer DMA into four buffers, requested three tiles ahead; the DMA
stream runs on across item boundaries.  Per tile and wave (lane = query row):
    S^T  = K Q^T                     16 MFMAs (unscaled scores, exact products summed in fp32)
    dP^T = V dO^T + (-D)             16 MFMAs (-D: the accumulators' start values, per item)
    dS^T = exp2(fma(S^T, scale*log2e, -LSE*log2e)) dP^T
                                     masked to 0 where the key is hidden, packed to fp16 in
                                     dP^T's registers as the B operand of
    dQ^T += K^T dS^T                 16 MFMAs, K^T read transposed (ds_read_b64_tr_b16)
Every K or V operand read from LDS feeds two MFMAs (both 32-row blocks).  A loop body runs 48
MFMA slots: S^T/dP^T of the next tile with this tile's elementwise work between them, one
workgroup barrier, then dQ^T of this tile with the request of the tile three ahead; the
scalar bookkeeping runs between the MFMAs and a body jumps straight into the next body's
common variant.  At an item's end its dQ leaves through per-wave LDS staging rows so that
each store writes whole 256-byte rows.
"""
from __future__ import annotations

import numpy as np

from .attn_dkdv import split_scalar
from .common import Lanes, lane_basics, row_read_offsets, swz, tr_read_offsets, xcd_slot
from .gfx950 import A, BRANCH, PERMLANE, Prog, S, V, ar, kernel_text, sr, vr

NAME = "tkm_fa_bwd_dq_d128_f16"
MFMA = "v_mfma_f32_32x32x16_f16"
MFMA_OF = {"f16": MFMA, "bf16": "v_mfma_f32_32x32x16_bf16"}
PACK_OF = {"f16": "v_cvt_pk_f16_f32", "bf16": "v_cvt_pk_bf16_f32"}
# bf16 (build(dt="bf16"), tkm_fa_bwd_dq_d128_bf16): dS^T goes to the dQ^T MFMAs as two bf16
# halves, hi = bf16(dS) in dP^T's registers (as fp16 dS^T) and lo = bf16(dS - hi) in S^T's
# registers at the same places (word 4ks + w of the block, written after the steps that read
# registers 0 .. 8ks+2w+1), so each K^T read feeds four MFMAs and a body has 64 slots: S^T/dP^T
# in 0..31, dQ^T in 32..63.  D sums the products of bf16 O and dO halves (unpacked by shift and
# mask) in fp32.
ROWB = 256
NBUF = 4
TILE = 32 * ROWB                    # 8 KB: one 32-key tile of K or V
BUFB = 2 * TILE                     # K then V
LDS_EPI = NBUF * BUFB               # per wave: 32 rows of 272 B staging dQ for the store
EPI_ROW = 272
EPI_WAVE = 32 * EPI_ROW
LDS_BYTES = LDS_EPI + 4 * EPI_WAVE
LK = 3                              # slots between a row read and its first MFMA
LV = 3                              # slots between a transposed read pair and its first MFMA
                                    # (4 and 4: ~110 cycles more per body, measured)
NRB = 4                             # row-read registers in rotation (x4)
NTB = 4                             # transposed-read registers in rotation (x4)
assert LK <= NRB                    # the first LK row reads of a tile are in flight across bodies

ARGS = [(8 * i, 8, "ptr") for i in range(8)] + [(64 + 4 * i, 4, "val") for i in range(18)]
KERNARG_BYTES = 136

# ---- SGPRs
S_WG, S_KA, S_KD, S_TK, S_CODE, S_IT = 2, 3, 4, 5, 6, 7
S_QKV, S_O, S_DOUT, S_LSE, S_DELTA, S_QUADS, S_DQKV, S_KVLEN = 8, 10, 12, 14, 16, 18, 20, 22
S_SEQ, S_HQ, S_HKV, S_SL2, S_CAUSAL, S_LDB, S_LDO, S_G = 24, 25, 26, 27, 28, 29, 30, 31
S_SCALE, S_NQBLK, S_SP, S_NWG, S_NI, S_BHQ, S_MAGNQ, S_MAGHQ = 32, 33, 34, 35, 36, 37, 38, 39
S_MAGG, S_WD = 40, 41
S_WAVE, S_KVL, S_Q0, S_NT, S_ACTEND, S_MASKB = 42, 43, 44, 45, 46, 47
S_RK, S_RV = 48, 52                    # DMA descriptors of the DMA stream's item
S_T3, S_NTD, S_LDSW, S_LDB32, S_BA, S_HA = 56, 57, 58, 59, 60, 61
S_TMP = 64                             # s64..s95
NEXT_FREE_SGPR = 96

# ---- VGPRs
V_SET = (0, 64)         # set J: S^T qb at +16qb, dP^T qb at +32+16qb; after the elementwise
                        # step, the packed dS^T (qb, ks) in dP^T qb's registers 4ks .. 4ks+3
V_CD = (128, 176)       # -D of the lane's row, 16 copies per qb (dP^T's start values)
V_CS = 144              # -LSE*log2e of the lane's row, at +16qb (the exps' offset)
V_RB = 192              # row-read buffers
V_TB = V_RB + 4 * NRB   # transposed-read buffers
V_KOFF = V_TB + 4 * NTB
V_VOFF = V_KOFF + 8
V_DOFF = V_VOFF + 8     # DMA rows (2)
V_DA = V_DOFF + 2       # DMA addresses (2: each is read when its request issues)
V_L32 = V_DA + 2
V_HI4 = V_L32 + 1
V_TK = V_HI4 + 1        # mask thresholds per qb (2)
V_T = V_TK + 2          # temporaries (8); D of the lane's row per qb in V_T+1, V_T+2 at an item start
V_ND = V_T + 1
V_SPL = V_CS + 1        # bf16 split temporaries (5): in a body only V_CS and V_CS + 16 of the
                        # start-value range are live (the rest serves the item boundary)
assert V_T + 8 <= 256
V_PT = 100              # prologue lane scratch (score set 1, free until the first body)
EPI_BASE = V_CD[0]      # epilogue temporaries at an item boundary (the start values are rebuilt
                        # after it): clear of the prefetched rows

# ---- AGPRs
A_DQ, A_Q, A_O = 0, 128, 192
ACC = set(A(A_DQ, 128))

VARIANTS = [("full", True, True, False), ("fullm", True, True, True), ("sdp", True, False, False),
            ("last", False, True, False), ("lastm", False, True, True), ("idle", False, False, False)]
CODES = {"full": (6,), "fullm": (7,), "sdp": (4, 5), "last": (2,), "lastm": (3,), "idle": (0, 1)}


def kc(r):
    """Key offset (within the tile, lane half aside) of accumulator register r."""
    return (r // 4) * 8 + (r % 4)


def sblk(J, which, qb):
    return V_SET[J] + 32 * which + 16 * qb


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
        saved = self.p
        self.p = Prog()
        try:
            fn(*args)
            return self.p.ins
        finally:
            self.p = saved

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

    def nrec_rows(self, dst, rows, stride):
        """dst = bytes of a descriptor over `rows` rows of `stride` bytes whose lanes touch
        the first 256 bytes of each row (one head): (rows-1)*stride + 256, 0 without rows.
        It ends at the last row's head, so no request reaches past the tensor's end."""
        s = self.s
        s(f"s_mul_i32 {sr(dst)}, {sr(rows)}, {sr(stride)}", S(rows) + S(stride), S(dst))
        s(f"s_sub_u32 {sr(dst)}, {sr(dst)}, {sr(stride)}", S(dst) + S(stride), S(dst))
        s(f"s_add_u32 {sr(dst)}, {sr(dst)}, 0x100", S(dst), S(dst))
        s(f"s_max_i32 {sr(dst)}, {sr(dst)}, 0", S(dst), S(dst))

    def rsrc(self, dst, src, rows, stride, extra, nrec):
        """Descriptor: base src + rows*stride (+ extra), nrec bytes (SGPR)."""
        self.add64(dst, src, rows, stride, extra)
        self.s(f"s_and_b32 {sr(dst + 1)}, {sr(dst + 1)}, 0xffff", S(dst + 1), S(dst + 1))
        self.s(f"s_mov_b32 {sr(dst + 2)}, {sr(nrec)}", S(nrec), S(dst + 2))
        self.s(f"s_mov_b32 {sr(dst + 3)}, 0x20000", [], S(dst + 3))

    # ---------------------------------------------------------------- items
    def item_index(self, k_sgpr, dst):
        s, T = self.s, S_TMP + 12
        s(f"s_mul_i32 {sr(dst)}, {sr(k_sgpr)}, {sr(S_NWG)}", S(k_sgpr) + S(S_NWG), S(dst))
        s(f"s_sub_u32 {sr(T)}, {sr(S_NWG)}, 1", S(S_NWG), S(T))
        s(f"s_sub_u32 {sr(T)}, {sr(T)}, {sr(S_WG)}", S(T) + S(S_WG), S(T))
        s(f"s_bitcmp1_b32 {sr(k_sgpr)}, 0", S(k_sgpr), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T)}, {sr(T)}, {sr(S_WG)}", S(T) + S(S_WG) + [("scc", 0)], S(T))
        s(f"s_add_u32 {sr(dst)}, {sr(dst)}, {sr(T)}", S(dst) + S(T), S(dst))

    def divide(self, x, d_sgpr, magic, q, rem):
        """q = x / d (multiply-high by the host's reciprocal, exact for the indices that occur;
        magic 0 means d = 1), rem = x - q*d."""
        s = self.s
        s(f"s_mul_hi_u32 {sr(q)}, {sr(x)}, {sr(magic)}", S(x) + S(magic), S(q))
        s(f"s_cmp_eq_u32 {sr(magic)}, 0", S(magic), [("scc", 0)])
        s(f"s_cselect_b32 {sr(q)}, {sr(x)}, {sr(q)}", S(x) + S(q) + [("scc", 0)], S(q))
        if rem is not None:
            s(f"s_mul_i32 {sr(rem)}, {sr(q)}, {sr(d_sgpr)}", S(q) + S(d_sgpr), S(rem))
            s(f"s_sub_u32 {sr(rem)}, {sr(x)}, {sr(rem)}", S(x) + S(rem), S(rem))

    def decode(self, i, z, b, h, kvh):
        """item i -> (b, h, kv head, query block z): z fastest."""
        R = S_TMP + 13
        self.divide(i, S_NQBLK, S_MAGNQ, R, z)
        self.divide(R, S_HQ, S_MAGHQ, b, h)
        self.divide(h, S_G, S_MAGG, kvh, None)

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

    def tiles_of(self, z, kvl, qblk, nt):
        """qblk = causal ? n_qblk-1-z : z; nt = max(1, ceil(kv_end/32)), kv_end = causal ?
        min(kvl, 256 qblk + 256) : kvl (an item without keys keeps one tile no wave uses)."""
        s, T = self.s, S_TMP + 12
        s(f"s_sub_u32 {sr(qblk)}, {sr(S_NQBLK)}, 1", S(S_NQBLK), S(qblk))
        s(f"s_sub_u32 {sr(qblk)}, {sr(qblk)}, {sr(z)}", S(qblk) + S(z), S(qblk))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(qblk)}, {sr(z)}, {sr(qblk)}", S(z) + S(qblk) + [("scc", 0)], S(qblk))
        s(f"s_lshl_b32 {sr(T)}, {sr(qblk)}, 8", S(qblk), S(T))
        s(f"s_add_u32 {sr(T)}, {sr(T)}, 0x100", S(T), S(T))
        s(f"s_min_u32 {sr(T)}, {sr(T)}, {sr(kvl)}", S(T) + S(kvl), S(T))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T)}, {sr(kvl)}, {sr(T)}", S(kvl) + S(T) + [("scc", 0)], S(T))
        s(f"s_add_u32 {sr(T)}, {sr(T)}, 31", S(T), S(T))
        s(f"s_lshr_b32 {sr(nt)}, {sr(T)}, 5", S(T), S(nt))
        s(f"s_max_u32 {sr(nt)}, {sr(nt)}, 1", S(nt), S(nt))

    def decode_d(self, sfx):
        """DMA stream: item of round S_KD -> K, V descriptors (rows past kv_len read as zero),
        NTD; tile 0.  Past the last item the stream keeps re-reading its item."""
        p, s = self.p, self.s
        I, Z, B, H, KVH, KVL, QB = (S_TMP + k for k in range(7))
        T0, COL = S_TMP + 7, S_TMP + 8
        NREC = S_TMP + 9
        self.item_index(S_KD, I)
        s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
        p.branch(f"s_cbranch_scc0 .Ldd_{sfx}", [("scc", 0)], skip_xdl=ACC)
        s(f"s_mov_b32 {sr(S_NTD)}, 0x7fffffff", [], S(S_NTD))
        p.branch(f"s_branch .Lde_{sfx}", skip_xdl=ACC)
        p.label(f".Ldd_{sfx}")
        self.decode(I, Z, B, H, KVH)
        self.kvl_of(B, KVL, f".Ldk_{sfx}")
        self.tiles_of(Z, KVL, QB, S_NTD)
        s(f"s_mov_b32 {sr(S_T3)}, 0", [], S(S_T3))
        s(f"s_mul_i32 {sr(T0)}, {sr(B)}, {sr(S_SEQ)}", S(B) + S(S_SEQ), S(T0))
        s(f"s_add_u32 {sr(COL)}, {sr(S_HQ)}, {sr(KVH)}", S(S_HQ) + S(KVH), S(COL))
        s(f"s_lshl_b32 {sr(COL)}, {sr(COL)}, 8", S(COL), S(COL))
        self.nrec_rows(NREC, KVL, S_LDB)
        self.rsrc(S_RK, S_QKV, T0, S_LDB, COL, NREC)
        s(f"s_lshl_b32 {sr(S_TMP + 10)}, {sr(S_HKV)}, 8", S(S_HKV), S(S_TMP + 10))
        s(f"s_add_u32 {sr(COL)}, {sr(COL)}, {sr(S_TMP + 10)}", S(COL) + S(S_TMP + 10), S(COL))
        self.rsrc(S_RV, S_QKV, T0, S_LDB, COL, NREC)
        p.label(f".Lde_{sfx}")

    def d_advance(self, sfx):
        """DMA stream to its next tile (outside the loop bodies)."""
        p, s = self.p, self.s
        s(f"s_add_u32 {sr(S_T3)}, {sr(S_T3)}, 1", S(S_T3), S(S_T3))
        s(f"s_cmp_lt_u32 {sr(S_T3)}, {sr(S_NTD)}", S(S_T3) + S(S_NTD), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lda_{sfx}", [("scc", 0)], skip_xdl=ACC)
        s(f"s_add_u32 {sr(S_KD)}, {sr(S_KD)}, 1", S(S_KD), S(S_KD))
        self.decode_d(sfx)
        p.label(f".Lda_{sfx}")

    def decode_a(self, i, sfx):
        """Current item i: rows, keys, tiles, per-wave activity and mask bounds."""
        s = self.s
        Z, KVH, QB = S_TMP, S_TMP + 1, S_TMP + 2
        T0, T1 = S_TMP + 3, S_TMP + 4
        self.decode(i, Z, S_BA, S_HA, KVH)
        self.kvl_of(S_BA, S_KVL, f".Lak_{sfx}")
        self.tiles_of(Z, S_KVL, QB, S_NT)
        s(f"s_lshl_b32 {sr(S_Q0)}, {sr(QB)}, 8", S(QB), S(S_Q0))
        s(f"s_lshl_b32 {sr(T0)}, {sr(S_WAVE)}, 6", S(S_WAVE), S(T0))
        s(f"s_add_u32 {sr(S_Q0)}, {sr(S_Q0)}, {sr(T0)}", S(S_Q0) + S(T0), S(S_Q0))
        # active tiles: t < ACTEND = causal ? min(NT, (q0 + 63)/32 + 1) : NT; none without keys
        s(f"s_add_u32 {sr(T0)}, {sr(S_Q0)}, 63", S(S_Q0), S(T0))
        s(f"s_lshr_b32 {sr(T0)}, {sr(T0)}, 5", S(T0), S(T0))
        s(f"s_add_u32 {sr(T0)}, {sr(T0)}, 1", S(T0), S(T0))
        s(f"s_min_u32 {sr(T0)}, {sr(T0)}, {sr(S_NT)}", S(T0) + S(S_NT), S(T0))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_ACTEND)}, {sr(S_NT)}, {sr(T0)}", S(S_NT) + S(T0) + [("scc", 0)], S(S_ACTEND))
        s(f"s_cmp_eq_u32 {sr(S_KVL)}, 0", S(S_KVL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_ACTEND)}, 0, {sr(S_ACTEND)}", S(S_ACTEND) + [("scc", 0)], S(S_ACTEND))
        # tiles needing a mask: t >= MASKB = min(kvl/32, causal ? q0/32 : NT)
        s(f"s_lshr_b32 {sr(T0)}, {sr(S_KVL)}, 5", S(S_KVL), S(T0))
        s(f"s_lshr_b32 {sr(T1)}, {sr(S_Q0)}, 5", S(S_Q0), S(T1))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T1)}, {sr(S_NT)}, {sr(T1)}", S(S_NT) + S(T1) + [("scc", 0)], S(T1))
        s(f"s_min_u32 {sr(S_MASKB)}, {sr(T0)}, {sr(T1)}", S(T0) + S(T1), S(S_MASKB))
        s(f"s_mov_b32 {sr(S_IT)}, 0", [], S(S_IT))

    def code(self):
        """S_CODE for body S_IT: 8 at the item's end, else 4*act(next) + 2*act(this) + mask."""
        s = self.s
        A0, A1, T = S_TMP + 15, S_TMP + 16, S_TMP + 17
        s(f"s_cmp_lt_u32 {sr(S_IT)}, {sr(S_ACTEND)}", S(S_IT) + S(S_ACTEND), [("scc", 0)])
        s(f"s_cselect_b32 {sr(A0)}, 2, 0", [("scc", 0)], S(A0))
        s(f"s_add_u32 {sr(T)}, {sr(S_IT)}, 1", S(S_IT), S(T))
        s(f"s_cmp_lt_u32 {sr(T)}, {sr(S_ACTEND)}", S(T) + S(S_ACTEND), [("scc", 0)])
        s(f"s_cselect_b32 {sr(A1)}, 4, 0", [("scc", 0)], S(A1))
        s(f"s_cmp_lt_u32 {sr(T)}, {sr(S_NT)}", S(T) + S(S_NT), [("scc", 0)])
        s(f"s_cselect_b32 {sr(A1)}, {sr(A1)}, 0", S(A1) + [("scc", 0)], S(A1))
        s(f"s_cmp_ge_u32 {sr(S_IT)}, {sr(S_MASKB)}", S(S_IT) + S(S_MASKB), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T)}, 1, 0", [("scc", 0)], S(T))
        s(f"s_or_b32 {sr(A0)}, {sr(A0)}, {sr(A1)}", S(A0) + S(A1), S(A0))
        s(f"s_or_b32 {sr(S_CODE)}, {sr(A0)}, {sr(T)}", S(A0) + S(T), S(S_CODE))
        s(f"s_cmp_ge_u32 {sr(S_IT)}, {sr(S_NT)}", S(S_IT) + S(S_NT), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_CODE)}, 8, {sr(S_CODE)}", S(S_CODE) + [("scc", 0)], S(S_CODE))

    def advance_and_code(self):
        s = self.s
        s(f"s_add_u32 {sr(S_T3)}, {sr(S_T3)}, 1", S(S_T3), S(S_T3))
        s(f"s_add_u32 {sr(S_IT)}, {sr(S_IT)}, 1", S(S_IT), S(S_IT))
        self.code()
        T = S_TMP + 17
        s(f"s_cmp_ge_u32 {sr(S_T3)}, {sr(S_NTD)}", S(S_T3) + S(S_NTD), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T)}, 16, 0", [("scc", 0)], S(T))
        s(f"s_or_b32 {sr(S_CODE)}, {sr(S_CODE)}, {sr(T)}", S(S_CODE) + S(T), S(S_CODE))

    def tile_offset(self):
        self.s(f"s_mul_i32 {sr(S_TK)}, {sr(S_T3)}, {sr(S_LDB32)}", S(S_T3) + S(S_LDB32), S(S_TK))

    # ---------------------------------------------------------------- DMA
    DMA_ORDER = (("k", 0), ("k", 1), ("v", 0), ("v", 1))

    def dma_m0(self, which, jb, i):
        k = (0 if which == "k" else 2) + i
        off = jb * BUFB + (TILE if which == "v" else 0) + i * 1024
        self.s(f"s_add_u32 m0, {sr(S_LDSW)}, {off}", S(S_LDSW), [("m0", 0)])
        self.p.valu(f"v_add_u32_e32 {vr(V_DA + k % 2)}, {sr(S_TK)}, {vr(V_DOFF + i)}", S(S_TK) + V(V_DOFF + i), V(V_DA + k % 2))

    def dma_ld(self, which, i):
        k = (0 if which == "k" else 2) + i
        rs = S_RK if which == "k" else S_RV
        self.p.dma(f"buffer_load_dwordx4 {vr(V_DA + k % 2)}, {sr(rs, 4)}, 0 offen lds", V(V_DA + k % 2) + S(rs, 4))

    def dma_all(self, jb):
        for which, i in self.DMA_ORDER:
            self.dma_m0(which, jb, i)
            self.dma_ld(which, i)

    # ---------------------------------------------------------------- LDS reads
    def row_read(self, ri, jb):
        """Read ri = 2ks + (0: K, 1: V) rows, chunk 2ks + hi, of tile buffer jb."""
        ks, which = ri // 2, ri % 2
        dst = V_RB + (ri % NRB) * 4
        off = jb * BUFB + which * TILE
        self.p.ds_read(f"ds_read_b128 {vr(dst, 4)}, {vr(V_KOFF + ks)} offset:{off}", V(dst, 4), V(V_KOFF + ks))

    def prefetch_regs(self):
        return [V(V_RB + (i % NRB) * 4, 4) for i in range(LK)]

    def tr_read(self, vi, jb):
        """K^T read vi = 4ks + db of tile buffer jb."""
        ks, db = vi // 4, vi % 4
        dst = V_TB + (vi % NTB) * 4
        off = jb * BUFB + ks * 16 * ROWB
        for tt in range(2):
            self.p.ds_read(f"ds_read_b64_tr_b16 {vr(dst + 2 * tt, 2)}, {vr(V_VOFF + tt * 4 + db)} offset:{off}",
                           V(dst + 2 * tt, 2), V(V_VOFF + tt * 4 + db))

    # ---------------------------------------------------------------- MFMAs
    def sdp_mfma(self, i, J):
        """Slot i of S^T/dP^T: ks = i // 4, (i % 4) = S qb0, S qb1, dP qb0, dP qb1."""
        ks, k4 = i // 4, i % 4
        which, qb = k4 // 2, k4 % 2
        dst = sblk(J, which, qb)
        if ks == 0:
            c = None if which == 0 else V_CD[qb]
        else:
            c = dst
        b = (A_Q if which == 0 else A_O) + (qb * 8 + ks) * 4
        self.p.mfma(self.mfma_op, dst, V_RB + ((2 * ks + which) % NRB) * 4, b, c, b_acc=True)

    @staticmethod
    def ds_reg(J, qb, ks):
        """First of the four registers of packed dS^T (qb, ks) of set J (in dP^T qb's registers)."""
        return sblk(J, 1, qb) + 4 * ks

    @staticmethod
    def ds_lo_reg(J, qb, ks):
        """bf16: first of the four registers of the lo halves of dS^T (qb, ks) (in S^T qb's)."""
        return sblk(J, 0, qb) + 4 * ks

    def dq_per_read(self):
        """dQ^T MFMAs per K^T read: one per block of 32 rows, twice with the bf16 split."""
        return 4 if self.split else 2

    def dq_mfma(self, j, J):
        """Slot j of dQ^T from set J: vi = j // dq_per_read() (ks = vi // 4, db = vi % 4),
        qb = j % 2; bf16: hi for j % 4 < 2, then lo."""
        n = self.dq_per_read()
        vi, qb, lo = j // n, j % 2, (j % n) >= 2
        ks, db = vi // 4, vi % 4
        acc = A_DQ + (db * 2 + qb) * 16
        b = self.ds_lo_reg(J, qb, ks) if lo else self.ds_reg(J, qb, ks)
        self.p.mfma(self.mfma_op, acc, V_TB + (vi % NTB) * 4, b, acc, dst_acc=True)

    # ---------------------------------------------------------------- elementwise (set J)
    @staticmethod
    def ew_regs(J, n):
        qb, ks, w = n // 8, (n % 8) // 4, n % 4
        r0 = 8 * ks + 2 * w
        return qb, ks, w, sblk(J, 0, qb) + r0, sblk(J, 1, qb) + r0, r0

    def ew_exp(self, J, n):
        qb, _, _, x, _, _ = self.ew_regs(J, n)
        for r in (x, x + 1):
            self.p.valu(f"v_fma_f32 {vr(r)}, {vr(r)}, {sr(S_SL2)}, {vr(V_CS + 16 * qb)}",
                        V(r) + S(S_SL2) + V(V_CS + 16 * qb), V(r))
        for r in (x, x + 1):
            self.p.trans(f"v_exp_f32_e32 {vr(r)}, {vr(r)}", V(r), V(r))

    def ew_rest(self, J, n, masked):
        p = self.p
        qb, ks, w, x, dp, r0 = self.ew_regs(J, n)
        for k in range(2):
            if masked:   # hidden iff kc > tq
                p.valu(f"v_cmp_gt_i32_e32 vcc, {kc(r0 + k)}, {vr(V_TK + qb)}", V(V_TK + qb), [("vcc", 0)])
                p.valu(f"v_cndmask_b32_e64 {vr(x + k)}, {vr(x + k)}, 0, vcc", V(x + k) + [("vcc", 0)], V(x + k))
            p.valu(f"v_mul_f32_e32 {vr(dp + k)}, {vr(x + k)}, {vr(dp + k)}", V(x + k) + V(dp + k), V(dp + k))
        # dS^T word (qb, ks, w) goes to register 4ks + w of dP^T qb: read by this step or an earlier one
        ds = self.ds_reg(J, qb, ks) + w
        if not self.split:
            p.valu(f"{self.pack_op} {vr(ds)}, {vr(dp)}, {vr(dp + 1)}", V(dp, 2), V(ds))
            return
        # bf16: hi = bf16(dS), lo = bf16(dS - hi); hi's halves as fp32 are its word shifted up /
        # masked.  The lo word goes to register 4ks + w of S^T qb, which this step or an
        # earlier one has read.  The hi word's register is this step's own dS (ks = w = 0), so
        # there it is formed in a temporary and moved after the residuals.
        t0, t1, th = V_SPL + 2 * (n % 2), V_SPL + 2 * (n % 2) + 1, V_SPL + 4
        hw = th if ds in (dp, dp + 1) else ds
        p.valu(f"v_cvt_pk_bf16_f32 {vr(hw)}, {vr(dp)}, {vr(dp + 1)}", V(dp, 2), V(hw))
        p.valu(f"v_lshlrev_b32_e32 {vr(t0)}, 16, {vr(hw)}", V(hw), V(t0))
        p.valu(f"v_and_b32_e32 {vr(t1)}, 0xffff0000, {vr(hw)}", V(hw), V(t1))
        p.valu(f"v_sub_f32_e32 {vr(dp)}, {vr(dp)}, {vr(t0)}", V(dp) + V(t0), V(dp))
        p.valu(f"v_sub_f32_e32 {vr(dp + 1)}, {vr(dp + 1)}, {vr(t1)}", V(dp + 1) + V(t1), V(dp + 1))
        lw = self.ds_lo_reg(J, qb, ks) + w
        p.valu(f"v_cvt_pk_bf16_f32 {vr(lw)}, {vr(dp)}, {vr(dp + 1)}", V(dp, 2), V(lw))
        if hw != ds:
            p.valu(f"v_mov_b32_e32 {vr(ds)}, {vr(hw)}", V(hw), V(ds))

    def mask_threshold(self):
        """Per qb: tq = min(causal ? q - k0 - 4hi : big, kvl - 1 - k0 - 4hi), k0 = 32*IT, q =
        q0 + 32qb + l32; key offset kc(r) is hidden iff kc(r) > tq."""
        p, s = self.p, self.s
        K0, T1, T2 = S_TMP + 9, S_TMP + 10, S_TMP + 11
        s(f"s_lshl_b32 {sr(K0)}, {sr(S_IT)}, 5", S(S_IT), S(K0))
        s(f"s_sub_u32 {sr(T1)}, {sr(S_KVL)}, {sr(K0)}", S(S_KVL) + S(K0), S(T1))
        s(f"s_sub_u32 {sr(T1)}, {sr(T1)}, 1", S(T1), S(T1))
        for qb in range(2):
            s(f"s_add_u32 {sr(T2)}, {sr(S_Q0)}, {32 * qb}", S(S_Q0), S(T2))
            s(f"s_sub_u32 {sr(T2)}, {sr(T2)}, {sr(K0)}", S(T2) + S(K0), S(T2))
            s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
            s(f"s_cselect_b32 {sr(T2)}, 0x3fffffff, {sr(T2)}", S(T2) + [("scc", 0)], S(T2))
            th = V_TK + qb
            p.valu(f"v_add_u32_e32 {vr(th)}, {sr(T2)}, {vr(V_L32)}", S(T2) + V(V_L32), V(th))
            p.valu(f"v_min_i32_e32 {vr(th)}, {sr(T1)}, {vr(th)}", S(T1) + V(th), V(th))
            p.valu(f"v_sub_u32_e32 {vr(th)}, {vr(th)}, {vr(V_HI4)}", V(th) + V(V_HI4), V(th))

    # ---------------------------------------------------------------- bodies
    def body(self, u, sdp, ew, masked):
        """Body of tile it (it % 4 == u): S^T/dP^T of tile it+1 (sdp), elementwise + dQ^T of
        tile it (ew), barrier, request of tile it+3.  Enters with the first LK row reads of
        tile it+1 in flight; leaves with those of tile it+2."""
        p = self.p
        J0, J1 = u % 2, (u + 1) % 2
        jb0, jb1, jb2, jb3 = u, (u + 1) % 4, (u + 2) % 4, (u + 3) % 4
        h1 = split_scalar(self.capture(self.tile_offset), 32)
        h2 = split_scalar(self.capture(self.advance_and_code), 16)
        rissued = LK
        tissued = 0
        if ew and masked:
            self.mask_threshold()
        # --- S^T/dP^T(it+1), elementwise(it) between: exp at slot 2n, the rest at 2n+1
        if sdp:
            for s_ in range(32):
                while rissued < 16 and 2 * rissued - LK <= s_:
                    self.row_read(rissued, jb1)
                    rissued += 1
                if ew:
                    while tissued < 8 and 32 + self.dq_per_read() * tissued - LV <= s_:
                        self.tr_read(tissued, jb0)
                        tissued += 1
                self.sdp_mfma(s_, J1)
                p.ins.extend(h1[s_])
                if ew:
                    if s_ % 2 == 0:
                        self.ew_exp(J0, s_ // 2)
                    else:
                        self.ew_rest(J0, s_ // 2, masked)
        else:
            for c in h1:
                p.ins.extend(c)
            if ew:
                for n in range(17):
                    if n < 16:
                        self.ew_exp(J0, n)
                    if n >= 1:
                        self.ew_rest(J0, n - 1, masked)
        p.waitcnt(vm=0)
        p.barrier()
        # --- dQ^T(it); DMA of tile it+3; first row reads of tile it+2
        dma_at = {34: 0, 38: 1, 42: 2, 46: 3}
        per = self.dq_per_read()
        end = 32 + 8 * per
        for s_ in range(32, end):
            if ew:
                while tissued < 8 and 32 + per * tissued - LV <= s_:
                    self.tr_read(tissued, jb0)
                    tissued += 1
            if s_ - 32 < len(h2):
                p.ins.extend(h2[s_ - 32])
            if s_ in dma_at:
                which, i = self.DMA_ORDER[dma_at[s_]]
                self.dma_m0(which, jb3, i)
            if ew:
                self.dq_mfma(s_ - 32, J0)
            if s_ in dma_at:
                which, i = self.DMA_ORDER[dma_at[s_]]
                self.dma_ld(which, i)
            if s_ >= end - LK:
                self.row_read(s_ - (end - LK), jb2)
        un = (u + 1) % 4
        p.salu(f"s_cmp_eq_u32 {sr(S_CODE)}, 6", S(S_CODE), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lfull{un}", [("scc", 0)], keep_lgkm=True, skip_xdl=ACC)
        p.branch(f"s_branch .Ldisp{un}", keep_lgkm=True, skip_xdl=ACC)

    # ---------------------------------------------------------------- item start / end
    def zero_acc(self):
        p = self.p
        for i in range(4):
            p.valu(f"v_mov_b32_e32 {vr(V_TB + i)}, 0", [], V(V_TB + i))
        for i in range(8):
            p.mfma(MFMA, A_DQ + 16 * i, V_TB, V_TB, None, dst_acc=True)

    def rows_issue(self, b, h, q0, prefetch, sfx):
        """Loads of Q, dO (and, computing D, O) of the wave's 64 rows of (batch b, head h)
        from row q0 (SGPRs), and of their LSE: lane (l32, hi) loads row q0 + 32qb + l32, bytes
        hi*16 + 32ks .. +15.  Q -> VGPRs 0..63; LSE -> V_T+5, +6.  Direct (item start): dO ->
        VGPRs 64..127, O -> 128..191, tracked.  Prefetch (before the previous item's
        epilogue, whose time covers their latency): dO -> its AGPRs, O -> VGPRs 64..127,
        untracked (the caller waits with vmcnt(0))."""
        p, s = self.p, self.s
        RQ, RDO, RO_, RL = S_TMP + 20, S_TMP + 24, S_TMP + 28, S_TMP + 4
        T0, COL, NREC = S_TMP, S_TMP + 1, S_TMP + 2
        s(f"s_mul_i32 {sr(T0)}, {sr(b)}, {sr(S_SEQ)}", S(b) + S(S_SEQ), S(T0))
        s(f"s_lshl_b32 {sr(COL)}, {sr(h)}, 8", S(h), S(COL))
        self.nrec_rows(NREC, S_SEQ, S_LDB)
        self.rsrc(RQ, S_QKV, T0, S_LDB, COL, NREC)
        self.nrec_rows(NREC, S_SEQ, S_LDO)
        self.rsrc(RDO, S_DOUT, T0, S_LDO, COL, NREC)
        self.rsrc(RO_, S_O, T0, S_LDO, COL, NREC)
        QO, OO = V_T, V_T + 2
        for qb in range(2):
            p.valu(f"v_add_u32_e32 {vr(V_T + 4)}, {sr(q0)}, {vr(V_L32)}", S(q0) + V(V_L32), V(V_T + 4))
            if qb:
                p.valu(f"v_add_u32_e32 {vr(V_T + 4)}, 32, {vr(V_T + 4)}", V(V_T + 4), V(V_T + 4))
            p.valu(f"v_mul_lo_u32 {vr(QO + qb)}, {vr(V_T + 4)}, {sr(S_LDB)}", V(V_T + 4) + S(S_LDB), V(QO + qb))
            p.valu(f"v_lshl_add_u32 {vr(QO + qb)}, {vr(V_HI4)}, 2, {vr(QO + qb)}", V(V_HI4) + V(QO + qb), V(QO + qb))
            p.valu(f"v_mul_lo_u32 {vr(OO + qb)}, {vr(V_T + 4)}, {sr(S_LDO)}", V(V_T + 4) + S(S_LDO), V(OO + qb))
            p.valu(f"v_lshl_add_u32 {vr(OO + qb)}, {vr(V_HI4)}, 2, {vr(OO + qb)}", V(V_HI4) + V(OO + qb), V(OO + qb))
        for qb in range(2):
            for ks in range(8):
                r = (qb * 8 + ks) * 4
                p.vmem_load(f"buffer_load_dwordx4 {vr(r, 4)}, {vr(QO + qb)}, {sr(RQ, 4)}, 0 offen offset:{ks * 32}",
                            V(r, 4), V(QO + qb) + S(RQ, 4), untracked=prefetch)
                dst, regs = (ar(A_O + r, 4), A(A_O + r, 4)) if prefetch else (vr(64 + r, 4), V(64 + r, 4))
                p.vmem_load(f"buffer_load_dwordx4 {dst}, {vr(OO + qb)}, {sr(RDO, 4)}, 0 offen offset:{ks * 32}",
                            regs, V(OO + qb) + S(RDO, 4), untracked=prefetch)
        # LSE (row q, zero past S)
        s(f"s_mul_i32 {sr(T0)}, {sr(b)}, {sr(S_HQ)}", S(b) + S(S_HQ), S(T0))
        s(f"s_add_u32 {sr(T0)}, {sr(T0)}, {sr(h)}", S(T0) + S(h), S(T0))
        s(f"s_lshl_b32 {sr(NREC)}, {sr(S_SEQ)}, 2", S(S_SEQ), S(NREC))
        s(f"s_mov_b32 {sr(COL)}, 4", [], S(COL))
        s(f"s_mul_i32 {sr(S_TMP + 3)}, {sr(T0)}, {sr(S_SEQ)}", S(T0) + S(S_SEQ), S(S_TMP + 3))
        self.rsrc(RL, S_LSE, S_TMP + 3, COL, None, NREC)
        LO = V_T + 4
        p.valu(f"v_add_u32_e32 {vr(LO)}, {sr(q0)}, {vr(V_L32)}", S(q0) + V(V_L32), V(LO))
        p.valu(f"v_lshlrev_b32_e32 {vr(LO)}, 2, {vr(LO)}", V(LO), V(LO))
        for qb in range(2):
            p.vmem_load(f"buffer_load_dword {vr(V_T + 5 + qb)}, {vr(LO)}, {sr(RL, 4)}, 0 offen offset:{128 * qb}",
                        V(V_T + 5 + qb), V(LO) + S(RL, 4), untracked=prefetch)
        s(f"s_cmp_eq_u32 {sr(S_WD)}, 0", S(S_WD), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lro_{sfx}", [("scc", 0)], skip_xdl=ACC)
        ob = 64 if prefetch else 128
        for qb in range(2):
            for ks in range(8):
                r = (qb * 8 + ks) * 4
                p.vmem_load(f"buffer_load_dwordx4 {vr(ob + r, 4)}, {vr(OO + qb)}, {sr(RO_, 4)}, 0 offen offset:{ks * 32}",
                            V(ob + r, 4), V(OO + qb) + S(RO_, 4), untracked=prefetch)
        p.label(f".Lro_{sfx}")

    def rows_d(self, prefetched, sfx):
        """D of the wave's rows (the current item's S_BA, S_HA, S_Q0): computed as fp32 sums of
        the exact fp16 products O*dO (plain VALU, no dot op) and written with the row values,
        or read from delta.  The row loads have arrived (tracked, or waited for)."""
        p, s = self.p, self.s
        T0 = S_TMP
        s(f"s_mul_i32 {sr(T0)}, {sr(S_BA)}, {sr(S_HQ)}", S(S_BA) + S(S_HQ), S(T0))
        s(f"s_add_u32 {sr(T0)}, {sr(T0)}, {sr(S_HA)}", S(T0) + S(S_HA), S(T0))
        s(f"s_cmp_eq_u32 {sr(S_WD)}, 0", S(S_WD), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lrd_{sfx}", [("scc", 0)], skip_xdl=ACC)
        ob, dt = (64, V_T + 7) if prefetched else (128, None)
        for qb in range(2):
            acc = V_ND + qb
            p.valu(f"v_mov_b32_e32 {vr(acc)}, 0", [], V(acc))
            for ks in range(8):   # this lane holds d = ks*16 + hi*8 .. +7, lane ^ 32 the rest
                for w in range(4):
                    r = (qb * 8 + ks) * 4 + w
                    if prefetched:
                        p.valu(f"v_accvgpr_read_b32 {vr(dt)}, {ar(A_O + r)}", A(A_O + r), V(dt))
                        dv = dt
                    else:
                        dv = 64 + r
                    if self.split:
                        t0, t1 = V_TB + 4, V_TB + 5   # free at an item start (zeroed after)
                        for op in ("v_lshlrev_b32_e32 {d}, 16, {s}", "v_and_b32_e32 {d}, 0xffff0000, {s}"):
                            p.valu(op.format(d=vr(t0), s=vr(ob + r)), V(ob + r), V(t0))
                            p.valu(op.format(d=vr(t1), s=vr(dv)), V(dv), V(t1))
                            p.valu(f"v_fmac_f32_e32 {vr(acc)}, {vr(t0)}, {vr(t1)}", V(t0) + V(t1) + V(acc), V(acc))
                        continue
                    for half in ("op_sel_hi:[1,1,0]", "op_sel:[1,1,0] op_sel_hi:[1,1,0]"):
                        p.valu(f"v_fma_mix_f32 {vr(acc)}, {vr(ob + r)}, {vr(dv)}, {vr(acc)} {half}",
                               V(ob + r) + V(dv) + V(acc), V(acc))
            t = V_T + 7
            p.valu(f"v_mov_b32_e32 {vr(t)}, {vr(acc)}", V(acc), V(t))
            p.emit(f"v_permlane32_swap_b32_e32 {vr(t)}, {vr(acc)}", PERMLANE, V(t) + V(acc), V(t) + V(acc))
            p.valu(f"v_add_f32_e32 {vr(acc)}, {vr(acc)}, {vr(t)}", V(acc) + V(t), V(acc))
        self.write_d(T0)
        p.branch(f"s_branch .Lrdd_{sfx}", skip_xdl=ACC)
        p.label(f".Lrd_{sfx}")
        COL, NREC, RL = S_TMP + 1, S_TMP + 2, S_TMP + 4
        s(f"s_lshl_b32 {sr(NREC)}, {sr(S_SEQ)}, 2", S(S_SEQ), S(NREC))
        s(f"s_mov_b32 {sr(COL)}, 4", [], S(COL))
        s(f"s_mul_i32 {sr(S_TMP + 3)}, {sr(T0)}, {sr(S_SEQ)}", S(T0) + S(S_SEQ), S(S_TMP + 3))
        self.rsrc(RL, S_DELTA, S_TMP + 3, COL, None, NREC)
        LO = V_T + 4
        p.valu(f"v_add_u32_e32 {vr(LO)}, {sr(S_Q0)}, {vr(V_L32)}", S(S_Q0) + V(V_L32), V(LO))
        p.valu(f"v_lshlrev_b32_e32 {vr(LO)}, 2, {vr(LO)}", V(LO), V(LO))
        for qb in range(2):
            p.vmem_load(f"buffer_load_dword {vr(V_ND + qb)}, {vr(LO)}, {sr(RL, 4)}, 0 offen offset:{128 * qb}",
                        V(V_ND + qb), V(LO) + S(RL, 4))
        p.waitcnt(vm=0)
        p.label(f".Lrdd_{sfx}")

    def rows_load(self, sfx):
        """The current item's rows at its start: loads, then D."""
        self.rows_issue(S_BA, S_HA, S_Q0, False, sfx)
        self.rows_d(False, sfx)

    def rows_prefetch(self, i, sfx):
        """Loads of item i's rows (decoded into temporaries; the current item's state is not
        touched), issued before the current item's epilogue."""
        s = self.s
        Z, B, H, KVH, Q0 = S_TMP + 8, S_TMP + 9, S_TMP + 10, S_TMP + 11, S_TMP + 12
        assert i not in (Z, B, H, KVH, Q0, S_TMP + 13)
        self.decode(i, Z, B, H, KVH)
        s(f"s_sub_u32 {sr(Q0)}, {sr(S_NQBLK)}, 1", S(S_NQBLK), S(Q0))
        s(f"s_sub_u32 {sr(Q0)}, {sr(Q0)}, {sr(Z)}", S(Q0) + S(Z), S(Q0))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(Q0)}, {sr(Z)}, {sr(Q0)}", S(Z) + S(Q0) + [("scc", 0)], S(Q0))
        s(f"s_lshl_b32 {sr(Q0)}, {sr(Q0)}, 8", S(Q0), S(Q0))
        s(f"s_lshl_b32 {sr(Z)}, {sr(S_WAVE)}, 6", S(S_WAVE), S(Z))
        s(f"s_add_u32 {sr(Q0)}, {sr(Q0)}, {sr(Z)}", S(Q0) + S(Z), S(Q0))
        self.rows_issue(B, H, Q0, True, sfx)

    def write_d(self, bh):
        """delta[row] = D and the row values (-LSE*log2e, -D) of the wave's rows (hi == 0 lanes;
        rows past S: only row values, zeros, up to SP)."""
        p, s = self.p, self.s
        RD, RQD = S_TMP + 8, S_TMP + 16
        NREC, C4, T = S_TMP + 2, S_TMP + 1, S_TMP + 3
        E8, NQ = S_TMP + 12, S_TMP + 13
        assert bh not in (NREC, C4, T)
        s(f"s_mul_i32 {sr(T)}, {sr(bh)}, {sr(S_SEQ)}", S(bh) + S(S_SEQ), S(T))
        s(f"s_mov_b32 {sr(C4)}, 4", [], S(C4))
        s(f"s_lshl_b32 {sr(NREC)}, {sr(S_SEQ)}, 2", S(S_SEQ), S(NREC))
        self.rsrc(RD, S_DELTA, T, C4, None, NREC)
        s(f"s_mul_i32 {sr(T)}, {sr(bh)}, {sr(S_SP)}", S(bh) + S(S_SP), S(T))
        s(f"s_mov_b32 {sr(E8)}, 8", [], S(E8))
        s(f"s_lshl_b32 {sr(NQ)}, {sr(S_SP)}, 3", S(S_SP), S(NQ))
        self.rsrc(RQD, S_QUADS, T, E8, None, NQ)
        p.waitcnt(vm=0)   # the LSE loads
        DO_, QD, LG = V_T + 3, V_T + 4, V_T + 0
        for qb in range(2):
            # row q = q0 + 32qb + l32: delta offset 4q; row-tile offset (q>>5)*256 + (q&31)*4
            # (its -D 128 bytes further); hi lanes off
            p.valu(f"v_add_u32_e32 {vr(QD)}, {sr(S_Q0)}, {vr(V_L32)}", S(S_Q0) + V(V_L32), V(QD))
            if qb:
                p.valu(f"v_add_u32_e32 {vr(QD)}, 32, {vr(QD)}", V(QD), V(QD))
            p.valu(f"v_lshlrev_b32_e32 {vr(DO_)}, 2, {vr(QD)}", V(QD), V(DO_))
            p.valu(f"v_and_b32_e32 {vr(V_T + 7)}, 31, {vr(QD)}", V(QD), V(V_T + 7))
            p.valu(f"v_lshrrev_b32_e32 {vr(QD)}, 5, {vr(QD)}", V(QD), V(QD))
            p.valu(f"v_lshlrev_b32_e32 {vr(QD)}, 8, {vr(QD)}", V(QD), V(QD))
            p.valu(f"v_lshl_add_u32 {vr(QD)}, {vr(V_T + 7)}, 2, {vr(QD)}", V(V_T + 7) + V(QD), V(QD))
            p.valu(f"v_cmp_eq_u32_e32 vcc, 0, {vr(V_HI4)}", V(V_HI4), [("vcc", 0)])
            p.valu(f"v_mov_b32_e32 {vr(V_T + 7)}, 0x7ffffff0", [], V(V_T + 7))
            p.valu(f"v_cndmask_b32_e32 {vr(DO_)}, {vr(V_T + 7)}, {vr(DO_)}, vcc", V(V_T + 7) + V(DO_) + [("vcc", 0)], V(DO_))
            p.valu(f"v_cndmask_b32_e32 {vr(QD)}, {vr(V_T + 7)}, {vr(QD)}, vcc", V(V_T + 7) + V(QD) + [("vcc", 0)], V(QD))
            p.vmem_store(f"buffer_store_dword {vr(V_ND + qb)}, {vr(DO_)}, {sr(RD, 4)}, 0 offen nt", V(V_ND + qb) + V(DO_) + S(RD, 4))
            p.valu(f"v_mul_f32_e32 {vr(LG)}, 0xbfb8aa3b, {vr(V_T + 5 + qb)}", V(V_T + 5 + qb), V(LG))
            p.valu(f"v_sub_f32_e32 {vr(V_T + 7)}, 0, {vr(V_ND + qb)}", V(V_ND + qb), V(V_T + 7))
            p.vmem_store(f"buffer_store_dword {vr(LG)}, {vr(QD)}, {sr(RQD, 4)}, 0 offen nt", V(LG) + V(QD) + S(RQD, 4))
            p.vmem_store(f"buffer_store_dword {vr(V_T + 7)}, {vr(QD)}, {sr(RQD, 4)}, 0 offen offset:128 nt",
                         V(V_T + 7) + V(QD) + S(RQD, 4))

    def finish_rows(self, do_in_acc=False):
        """dO -> AGPRs (unless loaded there), Q -> AGPRs, -LSE*log2e (the exps' offset) and
        -D (dP^T's start values)."""
        p = self.p
        p.waitcnt(vm=0)
        for i in range(0 if do_in_acc else 64):
            p.valu(f"v_accvgpr_write_b32 {ar(A_O + i)}, {vr(64 + i)}", V(64 + i), A(A_O + i))
        for i in range(64):
            p.valu(f"v_accvgpr_write_b32 {ar(A_Q + i)}, {vr(i)}", V(i), A(A_Q + i))
        for qb in range(2):
            c = V_CS + 16 * qb
            p.valu(f"v_mul_f32_e32 {vr(c)}, 0xbfb8aa3b, {vr(V_T + 5 + qb)}", V(V_T + 5 + qb), V(c))
            d = V_CD[qb]
            p.valu(f"v_sub_f32_e32 {vr(d)}, 0, {vr(V_ND + qb)}", V(V_ND + qb), V(d))
            for r in range(1, 16):
                p.valu(f"v_mov_b32_e32 {vr(d + r)}, {vr(d)}", V(d), V(d + r))

    def epilogue(self, base=8):
        """dQ^T * scale of the current item: lane holds row q0 + 32qb + l32, d = db*32 + g4*8 +
        hi*4 + 0..3; through the wave's LDS staging rows, whole 256-byte rows per store.  Its
        VGPR temporaries are base .. base+51."""
        p, s = self.p, self.s
        p.comment("epilogue")
        RQ = S_TMP + 4
        T0, COL, NREC, EPW, ROW4 = S_TMP, S_TMP + 1, S_TMP + 2, S_TMP + 3, S_TMP + 8
        s(f"s_mul_i32 {sr(T0)}, {sr(S_BA)}, {sr(S_SEQ)}", S(S_BA) + S(S_SEQ), S(T0))
        s(f"s_lshl_b32 {sr(COL)}, {sr(S_HA)}, 8", S(S_HA), S(COL))
        self.nrec_rows(NREC, S_SEQ, S_LDB)
        self.rsrc(RQ, S_DQKV, T0, S_LDB, COL, NREC)
        s(f"s_mul_i32 {sr(EPW)}, {sr(S_WAVE)}, {EPI_WAVE}", S(S_WAVE), S(EPW))
        s(f"s_add_u32 {sr(EPW)}, {sr(EPW)}, {LDS_EPI}", S(EPW), S(EPW))
        s(f"s_lshl_b32 {sr(ROW4)}, {sr(S_LDB)}, 2", S(S_LDB), S(ROW4))
        BW, BR, TA, TB, RBUF, OOS = base + 16, base + 17, base + 18, base + 19, base + 20, base + 36
        assert OOS + 16 <= 256 and (base + 52 <= V_RB or base >= V_T + 8)
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
        p.valu(f"v_add_u32_e32 {vr(TA)}, {sr(S_Q0)}, {vr(TA)}", S(S_Q0) + V(TA), V(TA))
        p.valu(f"v_mul_lo_u32 {vr(TA)}, {vr(TA)}, {sr(S_LDB)}", V(TA) + S(S_LDB), V(TA))
        p.valu(f"v_lshl_add_u32 {vr(OOS)}, {vr(TB)}, 4, {vr(TA)}", V(TB) + V(TA), V(OOS))
        for i in range(1, 16):
            p.valu(f"v_add_u32_e32 {vr(OOS + i)}, {sr(ROW4)}, {vr(OOS + i - 1)}", S(ROW4) + V(OOS + i - 1), V(OOS + i))
        W0 = W = base
        for qb in range(2):
            for db in range(4):
                for g4 in range(4):
                    a0 = A_DQ + (db * 2 + qb) * 16 + g4 * 4
                    for j in range(4):
                        p.valu(f"v_accvgpr_read_b32 {vr(W + j)}, {ar(a0 + j)}", A(a0 + j), V(W + j))
                    for j in range(4):
                        p.valu(f"v_mul_f32_e32 {vr(W + j)}, {sr(S_SCALE)}, {vr(W + j)}", V(W + j) + S(S_SCALE), V(W + j))
                    p.valu(f"{self.pack_op} {vr(W + 4)}, {vr(W)}, {vr(W + 1)}", V(W, 2), V(W + 4))
                    p.valu(f"{self.pack_op} {vr(W + 5)}, {vr(W + 2)}, {vr(W + 3)}", V(W + 2, 2), V(W + 5))
                    p.ds_write(f"ds_write_b64 {vr(BW)}, {vr(W + 4, 2)} offset:{(db * 4 + g4) * 16}", V(BW) + V(W + 4, 2))
                    W = W0 if W == W0 + 8 else W0 + 8
            for i in range(8):   # LDS operations of a wave complete in order: reads see the rows
                R = RBUF + 4 * (i % 4)
                p.ds_read(f"ds_read_b128 {vr(R, 4)}, {vr(BR)} offset:{i * 4 * EPI_ROW}", V(R, 4), V(BR))
                p.vmem_store(f"buffer_store_dwordx4 {vr(R, 4)}, {vr(OOS + qb * 8 + i)}, {sr(RQ, 4)}, 0 offen nt",
                             V(R, 4) + V(OOS + qb * 8 + i) + S(RQ, 4))

    def start_item(self, u, sfx):
        """Tile it of the current item (buffer u, score set u % 2): S^T/dP^T when the wave uses
        the tile, the body's variant, first row reads of tile it+1."""
        p, s = self.p, self.s
        self.code()
        s(f"s_bitcmp1_b32 {sr(S_CODE)}, 1", S(S_CODE), [("scc", 0)])     # act(this)
        p.branch(f"s_cbranch_scc0 .Lss_{sfx}", [("scc", 0)], skip_xdl=ACC)
        rissued = 0
        for i in range(32):
            while rissued < 16 and 2 * rissued - LK <= i:
                self.row_read(rissued, u)
                rissued += 1
            self.sdp_mfma(i, u % 2)
        p.label(f".Lss_{sfx}")
        for i in range(LK):
            self.row_read(i, (u + 1) % 4)
        p.branch(f"s_branch .Ldisp{u}", keep_lgkm=True, skip_xdl=ACC)


def build(check_ldb: int = 12288, dt: str = "f16") -> str:
    """The kernel's assembly text: tkm_fa_bwd_dq_d128_f16 (dt "f16") or _bf16."""
    p = Prog(coalesce_lgkm=True)
    sal = p.salu
    b = Body(p, dt)
    p.smem(f"s_load_dwordx16 {sr(8, 16)}, {sr(0, 2)}, 0x0", S(8, 16), S(0, 2))
    p.smem(f"s_load_dwordx16 {sr(24, 16)}, {sr(0, 2)}, 0x40", S(24, 16), S(0, 2))
    p.smem(f"s_load_dwordx2 {sr(S_MAGG, 2)}, {sr(0, 2)}, 0x80", S(S_MAGG, 2), S(0, 2))
    L = Lanes(p, check_ldb)
    L.shr(V_PT + 0, L.k(6), 0)
    p.readlane(f"v_readfirstlane_b32 {sr(S_WAVE)}, {vr(V_PT + 0)}", V(V_PT + 0), S(S_WAVE))
    p.waitcnt(lgkm=0)
    xcd_slot(p, S_WG, S_NWG, S_TMP, S_TMP + 1)
    T3 = S_TMP + 3
    sal(f"s_lshl_b32 {sr(S_LDB32)}, {sr(S_LDB)}, 5", S(S_LDB), S(S_LDB32))
    sal(f"s_lshl_b32 {sr(S_LDSW)}, {sr(S_WAVE)}, 11", S(S_WAVE), S(S_LDSW))
    # ---------------------------------------------------------------- DMA lane offsets
    LANE, L32, HI = V_PT + 1, V_PT + 2, V_PT + 3
    DR, DP, TA, TB, TC = V_PT + 4, V_PT + 5, V_PT + 6, V_PT + 7, V_PT + 8
    lane_basics(L, (LANE, L32, HI))
    L.shr(DR, L.k(4), LANE)
    L.and_(DP, L.k(15), LANE)
    # wave w, instruction i moves rows w*8 + i*4 + dr of a 32-row tile: chunk dp ^ swz(row)
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
    p.valu(f"v_mov_b32_e32 {vr(V_L32)}, {vr(L32)}", V(L32), V(V_L32))
    p.valu(f"v_lshlrev_b32_e32 {vr(V_HI4)}, 2, {vr(HI)}", V(HI), V(V_HI4))
    row_read_offsets(L, V_KOFF, (LANE, L32, HI), (TA, TB, TC))
    tr_read_offsets(L, V_VOFF, (LANE, L32, HI), (TA, TB, TC, V_PT + 9, V_PT + 10, V_PT + 11, V_PT + 12))
    _check_lanes(L, check_ldb)
    # ---------------------------------------------------------------- first item, tiles 0..2
    sal(f"s_mov_b32 {sr(S_KA)}, 0", [], S(S_KA))
    sal(f"s_mov_b32 {sr(S_KD)}, 0", [], S(S_KD))
    b.decode_d("p0")
    for t in range(2):
        b.tile_offset()
        b.dma_all(t)
        b.d_advance(f"p{t + 1}")
    b.item_index(S_KA, S_TMP + 17)
    b.decode_a(S_TMP + 17, "p")
    b.rows_load("p")
    b.tile_offset()
    b.dma_all(2)
    b.d_advance("p3")
    b.zero_acc()
    b.finish_rows()
    p.waitcnt(vm=0)
    p.barrier()
    b.start_item(0, "p")
    for u in range(4):
        _dispatch(b, u)
    for u in range(4):
        _boundary(b, u)
    p.label(".Lexit")
    p.waitcnt(vm=0, lgkm=0)
    p.emit("s_endpgm", BRANCH)
    return kernel_text(f"tkm_fa_bwd_dq_d128_{dt}", p.finalize(), lds_bytes=LDS_BYTES, kernarg_bytes=KERNARG_BYTES,
                       next_free_sgpr=NEXT_FREE_SGPR, args=ARGS, wg_ids=(1, 0, 0))


def _check_lanes(L: Lanes, ldb):
    tid = np.arange(256)
    lane, wave = tid & 63, tid >> 6
    dr, dp = lane // 16, lane % 16
    for i in range(2):
        row = wave * 8 + i * 4 + dr
        chunk = (dp ^ np.vectorize(swz)(row)) << 4
        assert np.array_equal(L.val[V_DOFF + i], (row * ldb + chunk) & 0xFFFFFFFF), f"K/V dma {i}"


def _dispatch(b: Body, u: int):
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
    for lab, sdp, ew, masked in VARIANTS[::-1]:
        p.label(f".L{lab}{u}")
        p.assume_lgkm(pend)
        b.body(u, sdp=sdp, ew=ew, masked=masked)


def _boundary(b: Body, u: int):
    """End of the current item before body residue u: request the next item's rows (their
    latency hides behind the epilogue), store the current dQ; take the next item (or stop),
    its D, and start it on tile it (buffer u, already delivered)."""
    p, s = b.p, b.s
    I = S_TMP + 17
    p.label(f".Lbnd{u}")
    p.nop(16)
    p.waitcnt(lgkm=0)
    K1 = S_TMP + 16
    s(f"s_add_u32 {sr(K1)}, {sr(S_KA)}, 1", S(S_KA), S(K1))
    b.item_index(K1, I)
    s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
    p.branch(f"s_cbranch_scc1 .Lnopf{u}", [("scc", 0)], skip_xdl=ACC)
    p.comment("next rows")
    b.rows_prefetch(I, f"b{u}")
    p.label(f".Lnopf{u}")
    b.epilogue(EPI_BASE)
    s(f"s_add_u32 {sr(S_KA)}, {sr(S_KA)}, 1", S(S_KA), S(S_KA))
    s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lexit", [("scc", 0)], skip_xdl=ACC)
    b.decode_a(I, f"b{u}")
    p.comment("item")
    p.waitcnt(vm=0)
    b.rows_d(True, f"b{u}")
    b.zero_acc()
    b.finish_rows(do_in_acc=True)
    b.start_item(u, f"b{u}")


def main(path: str) -> None:
    with open(path, "w") as f:
        f.write(build())


if __name__ == "__main__":
    import sys
    main(sys.argv[1])

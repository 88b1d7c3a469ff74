"""Generator of the gfx950 assembly FlashAttention forward, D = 128, fp16 (causal or not,
optional kv_len).

Contract: identical to fa_fwd_kernel (tokamak_amd/csrc/attn_fwd.hip), which replaces the
reference's k_gqa_flash_attn_tc_fwd<128> (src/tkm_gpu.cu:302-438): packed
qkv [B][S][(Hq+2Hkv)*128] fp16 in; O [B][S][Hq*128] fp16 and LSE [B][Hq][S] fp32 (natural
log of the scaled scores) out; q-head h reads kv-head h/(Hq/Hkv); key j is visible from
query i iff j < kv_len[b] and (!causal || j <= i).

Work decomposition: persistent, one workgroup (4 waves, one per SIMD) per compute unit walks
items (batch, q-head, block of 256 query rows; block fastest) in snake order over rounds of NWG
items, consecutive items of a round on one XCD (xcd_slot): the query blocks of a head, and the
q-heads of a kv group, read the same K/V tiles through that XCD's L2, and for causal the long
and short blocks of consecutive rounds pair up.  A wave owns 64 query rows: Q (fp16, as loaded) sits in AGPRs as two 32-row blocks, so every K or V operand read from LDS feeds two
MFMAs, and its O^T accumulators sit in AGPRs.  K/V tiles of 64 keys go HBM -> LDS by buffer
DMA into two K and two V buffers (rows past the valid range read as zero), row-major with the
XOR chunk swizzle chunk' = chunk ^ (4*(row&3) + (row>>2&3)).  The DMA stream is a cursor of
its own, two tiles ahead for K and one for V, that runs on across item boundaries: when an
item ends, the next item's first tiles are already in LDS.

Per tile t a wave runs a fixed 64-slot schedule (one v_mfma_f32_32x32x16_f16 per slot):
  slots  0..31   S(t+1) = K(t+1) Q^T into the free score register set;
  slots 32..63   O^T += V(t)^T P(t)^T, V^T read from the row-major tile by ds_read_b64_tr_b16;
the softmax of S(t) runs between the MFMAs of slots 0..56: P = exp2(fma(S, scale*log2(e),
-m)), m in log2 units.  The scores are the unscaled
fp16 products, summed in fp32, and the scale is applied in fp32, as the reference's kernel
does: a scale folded into Q and rounded to fp16 moves a score s by up to |s|*2^-12, which
trained attention logits turn into errors past the bars.  P is packed to fp16 for the MFMA,
and the row sums accumulate in fp32 by v_add_f32.  The eight DMA requests of K(t+2) and V(t+1) go one
every four slots; the scalar bookkeeping (the stream's next tile descriptors, the next
body's variant) is spliced between the MFMAs of slots 32..63, and a body jumps straight into
the next common body.  A wave's last active tile (the only one that can need a mask: causal
diagonal or kv_len edge) runs unpipelined; tiles past it only move data.

The row offset m starts as the row max of the item's first tile and moves only when it has
to (a lazy online softmax): between the MFMAs of slots 17..61 each lane takes the max of its
scores in S(t+1), and if any lane of the wave has a score above m + RESCALE_LOG2 (log2
units) the wave raises m of every row to max(m, row max of S(t+1)) after the body and
multiplies its O accumulators and row sums by 2^(m_old - m_new) (exactly 1 for the rows whose
m stays).  So no P exceeds 2^RESCALE_LOG2 and the fp16 pack cannot overflow, while inputs
whose later keys stay near the first tile's scores never pay for the rescale.  A wave's
masked last tile makes the same check after its mask.  O leaves through per-wave LDS staging
rows so that each store writes whole 256-byte rows.

The generated code's per-lane address arithmetic is evaluated here over all 4 x 64 lanes and
checked against the HIP kernel's index formulas before any text is written.
"""
from __future__ import annotations

import numpy as np

from .attn_dkdv import split_scalar
from .common import Lanes, lane_basics, row_read_offsets, swz, tr_read_offsets, xcd_slot
from .gfx950 import A, BRANCH, PERMLANE, Prog, S, V, ar, kernel_text, sr, vr

NAME = "tkm_fa_fwd_d128_f16"        # the bf16 kernel: tkm_fa_fwd_d128_bf16 (build(dt="bf16"))
D = 128
ROWB = D * 2            # bytes per K/V row in LDS
TILE = 64 * ROWB        # one 64-key tile
LDS_K = (0, TILE)       # K buffers
LDS_V = (2 * TILE, 3 * TILE)
LDS_EPI = 4 * TILE          # per wave: 32 rows of 272 B staging O for the store
EPI_ROW = 272               # 256 B + 16 B pad: rows 16 B apart in the banks
EPI_WAVE = 32 * EPI_ROW
LDS_BYTES = LDS_EPI + 4 * EPI_WAVE
LK = 5                  # slots between a K read and its first MFMA (4 puts the K and V reads
LV = 3                  # on the DMA slots' parity: ~120 cycles more per tile, measured)
NKB = 4                 # K operand registers in rotation (need 2*NKB > LK + 2)
NVB = 4
assert 2 * NKB > LK + 2 and 2 * NVB > LV + 2   # a read reuses its register four reads later
DMA0 = 2                # slot of the first DMA request (then one every four slots)
RESCALE_LOG2 = 15.0     # m moves when a score exceeds it by more than this (P <= 32768)
# slots of the 32 lane-max instructions of S(t+1) (blocks kb = 0 first) and of the test
MAX_SLOTS = tuple(range(17, 33)) + tuple(range(44, 60))
TEST_SLOT = 61
MFMA = "v_mfma_f32_32x32x16_f16"
MFMA_OF = {"f16": MFMA, "bf16": "v_mfma_f32_32x32x16_bf16"}
PACK_OF = {"f16": "v_cvt_pk_f16_f32", "bf16": "v_cvt_pk_bf16_f32"}
# bf16: P goes to the PV MFMAs as two bf16 halves, hi = bf16(P) and lo = bf16(P - hi) (about 16
# significant bits; 8-bit P alone misses the O tolerance on rows with few keys), so every PV
# step is two MFMAs on the same V operand and a body has 96 slots: S(t+1) in 0..31, PV in
# 32..95 (k-step ks at 32 + 16ks), softmax step n at floor(5n/2).  The lo words of P[qb][ks]
# go into the first four registers of the eight scores they come from (step w of the block
# writes register w after steps 0..w-1 have read registers 0..2w-1), which the next S MFMAs
# into that set overwrite only in the next body.

# kernel arguments (byte offsets in the kernarg segment): qkv, out, lse, kv_len, then
# S, Hq, Hkv, sl2, causal, n_qblk, ldb, ldo, group, n_wg, n_items, B*Hq and the reciprocals
# of B*Hq, Hq and group
ARGS = [(0, 8, "ptr"), (8, 8, "ptr"), (16, 8, "ptr"), (24, 8, "ptr")] + \
       [(32 + 4 * i, 4, "val") for i in range(15)]
KERNARG_BYTES = 96

# ---- SGPRs
S_KARG, S_WG = 0, 2
S_QKV, S_OUT, S_LSE, S_KVLEN = 8, 10, 12, 14
S_SEQ, S_HQ, S_HKV, S_SL2, S_CAUSAL, S_NQBLK, S_LDB, S_LDO = 16, 17, 18, 19, 20, 21, 22, 23
S_G, S_NWG, S_NI, S_BHQ, S_MAGNQ, S_MAGHQ, S_MAGG = 24, 25, 26, 27, 28, 29, 30
# the current item
S_KA, S_IT, S_NT, S_ACTEND, S_MASKB, S_Q0, S_KVL, S_BA = 32, 33, 34, 35, 36, 37, 38, 39
S_HA, S_CODE, S_WAVE, S_THR, S_LDSW, S_KVEND, S_KVHA = 40, 41, 42, 43, 44, 45, 46
# the DMA stream: round KD's item, tile TD of the K position, TDP of the V position (one back)
S_KD, S_TD, S_NTD, S_KVEND_D, S_TDP, S_KVEND_DP = 47, 48, 49, 50, 51, 52
S_KB, S_VB, S_VBP = 54, 56, 58      # K / V row-0 addresses of the stream's items (64-bit)
S_RK, S_RV, S_RQ, S_RL = 60, 64, 68, 72
S_TMP = 76                          # s76..s95
S_RSF = 96                          # lanes whose S(t+1) needs a larger m (64-bit mask)
NEXT_FREE_SGPR = 98

# ---- VGPRs
V_SET = (0, 64)         # score register sets; block (kb, qb) at +(kb*2+qb)*16
V_NEGM = 128            # -m of the lane's row in log2 units, per qb
V_MX = 130              # the lane's max unscaled score of the next tile, per qb
V_RT = 132              # rescale temporaries (2)
V_P = 160               # P[qb][ks] at 160 + (qb*4+ks)*4
V_SPL = 134             # bf16: split temporaries (4)
V_KBUF = 192
V_VBUF = V_KBUF + 4 * NKB
V_KOFF = V_VBUF + 4 * NVB   # 8
V_VOFF = V_KOFF + 8         # 8: tt*4 + db
V_DOFF = V_VOFF + 8         # 4
V_LSUM = V_DOFF + 4         # row sums (fp32 P, this lane's half of the keys), per qb
V_LT = V_LSUM + 2           # this tile's partial sums: qb*2 + (0, 1)
V_NINF = V_LT + 4
V_TMP = V_NINF + 1          # 1
V_L32 = V_TMP + 1           # lane & 31
V_HI4 = V_TMP + 2           # 4 * (lane >> 5)
assert V_HI4 < 256
V_PT = 64                   # prologue scratch (score set 1, free until the first S(1))
V_T = V_P + 4               # temporaries of the item boundary, when P is free (5)

# ---- AGPRs
A_O = 0                 # o[db][qb] at (db*2+qb)*16
A_Q = 128               # q[qb][ks] at 128 + (qb*8+ks)*4
A_QN = 192              # the next item's Q as loaded (same order)
ACC = set(A(A_O, 128))

# body variants by code: 4*act(t+1) + 2*act(t) + mask(t); 8 = the item's end
VARIANTS = [("full", 6), ("last", 2), ("lastm", 3), ("idle", 0)]


def sblk(J, kb, qb):
    return V_SET[J] + (kb * 2 + qb) * 16


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

    # ---------------------------------------------------------------- scalar helpers
    def add64(self, dst, src, rows, stride, extra, lo, hi):
        """s[dst:dst+1] = s[src:src+1] + rows*stride (+ extra)."""
        s = self.s
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

    def rsrc_tile(self, dst, base, t, kvend, tmp):
        """dst[0:3] = descriptor of 64-key tile t (SGPR) of the rows at base (64-bit SGPR
        pair): rows clamp(kvend - 64t, 0, 64) of ldb bytes, up to the last row's head."""
        s = self.s
        k0, rows, lo, hi = tmp, tmp + 1, tmp + 2, tmp + 3
        s(f"s_lshl_b32 {sr(k0)}, {sr(t)}, 6", S(t), S(k0))
        s(f"s_sub_i32 {sr(rows)}, {sr(kvend)}, {sr(k0)}", S(kvend) + S(k0), S(rows))
        s(f"s_min_i32 {sr(rows)}, {sr(rows)}, 64", S(rows), S(rows))
        s(f"s_max_i32 {sr(rows)}, {sr(rows)}, 0", S(rows), S(rows))
        self.nrec_rows(dst + 2, rows, S_LDB)
        s(f"s_mul_i32 {sr(lo)}, {sr(k0)}, {sr(S_LDB)}", S(k0) + S(S_LDB), S(lo))
        s(f"s_mul_hi_u32 {sr(hi)}, {sr(k0)}, {sr(S_LDB)}", S(k0) + S(S_LDB), S(hi))
        s(f"s_add_u32 {sr(dst)}, {sr(base)}, {sr(lo)}", S(base) + S(lo), S(dst) + [("scc", 0)])
        s(f"s_addc_u32 {sr(dst + 1)}, {sr(base + 1)}, {sr(hi)}", S(base + 1) + S(hi) + [("scc", 0)], S(dst + 1))
        s(f"s_and_b32 {sr(dst + 1)}, {sr(dst + 1)}, 0xffff", S(dst + 1), S(dst + 1))
        s(f"s_mov_b32 {sr(dst + 3)}, 0x20000", [], S(dst + 3))

    def item_index(self, k_sgpr, dst, tmp):
        """dst = item of round k: k*NWG + (k odd ? NWG-1-v : v), v the workgroup's place."""
        s = self.s
        s(f"s_mul_i32 {sr(dst)}, {sr(k_sgpr)}, {sr(S_NWG)}", S(k_sgpr) + S(S_NWG), S(dst))
        s(f"s_sub_u32 {sr(tmp)}, {sr(S_NWG)}, 1", S(S_NWG), S(tmp))
        s(f"s_sub_u32 {sr(tmp)}, {sr(tmp)}, {sr(S_WG)}", S(tmp) + S(S_WG), S(tmp))
        s(f"s_bitcmp1_b32 {sr(k_sgpr)}, 0", S(k_sgpr), [("scc", 0)])
        s(f"s_cselect_b32 {sr(tmp)}, {sr(tmp)}, {sr(S_WG)}", S(tmp) + S(S_WG) + [("scc", 0)], S(tmp))
        s(f"s_add_u32 {sr(dst)}, {sr(dst)}, {sr(tmp)}", S(dst) + S(tmp), S(dst))

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

    def decode(self, i, z, b, h, kvh, r):
        """item i -> (b, h, kv head, query block z): z fastest."""
        self.divide(i, S_NQBLK, S_MAGNQ, r, z)
        self.divide(r, S_HQ, S_MAGHQ, b, h)
        self.divide(h, S_G, S_MAGG, kvh, None)

    def kvl_of(self, b, dst, label, tmp):
        """dst = clamp(kv_len[b], 0, S), or S without kv_len.  No LDS read may be in flight."""
        p, s = self.p, self.s
        s(f"s_mov_b32 {sr(dst)}, {sr(S_SEQ)}", S(S_SEQ), S(dst))
        s(f"s_cmp_eq_u64 {sr(S_KVLEN, 2)}, 0", S(S_KVLEN, 2), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 {label}", [("scc", 0)], skip_xdl=ACC)
        s(f"s_lshl_b32 {sr(tmp)}, {sr(b)}, 2", S(b), S(tmp))
        p.smem(f"s_load_dword {sr(dst)}, {sr(S_KVLEN, 2)}, {sr(tmp)}", S(dst), S(S_KVLEN, 2) + S(tmp))
        p.waitcnt(lgkm=0)
        s(f"s_max_i32 {sr(dst)}, {sr(dst)}, 0", S(dst), S(dst))
        s(f"s_min_i32 {sr(dst)}, {sr(dst)}, {sr(S_SEQ)}", S(dst) + S(S_SEQ), S(dst))
        p.label(label)

    def tiles_of(self, z, kvl, qblk, kvend, nt, tmp):
        """qblk = causal ? n_qblk-1-z : z; kvend = causal ? min(kvl, 256 qblk + 256) : kvl;
        nt = max(1, ceil(kvend/64)) (an item without keys keeps one tile no wave uses)."""
        s = self.s
        s(f"s_sub_u32 {sr(qblk)}, {sr(S_NQBLK)}, 1", S(S_NQBLK), S(qblk))
        s(f"s_sub_u32 {sr(qblk)}, {sr(qblk)}, {sr(z)}", S(qblk) + S(z), S(qblk))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(qblk)}, {sr(z)}, {sr(qblk)}", S(z) + S(qblk) + [("scc", 0)], S(qblk))
        s(f"s_lshl_b32 {sr(tmp)}, {sr(qblk)}, 8", S(qblk), S(tmp))
        s(f"s_add_u32 {sr(tmp)}, {sr(tmp)}, 0x100", S(tmp), S(tmp))
        s(f"s_min_u32 {sr(tmp)}, {sr(tmp)}, {sr(kvl)}", S(tmp) + S(kvl), S(tmp))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(kvend)}, {sr(kvl)}, {sr(tmp)}", S(kvl) + S(tmp) + [("scc", 0)], S(kvend))
        s(f"s_add_u32 {sr(tmp)}, {sr(kvend)}, 63", S(kvend), S(tmp))
        s(f"s_lshr_b32 {sr(nt)}, {sr(tmp)}, 6", S(tmp), S(nt))
        s(f"s_max_u32 {sr(nt)}, {sr(nt)}, 1", S(nt), S(nt))

    # ---------------------------------------------------------------- the DMA stream
    def decode_d(self, sfx):
        """Stream item of round KD -> K, V row-0 addresses, kvend, tile count; tile 0.  Past
        the last item the stream reads nothing (kvend 0: descriptors of zero bytes)."""
        p, s = self.p, self.s
        I, Z, B, H, KVH, KVL, QB, R = (S_TMP + k for k in range(8))
        T0, COL, LO, HI = S_TMP + 8, S_TMP + 9, S_TMP + 10, S_TMP + 11
        self.item_index(S_KD, I, T0)
        s(f"s_mov_b32 {sr(S_TD)}, 0", [], S(S_TD))
        s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
        p.branch(f"s_cbranch_scc0 .Ldd_{sfx}", [("scc", 0)], skip_xdl=ACC)
        s(f"s_mov_b32 {sr(S_NTD)}, 0x7fffffff", [], S(S_NTD))
        s(f"s_mov_b32 {sr(S_KVEND_D)}, 0", [], S(S_KVEND_D))
        s(f"s_mov_b64 {sr(S_KB, 2)}, {sr(S_QKV, 2)}", S(S_QKV, 2), S(S_KB, 2))
        s(f"s_mov_b64 {sr(S_VB, 2)}, {sr(S_QKV, 2)}", S(S_QKV, 2), S(S_VB, 2))
        p.branch(f"s_branch .Lde_{sfx}", skip_xdl=ACC)
        p.label(f".Ldd_{sfx}")
        self.decode(I, Z, B, H, KVH, R)
        self.kvl_of(B, KVL, f".Ldk_{sfx}", T0)
        self.tiles_of(Z, KVL, QB, S_KVEND_D, S_NTD, T0)
        s(f"s_mul_i32 {sr(T0)}, {sr(B)}, {sr(S_SEQ)}", S(B) + S(S_SEQ), S(T0))
        s(f"s_add_u32 {sr(COL)}, {sr(S_HQ)}, {sr(KVH)}", S(S_HQ) + S(KVH), S(COL))
        s(f"s_lshl_b32 {sr(COL)}, {sr(COL)}, 8", S(COL), S(COL))
        self.add64(S_KB, S_QKV, T0, S_LDB, COL, LO, HI)
        s(f"s_lshl_b32 {sr(T0)}, {sr(S_HKV)}, 8", S(S_HKV), S(T0))
        s(f"s_add_u32 {sr(S_VB)}, {sr(S_KB)}, {sr(T0)}", S(S_KB) + S(T0), S(S_VB) + [("scc", 0)])
        s(f"s_addc_u32 {sr(S_VB + 1)}, {sr(S_KB + 1)}, 0", S(S_KB + 1) + [("scc", 0)], S(S_VB + 1))
        p.label(f".Lde_{sfx}")

    def d_shift(self):
        """Stream one position on: the K position's tile becomes the V position's."""
        s = self.s
        s(f"s_mov_b32 {sr(S_TDP)}, {sr(S_TD)}", S(S_TD), S(S_TDP))
        s(f"s_mov_b64 {sr(S_VBP, 2)}, {sr(S_VB, 2)}", S(S_VB, 2), S(S_VBP, 2))
        s(f"s_mov_b32 {sr(S_KVEND_DP)}, {sr(S_KVEND_D)}", S(S_KVEND_D), S(S_KVEND_DP))
        s(f"s_add_u32 {sr(S_TD)}, {sr(S_TD)}, 1", S(S_TD), S(S_TD))

    def d_step(self, sfx):
        """d_shift, then the next item's tile 0 when the stream's item is done (outside the
        loop bodies)."""
        p, s = self.p, self.s
        self.d_shift()
        s(f"s_cmp_lt_u32 {sr(S_TD)}, {sr(S_NTD)}", S(S_TD) + S(S_NTD), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lds_{sfx}", [("scc", 0)], skip_xdl=ACC)
        s(f"s_add_u32 {sr(S_KD)}, {sr(S_KD)}, 1", S(S_KD), S(S_KD))
        self.decode_d(sfx)
        p.label(f".Lds_{sfx}")

    def rsrc_k(self, tmp):
        self.rsrc_tile(S_RK, S_KB, S_TD, S_KVEND_D, tmp)

    def rsrc_v(self, tmp):
        self.rsrc_tile(S_RV, S_VBP, S_TDP, S_KVEND_DP, tmp)

    def stream_start(self, u, sfx):
        """With the stream at an item's tile 0: K(0) -> K buffer u, K(1) -> K buffer u^1,
        V(0) -> V buffer u; then the descriptors of the first body's requests."""
        T = S_TMP + 12
        self.rsrc_k(T)
        self.dma_tile(S_RK, LDS_K[u])
        self.d_step(f"{sfx}a")
        self.rsrc_k(T)
        self.dma_tile(S_RK, LDS_K[u ^ 1])
        self.rsrc_v(T)
        self.dma_tile(S_RV, LDS_V[u])
        self.d_step(f"{sfx}b")
        self.rsrc_k(T)
        self.rsrc_v(T)

    def dma_m0(self, lds_base, i):
        self.s(f"s_add_u32 m0, {sr(S_LDSW)}, {lds_base + i * 1024}", S(S_LDSW), [("m0", 0)])

    def dma_ld(self, rs, i):
        self.p.dma(f"buffer_load_dwordx4 {vr(V_DOFF + i)}, {sr(rs, 4)}, 0 offen lds",
                   V(V_DOFF + i) + S(rs, 4))

    def dma_tile(self, rs, lds_base):
        for i in range(4):
            self.dma_m0(lds_base, i)
            self.dma_ld(rs, i)

    # ---------------------------------------------------------------- the current item
    def decode_a(self, i, sfx):
        """Current item i: rows, keys, tiles, per-wave activity and mask bounds."""
        s = self.s
        R, Z, QB, T0, T1 = S_TMP + 14, S_TMP + 16, S_TMP + 17, S_TMP + 18, S_TMP + 19
        assert i not in (R, Z, QB, T0, T1)
        self.decode(i, Z, S_BA, S_HA, S_KVHA, R)
        self.kvl_of(S_BA, S_KVL, f".Lak_{sfx}", T0)
        self.tiles_of(Z, S_KVL, QB, S_KVEND, S_NT, T0)
        s(f"s_lshl_b32 {sr(S_Q0)}, {sr(QB)}, 8", S(QB), S(S_Q0))
        s(f"s_lshl_b32 {sr(T0)}, {sr(S_WAVE)}, 6", S(S_WAVE), S(T0))
        s(f"s_add_u32 {sr(S_Q0)}, {sr(S_Q0)}, {sr(T0)}", S(S_Q0) + S(T0), S(S_Q0))
        # active tiles: t < ACTEND = causal ? min(NT, q0/64 + 1) : NT; none without keys
        s(f"s_lshr_b32 {sr(T0)}, {sr(S_Q0)}, 6", S(S_Q0), S(T0))
        s(f"s_add_u32 {sr(T0)}, {sr(T0)}, 1", S(T0), S(T0))
        s(f"s_min_u32 {sr(T0)}, {sr(T0)}, {sr(S_NT)}", S(T0) + S(S_NT), S(T0))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_ACTEND)}, {sr(S_NT)}, {sr(T0)}", S(S_NT) + S(T0) + [("scc", 0)], S(S_ACTEND))
        s(f"s_cmp_eq_u32 {sr(S_KVL)}, 0", S(S_KVL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_ACTEND)}, 0, {sr(S_ACTEND)}", S(S_ACTEND) + [("scc", 0)], S(S_ACTEND))
        # tiles needing a mask: t >= MASKB = min(kvl/64, causal ? q0/64 : NT)
        s(f"s_lshr_b32 {sr(T0)}, {sr(S_KVL)}, 6", S(S_KVL), S(T0))
        s(f"s_lshr_b32 {sr(T1)}, {sr(S_Q0)}, 6", S(S_Q0), S(T1))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T1)}, {sr(S_NT)}, {sr(T1)}", S(S_NT) + S(T1) + [("scc", 0)], S(T1))
        s(f"s_min_u32 {sr(S_MASKB)}, {sr(T0)}, {sr(T1)}", S(T0) + S(T1), S(S_MASKB))
        s(f"s_mov_b32 {sr(S_IT)}, 0", [], S(S_IT))

    def code(self, t0, t1, t2):
        """S_CODE for body S_IT: 8 at the item's end, else 4*act(t+1) + 2*act(t) + mask(t)
        (act(t+1) implies act(t) and no mask: a masked tile is a wave's last active one)."""
        s = self.s
        s(f"s_cmp_lt_u32 {sr(S_IT)}, {sr(S_ACTEND)}", S(S_IT) + S(S_ACTEND), [("scc", 0)])
        s(f"s_cselect_b32 {sr(t0)}, 2, 0", [("scc", 0)], S(t0))
        s(f"s_add_u32 {sr(t2)}, {sr(S_IT)}, 1", S(S_IT), S(t2))
        s(f"s_cmp_lt_u32 {sr(t2)}, {sr(S_ACTEND)}", S(t2) + S(S_ACTEND), [("scc", 0)])
        s(f"s_cselect_b32 {sr(t1)}, 4, 0", [("scc", 0)], S(t1))
        s(f"s_cmp_ge_u32 {sr(S_IT)}, {sr(S_MASKB)}", S(S_IT) + S(S_MASKB), [("scc", 0)])
        s(f"s_cselect_b32 {sr(t2)}, 1, 0", [("scc", 0)], S(t2))
        s(f"s_or_b32 {sr(t0)}, {sr(t0)}, {sr(t1)}", S(t0) + S(t1), S(t0))
        s(f"s_or_b32 {sr(S_CODE)}, {sr(t0)}, {sr(t2)}", S(t0) + S(t2), S(S_CODE))
        s(f"s_cmp_ge_u32 {sr(S_IT)}, {sr(S_NT)}", S(S_IT) + S(S_NT), [("scc", 0)])
        s(f"s_cselect_b32 {sr(S_CODE)}, 8, {sr(S_CODE)}", S(S_CODE) + [("scc", 0)], S(S_CODE))

    def body_scalar(self):
        """The body's scalar work: the stream one position on with the next body's request
        descriptors, the tile counter, the next body's code (+16: the stream's item is done)."""
        s = self.s
        self.d_shift()
        self.rsrc_v(S_TMP)
        self.rsrc_k(S_TMP + 4)
        s(f"s_add_u32 {sr(S_IT)}, {sr(S_IT)}, 1", S(S_IT), S(S_IT))
        self.code(S_TMP + 8, S_TMP + 9, S_TMP + 10)
        T = S_TMP + 11
        s(f"s_cmp_ge_u32 {sr(S_TD)}, {sr(S_NTD)}", S(S_TD) + S(S_NTD), [("scc", 0)])
        s(f"s_cselect_b32 {sr(T)}, 16, 0", [("scc", 0)], S(T))
        s(f"s_or_b32 {sr(S_CODE)}, {sr(S_CODE)}, {sr(T)}", S(S_CODE) + S(T), S(S_CODE))

    # ---------------------------------------------------------------- LDS operand reads
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

    # ---------------------------------------------------------------- MFMAs
    def s_mfma(self, i, J, qbase=A_Q):
        """S MFMA i of set J (unscaled scores, from 0): ri = i//2, qb = i%2, kb = ri//8,
        ks = ri%8; Q from the AGPRs at qbase."""
        ri, qb = i // 2, i % 2
        kb, ks = ri // 8, ri % 8
        dst = sblk(J, kb, qb)
        c = None if ks == 0 else dst
        self.p.mfma(self.mfma_op, dst, V_KBUF + (ri % NKB) * 4, qbase + (qb * 8 + ks) * 4, c, b_acc=True)

    def pv_per_read(self):
        """PV MFMAs per V operand read: one per block of 32 rows, twice with the bf16 split."""
        return 4 if self.split else 2

    def pv_mfma(self, j, J):
        """PV MFMA j of set J's tile: V read vi = j // pv_per_read(), rows qb = j % 2; bf16:
        hi (P) for j % 4 < 2, then lo (the residual, in set J's score registers), so that the
        two MFMAs into one accumulator have another between them."""
        n = self.pv_per_read()
        vi, qb, lo = j // n, j % 2, (j % n) >= 2
        ks, db = vi // 4, vi % 4
        o = A_O + (db * 2 + qb) * 16
        b = sblk(J, ks // 2, qb) + (ks % 2) * 8 if lo else V_P + (qb * 4 + ks) * 4
        self.p.mfma(self.mfma_op, o, V_VBUF + (vi % NVB) * 4, b, o, dst_acc=True)

    # ---- softmax steps (n = 0..31), k-step major: step n covers P[qb][ks] word w with
    #      ks = n // 8, qb = (n % 8) // 4, w = n % 4, i.e. scores r0 + 2w, r0 + 2w + 1 of block
    #      (kb = ks // 2, qb), r0 = 8 (ks % 2).  The exp half writes exp2 in place; the pack
    #      half packs the pair to fp16 (the MFMA operand) and adds both fp32 values to this
    #      tile's partial sums of the row (two accumulators per block of 32 rows), as the
    #      reference sums the fp32 P (tkm_gpu.cu:403).  (A v_dot2_f32_f16 of each packed pair
    #      with (1, 1) instead of the two adds measured 4 us slower per forward.)
    @staticmethod
    def sm_regs(J, n):
        ks, qb, w = n // 8, (n % 8) // 4, n % 4
        kb, r0 = ks // 2, (ks % 2) * 8
        x0 = sblk(J, kb, qb) + r0 + 2 * w
        return x0, qb, ks, w

    def sm_exp(self, J, n):
        x0, qb, _, _ = self.sm_regs(J, n)
        for x in (x0, x0 + 1):
            self.p.valu(f"v_fma_f32 {vr(x)}, {vr(x)}, {sr(S_SL2)}, {vr(V_NEGM + qb)}",
                        V(x) + S(S_SL2) + V(V_NEGM + qb), V(x))
        for x in (x0, x0 + 1):
            self.p.trans(f"v_exp_f32_e32 {vr(x)}, {vr(x)}", V(x), V(x))

    def sm_pack(self, J, n):
        x0, qb, ks, w = self.sm_regs(J, n)
        pw = V_P + (qb * 4 + ks) * 4 + w
        p = self.p
        p.valu(f"{self.pack_op} {vr(pw)}, {vr(x0)}, {vr(x0 + 1)}", V(x0, 2), V(pw))
        for i in range(2):
            lt = V_LT + qb * 2 + i
            if ks == 0 and w == 0:   # first step of this block of rows in the tile
                p.valu(f"v_mov_b32_e32 {vr(lt)}, {vr(x0 + i)}", V(x0 + i), V(lt))
            else:
                p.valu(f"v_add_f32_e32 {vr(lt)}, {vr(lt)}, {vr(x0 + i)}", V(lt) + V(x0 + i), V(lt))
        if self.split:
            # lo = bf16(P - hi): hi's halves as fp32 are its words shifted up / masked
            t0, t1 = V_SPL + 2 * (n % 2), V_SPL + 2 * (n % 2) + 1
            pl = x0 - w          # register w of this block of eight scores
            p.valu(f"v_lshlrev_b32_e32 {vr(t0)}, 16, {vr(pw)}", V(pw), V(t0))
            p.valu(f"v_and_b32_e32 {vr(t1)}, 0xffff0000, {vr(pw)}", V(pw), V(t1))
            p.valu(f"v_sub_f32_e32 {vr(x0)}, {vr(x0)}, {vr(t0)}", V(x0) + V(t0), V(x0))
            p.valu(f"v_sub_f32_e32 {vr(x0 + 1)}, {vr(x0 + 1)}, {vr(t1)}", V(x0 + 1) + V(t1), V(x0 + 1))
            p.valu(f"v_cvt_pk_bf16_f32 {vr(pl)}, {vr(x0)}, {vr(x0 + 1)}", V(x0, 2), V(pl))

    def sm_finish(self, qb):
        """Tile done: row sum += partial sum."""
        lt = V_LT + qb * 2
        self.p.valu(f"v_add_f32_e32 {vr(lt)}, {vr(lt)}, {vr(lt + 1)}", V(lt, 2), V(lt))
        self.p.valu(f"v_add_f32_e32 {vr(V_LSUM + qb)}, {vr(V_LSUM + qb)}, {vr(lt)}", V(V_LSUM + qb) + V(lt), V(V_LSUM + qb))

    # ---- the lazy rescale: lane max of a score set, the test against m, the rescale
    @staticmethod
    def lane_max_steps(J):
        """The 32 instructions that leave in V_MX + qb the lane's max of set J's scores of
        block qb: per (qb, kb) block of 16 registers, 8 steps (v_max3 over two or three)."""
        steps = []
        for qb, kb in ((0, 0), (1, 0), (0, 1), (1, 1)):
            base, mx = sblk(J, kb, qb), V_MX + qb
            if kb == 0:
                steps.append(("v_max3_f32", mx, (base, base + 1, base + 2)))
                for k in range(1, 7):
                    steps.append(("v_max3_f32", mx, (mx, base + 2 * k + 1, base + 2 * k + 2)))
                steps.append(("v_max_f32_e32", mx, (mx, base + 15)))
            else:
                for k in range(8):
                    steps.append(("v_max3_f32", mx, (mx, base + 2 * k, base + 2 * k + 1)))
        return steps

    def lane_max_step(self, step):
        op, dst, srcs = step
        regs = []
        for r in srcs:
            regs += V(r)
        self.p.valu(f"{op} {vr(dst)}, " + ", ".join(vr(r) for r in srcs), regs, V(dst))

    def rescale_test(self):
        """S_RSF = lanes where fma(lane max, scale log2 e, -m) > RESCALE_LOG2 for either
        block of rows."""
        p = self.p
        for qb in range(2):
            p.valu(f"v_fma_f32 {vr(V_RT + qb)}, {vr(V_MX + qb)}, {sr(S_SL2)}, {vr(V_NEGM + qb)}",
                   V(V_MX + qb) + S(S_SL2) + V(V_NEGM + qb), V(V_RT + qb))
        p.valu(f"v_max_f32_e32 {vr(V_RT)}, {vr(V_RT)}, {vr(V_RT + 1)}", V(V_RT, 2), V(V_RT))
        p.valu(f"v_cmp_lt_f32_e64 {sr(S_RSF, 2)}, {sr(S_THR)}, {vr(V_RT)}", S(S_THR) + V(V_RT), S(S_RSF, 2))

    def rescale_if(self, label):
        """When S_RSF has a lane: m of every row = max(m, the row max of the tested set)
        (both lane halves), O accumulators and row sums times 2^(m_old - m_new)."""
        p, s = self.p, self.s
        s(f"s_cmp_lg_u64 {sr(S_RSF, 2)}, 0", S(S_RSF, 2), [("scc", 0)])
        p.branch(f"s_cbranch_scc0 {label}", [("scc", 0)], skip_xdl=ACC)
        p.nop(16)      # the O accumulators' last MFMAs, on every path here
        W = V_P        # the P registers are free between bodies
        for qb in range(2):
            mx, nm, al = V_MX + qb, V_RT, V_RT + 1
            p.valu(f"v_mov_b32_e32 {vr(nm)}, {vr(mx)}", V(mx), V(nm))
            p.emit(f"v_permlane32_swap_b32_e32 {vr(nm)}, {vr(mx)}", PERMLANE, V(nm) + V(mx), V(nm) + V(mx))
            p.valu(f"v_max_f32_e32 {vr(mx)}, {vr(mx)}, {vr(nm)}", V(mx) + V(nm), V(mx))
            p.valu(f"v_mul_f32_e64 {vr(nm)}, -{sr(S_SL2)}, {vr(mx)}", S(S_SL2) + V(mx), V(nm))
            p.valu(f"v_min_f32_e32 {vr(nm)}, {vr(nm)}, {vr(V_NEGM + qb)}", V(nm) + V(V_NEGM + qb), V(nm))
            p.valu(f"v_sub_f32_e32 {vr(al)}, {vr(nm)}, {vr(V_NEGM + qb)}", V(nm) + V(V_NEGM + qb), V(al))
            p.trans(f"v_exp_f32_e32 {vr(al)}, {vr(al)}", V(al), V(al))
            p.valu(f"v_mov_b32_e32 {vr(V_NEGM + qb)}, {vr(nm)}", V(nm), V(V_NEGM + qb))
            p.valu(f"v_mul_f32_e32 {vr(V_LSUM + qb)}, {vr(V_LSUM + qb)}, {vr(al)}", V(V_LSUM + qb) + V(al), V(V_LSUM + qb))
            for db in range(4):
                o = A_O + (db * 2 + qb) * 16
                for j0 in (0, 8):
                    for j in range(8):
                        p.valu(f"v_accvgpr_read_b32 {vr(W + j)}, {ar(o + j0 + j)}", A(o + j0 + j), V(W + j))
                    for j in range(8):
                        p.valu(f"v_mul_f32_e32 {vr(W + j)}, {vr(W + j)}, {vr(al)}", V(W + j) + V(al), V(W + j))
                    for j in range(8):
                        p.valu(f"v_accvgpr_write_b32 {ar(o + j0 + j)}, {vr(W + j)}", V(W + j), A(o + j0 + j))
                    W = V_P if W == V_P + 8 else V_P + 8
        p.label(label)

    # ---- whole stages (unpipelined)
    def stage_s(self, J, kbase):
        """S(J) = K Q^T from the K buffer at kbase; reads run LK slots ahead."""
        reads_issued = 0
        for i in range(32):
            while reads_issued < 16 and reads_issued * 2 - LK <= i:
                self.k_read(reads_issued, kbase)
                reads_issued += 1
            self.s_mfma(i, J)

    def stage_s_next(self, J, kbase):
        """S(J) = K Q^T of a new item from the next item's Q AGPRs, where its loads put it,
        while those words are copied into the Q AGPRs for the item's bodies: two copies after
        every MFMA, beside the MFMAs."""
        reads_issued = 0
        copied = 0
        for i in range(32):
            while reads_issued < 16 and reads_issued * 2 - LK <= i:
                self.k_read(reads_issued, kbase)
                reads_issued += 1
            self.s_mfma(i, J, A_QN)
            for _ in range(2):
                self.p.valu(f"v_accvgpr_mov_b32 {ar(A_Q + copied)}, {ar(A_QN + copied)}", A(A_QN + copied),
                            A(A_Q + copied))
                copied += 1

    def copy_next_q(self):
        """The next item's Q into the Q AGPRs (a wave that uses no tile of the item)."""
        for w in range(64):
            self.p.valu(f"v_accvgpr_mov_b32 {ar(A_Q + w)}, {ar(A_QN + w)}", A(A_QN + w), A(A_Q + w))

    def stage_softmax_pv(self, J, vbase):
        """Softmax of set J and O += V P from the V buffer at vbase, interleaved: PV k-step ks
        (MFMAs 8ks .. 8ks+7) needs only P[*][ks] (softmax steps 8ks .. 8ks+7), so the softmax
        of k-step ks+1 runs between the MFMAs of k-step ks."""
        for n in range(8):
            self.sm_exp(J, n)
            self.sm_pack(J, n)
        issued = 0
        per = self.pv_per_read()
        fin = (25, 27) if per == 2 else (49, 51)
        for j in range(16 * per):
            while issued < 16 and issued * per - LV <= j:
                self.v_read(issued, vbase)
                issued += 1
            self.pv_mfma(j, J)
            if j % (per // 2) == 0:
                n = 8 + j // (per // 2)   # softmax step of the next k-step, one per PV k-pair
                if n < 32:
                    self.sm_exp(J, n)
                    self.sm_pack(J, n)
            if j in fin:
                self.sm_finish(fin.index(j))

    def stage_mask(self, J, tsg):
        """Scores of set J, tile t (SGPR tsg), set to -inf where key > q (causal) or
        key >= kv_len.  Per lane and 32-row block: thr = min(causal ? q - k0 - 4hi : big,
        kvl - 1 - k0 - 4hi); element key offset c = kb*32 + (r>>2)*8 + (r&3) is masked
        iff c > thr."""
        p, s = self.p, self.s
        t0, t1, t2 = S_TMP + 12, S_TMP + 13, S_TMP + 14
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
            p.valu(f"v_add_u32 {vr(TH)}, {sr(t2)}, {vr(V_L32)}", S(t2) + V(V_L32), V(TH))
            p.valu(f"v_min_i32 {vr(TH)}, {vr(TH)}, {sr(t1)}", V(TH) + S(t1), V(TH))
            p.valu(f"v_sub_u32 {vr(TH)}, {vr(TH)}, {vr(V_HI4)}", V(TH) + V(V_HI4), V(TH))
            for kb in range(2):
                base = sblk(J, kb, qb)
                for r in range(16):
                    c = kb * 32 + (r >> 2) * 8 + (r & 3)
                    p.valu(f"v_cmp_gt_i32_e32 vcc, {c}, {vr(TH)}", V(TH), [("vcc", 0)])
                    p.valu(f"v_cndmask_b32_e32 {vr(base + r)}, {vr(base + r)}, {vr(V_NINF)}, vcc",
                           V(base + r) + V(V_NINF) + [("vcc", 0)], V(base + r))

    def row_max_set_m(self, J):
        """m = row max of set J (unscaled; 0 if -inf): -m in log2 units for the exps."""
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
            self.set_negm(qb, mx)

    def set_negm(self, qb, mx):
        """-m in log2 units for the unscaled row max mx."""
        self.p.valu(f"v_mul_f32_e64 {vr(V_NEGM + qb)}, -{sr(S_SL2)}, {vr(mx)}", S(S_SL2) + V(mx),
                    V(V_NEGM + qb))

    # ---------------------------------------------------------------- loop bodies
    def tile_pipe(self, J, h):
        """Tile t with set J (= the parity of the stream position of tile t): S(t+1) into set
        J^1 from K buffer J^1, softmax of set J, O += V(t) P from V buffer J; requests of
        K(t+2) -> K buffer J and V(t+1) -> V buffer J^1 (the descriptors the previous body
        computed).  Slots 0..31 run the S MFMAs, 32..63 the PV MFMAs (k-step major, so
        PV(ks) starts at slot 32 + 8ks).  Softmax step n has its exp half at slot
        e(n) = floor(7n/4) and its pack half one slot later (P[*][ks] is complete at slot
        e(8ks+7) + 1 <= 32 + 8ks); the DMA instructions go one every four slots from slot 2
        so the vector memory path never backs up into the issue of the MFMA stream; the
        scalar chunks h[0..31] go between the MFMAs of slots 32..63.  The lane max of S(t+1)
        takes one instruction in each of the slots MAX_SLOTS (each block of rows after its
        last MFMA: blocks kb = 0 end at slots 14/15, kb = 1 at 30/31), and the rescale test
        follows at TEST_SLOT."""
        Jn = J ^ 1
        kbase, vbase = LDS_K[Jn], LDS_V[J]
        per = self.pv_per_read()
        nslot = 32 + 16 * per
        max_at = dict(zip(MAX_SLOTS, self.lane_max_steps(Jn)))
        assert len(max_at) == 32 and max(MAX_SLOTS) < TEST_SLOT < 64
        assert min(k for k, st in max_at.items() if st[2][-1] >= sblk(Jn, 1, 0)) >= 33
        assert min(max_at) >= 17
        if per == 2:
            exp_at = {(7 * n) // 4: n for n in range(32)}
            fin_at = (57, 59)
        else:
            exp_at = {(5 * n) // 2: n for n in range(32)}
            fin_at = (81, 83)
        pack_at = {e + 1: n for e, n in exp_at.items()}
        # P[*][ks] (softmax steps 8ks .. 8ks+7) is packed before PV k-step ks, at slot 32 + 8*per*ks
        assert all(max(e + 1 for e, n in exp_at.items() if n // 8 == ks) < 32 + 8 * per * ks for ks in range(4))
        dma_at = {DMA0 + 4 * i: i for i in range(8)}
        kissued = 0
        while kissued * 2 - LK < 0:
            self.k_read(kissued, kbase)
            kissued += 1
        vissued = 0
        for s_ in range(nslot):
            while kissued < 16 and kissued * 2 - LK <= s_:
                self.k_read(kissued, kbase)
                kissued += 1
            while vissued < 16 and 32 + vissued * per - LV <= s_:
                self.v_read(vissued, vbase)
                vissued += 1
            if s_ in dma_at:
                i = dma_at[s_]
                self.dma_m0(LDS_K[J] if i < 4 else LDS_V[Jn], i % 4)
            if s_ < 32:
                self.s_mfma(s_, Jn)
            else:
                self.pv_mfma(s_ - 32, J)
                if s_ - 32 < len(h):
                    self.p.ins.extend(h[s_ - 32])
            if s_ in exp_at:
                self.sm_exp(J, exp_at[s_])
            if s_ in pack_at:
                self.sm_pack(J, pack_at[s_])
            if s_ in fin_at:
                self.sm_finish(fin_at.index(s_))
            if s_ in max_at:
                self.lane_max_step(max_at[s_])
            if s_ == TEST_SLOT:
                self.rescale_test()
            if s_ in dma_at:
                i = dma_at[s_]
                self.dma_ld(S_RK if i < 4 else S_RV, i % 4)

    def body(self, u, variant):
        """Loop body of tile S_IT with stream parity u, one of the variants: full (S(t+1),
        softmax(t), PV(t)), last / lastm (softmax and PV of a wave's last active tile,
        unpipelined; lastm masks it first), idle (requests only).  Every variant makes the
        stream's two requests and ends with one workgroup barrier."""
        p = self.p
        Jn = u ^ 1
        p.comment(f"body {variant} {u}")
        h = split_scalar(self.capture(self.body_scalar), 32)
        if variant == "full":
            self.tile_pipe(u, h)
        else:
            if variant == "lastm":
                self.stage_mask(u, S_IT)
                for st in self.lane_max_steps(u):
                    self.lane_max_step(st)
                self.rescale_test()
                self.rescale_if(f".Lnr_lastm{u}")
            self.dma_tile(S_RK, LDS_K[u])
            self.dma_tile(S_RV, LDS_V[Jn])
            if variant != "idle":
                self.stage_softmax_pv(u, LDS_V[u])
            for c in h:
                p.ins.extend(c)
        p.waitcnt(vm=0)
        p.barrier()
        if variant == "full":
            # S(t+1)'s test stands unless tile t+1 gets a mask first (its body tests again)
            self.s(f"s_bitcmp1_b32 {sr(S_CODE)}, 0", S(S_CODE), [("scc", 0)])
            p.branch(f"s_cbranch_scc1 .Lnr_full{u}", [("scc", 0)], skip_xdl=ACC)
            self.rescale_if(f".Lnr_full{u}")
        self.s(f"s_cmp_eq_u32 {sr(S_CODE)}, 6", S(S_CODE), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lfull{Jn}", [("scc", 0)], skip_xdl=ACC)
        p.branch(f"s_branch .Ldisp{Jn}", skip_xdl=ACC)

    # ---------------------------------------------------------------- item start / end
    def q_loads(self, b, h, q0, abase):
        """Issue the loads of Q rows q0 + 32qb + l32 of (batch b, head h) for this wave into
        the AGPRs at abase (untracked: the prologue waits for them itself, and for the next
        item's, in the next-item AGPRs, the next loop body's vmcnt(0)): lane (l32, hi) loads
        bytes hi*16 + 32ks .. +15."""
        p, s = self.p, self.s
        RQ = S_TMP + 16
        T0, COL, LO, HI = S_TMP + 8, S_TMP + 9, S_TMP + 10, S_TMP + 11
        s(f"s_mul_i32 {sr(T0)}, {sr(b)}, {sr(S_SEQ)}", S(b) + S(S_SEQ), S(T0))
        s(f"s_lshl_b32 {sr(COL)}, {sr(h)}, 8", S(h), S(COL))
        self.add64(RQ, S_QKV, T0, S_LDB, COL, LO, HI)
        s(f"s_and_b32 {sr(RQ + 1)}, {sr(RQ + 1)}, 0xffff", S(RQ + 1), S(RQ + 1))
        self.nrec_rows(RQ + 2, S_SEQ, S_LDB)
        s(f"s_mov_b32 {sr(RQ + 3)}, 0x20000", [], S(RQ + 3))
        QOFF = V_P  # two registers
        p.valu(f"v_lshlrev_b32_e32 {vr(V_T)}, 2, {vr(V_HI4)}", V(V_HI4), V(V_T))     # 16*hi
        for qb in range(2):
            p.valu(f"v_add_u32_e32 {vr(QOFF + qb)}, {sr(q0)}, {vr(V_L32)}", S(q0) + V(V_L32), V(QOFF + qb))
            if qb:
                p.valu(f"v_add_u32_e32 {vr(QOFF + qb)}, 32, {vr(QOFF + qb)}", V(QOFF + qb), V(QOFF + qb))
            p.valu(f"v_mul_lo_u32 {vr(QOFF + qb)}, {vr(QOFF + qb)}, {sr(S_LDB)}", V(QOFF + qb) + S(S_LDB), V(QOFF + qb))
            p.valu(f"v_add_u32_e32 {vr(QOFF + qb)}, {vr(QOFF + qb)}, {vr(V_T)}", V(QOFF + qb) + V(V_T), V(QOFF + qb))
        for qb in range(2):
            for ks in range(8):
                i = (qb * 8 + ks) * 4
                p.vmem_load(f"buffer_load_dwordx4 {ar(abase + i, 4)}, {vr(QOFF + qb)}, {sr(RQ, 4)}, 0 offen offset:{ks * 32}",
                            A(abase + i, 4), V(QOFF + qb) + S(RQ, 4), untracked=True)

    def prefetch_next_q(self, sfx):
        """Loads of the next round's item's Q rows into the next-item AGPRs (none after the
        last item)."""
        p, s = self.p, self.s
        K, I, Z, B, H, KVH, R, QB = (S_TMP + k for k in range(8))
        s(f"s_add_u32 {sr(K)}, {sr(S_KA)}, 1", S(S_KA), S(K))
        self.item_index(K, I, S_TMP + 12)
        s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lpq_{sfx}", [("scc", 0)], skip_xdl=ACC)
        self.decode(I, Z, B, H, KVH, R)
        s(f"s_sub_u32 {sr(QB)}, {sr(S_NQBLK)}, 1", S(S_NQBLK), S(QB))
        s(f"s_sub_u32 {sr(QB)}, {sr(QB)}, {sr(Z)}", S(QB) + S(Z), S(QB))
        s(f"s_cmp_eq_u32 {sr(S_CAUSAL)}, 0", S(S_CAUSAL), [("scc", 0)])
        s(f"s_cselect_b32 {sr(QB)}, {sr(Z)}, {sr(QB)}", S(Z) + S(QB) + [("scc", 0)], S(QB))
        s(f"s_lshl_b32 {sr(QB)}, {sr(QB)}, 8", S(QB), S(QB))
        s(f"s_lshl_b32 {sr(Z)}, {sr(S_WAVE)}, 6", S(S_WAVE), S(Z))
        s(f"s_add_u32 {sr(QB)}, {sr(QB)}, {sr(Z)}", S(QB) + S(Z), S(QB))
        self.q_loads(B, H, QB, A_QN)
        p.label(f".Lpq_{sfx}")

    def reset_acc(self):
        """O accumulators and row sums to 0 (O by 8 MFMAs of zeros)."""
        p = self.p
        for i in range(4):
            p.valu(f"v_mov_b32_e32 {vr(V_KBUF + i)}, 0", [], V(V_KBUF + i))
        for i in range(8):
            p.mfma(MFMA, A_O + 16 * i, V_KBUF, V_KBUF, None, dst_acc=True)
        for qb in range(2):
            p.valu(f"v_mov_b32_e32 {vr(V_LSUM + qb)}, 0", [], V(V_LSUM + qb))

    def start_item(self, u, sfx, prefetch=True, drain=False, next_q=False):
        """Tile 0 of the current item (stream parity u): S(0) into set u when the wave uses
        it, its mask, and m = its row max; one barrier (the first body's requests
        overwrite K buffer u; drain: every DMA of this wave done before it, for the prologue,
        whose K(1) and V(0) may still be in flight); the loads of the next item's Q
        (prefetch); then the first body.  next_q: the item's Q is still in the next-item
        AGPRs; S(0) reads it there while it is copied into the Q AGPRs (or only copied, when
        the wave uses no tile of the item), and the O accumulators are reset first."""
        p, s = self.p, self.s
        p.comment(f"start {u}")
        if next_q:
            self.reset_acc()
        s(f"s_cmp_eq_u32 {sr(S_ACTEND)}, 0", S(S_ACTEND), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .Lsn_{sfx}", [("scc", 0)], skip_xdl=ACC)
        if next_q:
            self.stage_s_next(u, LDS_K[u])
        else:
            self.stage_s(u, LDS_K[u])
        s(f"s_cmp_eq_u32 {sr(S_MASKB)}, 0", S(S_MASKB), [("scc", 0)])
        p.branch(f"s_cbranch_scc0 .Lsm_{sfx}", [("scc", 0)], skip_xdl=ACC)
        self.stage_mask(u, S_IT)
        p.label(f".Lsm_{sfx}")
        self.row_max_set_m(u)
        if next_q:
            p.branch(f"s_branch .Lsj_{sfx}", skip_xdl=ACC)
        p.label(f".Lsn_{sfx}")
        if next_q:
            self.copy_next_q()
            p.label(f".Lsj_{sfx}")
        p.waitcnt(vm=0 if drain else None, lgkm=0)
        p.barrier()
        if prefetch:
            self.prefetch_next_q(sfx)
        self.code(S_TMP + 8, S_TMP + 9, S_TMP + 10)
        p.branch(f"s_branch .Ldisp{u}", skip_xdl=ACC)

    def epilogue(self):
        """O = acc / l (fp16) through the wave's LDS staging rows, LSE = (m + log2 l) ln 2."""
        p, s = self.p, self.s
        p.comment("epilogue")
        T0, T1, T2 = S_TMP, S_TMP + 1, S_TMP + 2
        # O descriptor: base out + b*S*ldo + h*256, S rows of ldo bytes up to the last row's head
        T3 = S_TMP + 3
        s(f"s_mul_i32 {sr(T0)}, {sr(S_BA)}, {sr(S_SEQ)}", S(S_BA) + S(S_SEQ), S(T0))
        s(f"s_lshl_b32 {sr(T3)}, {sr(S_HA)}, 8", S(S_HA), S(T3))
        self.add64(S_RQ, S_OUT, T0, S_LDO, T3, T1, T2)
        s(f"s_and_b32 {sr(S_RQ + 1)}, {sr(S_RQ + 1)}, 0xffff", S(S_RQ + 1), S(S_RQ + 1))
        self.nrec_rows(S_RQ + 2, S_SEQ, S_LDO)
        s(f"s_mov_b32 {sr(S_RQ + 3)}, 0x20000", [], S(S_RQ + 3))
        # LSE descriptor: base lse + (b*Hq + h)*S*4, S*4 bytes (none when lse is null)
        s(f"s_mul_i32 {sr(T0)}, {sr(S_BA)}, {sr(S_HQ)}", S(S_BA) + S(S_HQ), S(T0))
        s(f"s_add_u32 {sr(T0)}, {sr(T0)}, {sr(S_HA)}", S(T0) + S(S_HA), S(T0))
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
        Q, LO, L_, INV, LG = 0, 2, 3, 4, 5           # registers in the free score region
        W = 8                                        # 4 values + 2 packed words
        # staging: write address EPW + l32*272 + hi*8, read address EPW + (lane>>4)*272 +
        # (lane&15)*16; each read of 4 rows x 16 chunks becomes one store of 4 whole rows
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
        # offset of row q0 + (lane >> 4), chunk lane & 15 from the head's descriptor; +4 rows
        # per read
        p.valu(f"v_add_u32_e32 {vr(TA)}, {sr(S_Q0)}, {vr(TA)}", S(S_Q0) + V(TA), V(TA))
        p.valu(f"v_mul_lo_u32 {vr(TA)}, {vr(TA)}, {sr(S_LDO)}", V(TA) + S(S_LDO), V(TA))
        p.valu(f"v_lshl_add_u32 {vr(OOS)}, {vr(TB)}, 4, {vr(TA)}", V(TB) + V(TA), V(OOS))
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
            p.valu(f"v_sub_f32_e32 {vr(LG)}, {vr(LG)}, {vr(V_NEGM + qb)}", V(LG) + V(V_NEGM + qb), V(LG))
            p.valu(f"v_mul_f32_e32 {vr(LG)}, 0x3f317218, {vr(LG)}", V(LG), V(LG))
            p.valu(f"v_cndmask_b32_e32 {vr(LG)}, {vr(V_NINF)}, {vr(LG)}, vcc", V(V_NINF) + V(LG) + [("vcc", 0)], V(LG))
            p.vmem_store(f"buffer_store_dword {vr(LG)}, {vr(LO)}, {sr(S_RL, 4)}, 0 offen nt", V(LG) + V(LO) + S(S_RL, 4))
            for db in range(4):
                for g4 in range(4):
                    o = A_O + (db * 2 + qb) * 16 + g4 * 4
                    for j in range(4):
                        p.valu(f"v_accvgpr_read_b32 {vr(W + j)}, {ar(o + j)}", A(o + j), V(W + j))
                    for j in range(4):
                        p.valu(f"v_mul_f32_e32 {vr(W + j)}, {vr(W + j)}, {vr(INV)}", V(W + j) + V(INV), V(W + j))
                    p.valu(f"{self.pack_op} {vr(W + 4)}, {vr(W)}, {vr(W + 1)}", V(W, 2), V(W + 4))
                    p.valu(f"{self.pack_op} {vr(W + 5)}, {vr(W + 2)}, {vr(W + 3)}", V(W + 2, 2), V(W + 5))
                    p.ds_write(f"ds_write_b64 {vr(BW)}, {vr(W + 4, 2)} offset:{(db * 4 + g4) * 16}", V(BW) + V(W + 4, 2))
                    W = 8 if W == 16 else 16   # alternate register sets
            for i in range(8):   # LDS operations of a wave complete in order: reads see the rows
                R = RBUF + 4 * (i % 4)
                p.ds_read(f"ds_read_b128 {vr(R, 4)}, {vr(BR)} offset:{i * 4 * EPI_ROW}", V(R, 4), V(BR))
                p.vmem_store(f"buffer_store_dwordx4 {vr(R, 4)}, {vr(OOS + qb * 8 + i)}, {sr(S_RQ, 4)}, 0 offen nt",
                             V(R, 4) + V(OOS + qb * 8 + i) + S(S_RQ, 4))


def build(check_ldb: int = 12288, dt: str = "f16") -> str:
    """The kernel's assembly text: tkm_fa_fwd_d128_f16 (dt "f16") or tkm_fa_fwd_d128_bf16."""
    p = Prog()
    b = Body(p, dt)
    sal = p.salu
    # ------------------------------------------------------------------ prologue: scalars
    p.smem(f"s_load_dwordx16 {sr(8, 16)}, {sr(S_KARG, 2)}, 0x0", S(8, 16), S(S_KARG, 2))
    p.smem(f"s_load_dwordx8 {sr(24, 8)}, {sr(S_KARG, 2)}, 0x40", S(24, 8), S(S_KARG, 2))
    L = Lanes(p, check_ldb)
    L.shr(V_PT + 0, L.k(6), 0)
    p.readlane(f"v_readfirstlane_b32 {sr(S_WAVE)}, {vr(V_PT + 0)}", V(V_PT + 0), S(S_WAVE))
    p.waitcnt(lgkm=0)
    xcd_slot(p, S_WG, S_NWG, S_TMP, S_TMP + 1)
    # DMA row offset of this wave inside a tile: wave * 4 instructions * 4 rows * 256 B
    sal(f"s_lshl_b32 {sr(S_LDSW)}, {sr(S_WAVE)}, 12", S(S_WAVE), S(S_LDSW))
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
        sal(f"s_lshl_b32 {sr(T3)}, {sr(S_WAVE)}, 4", S(S_WAVE), S(T3))
        sal(f"s_add_u32 {sr(T3)}, {sr(T3)}, {4 * i}", S(T3), S(T3))
        L.add(TB, DR, L.s(T3, wave_vals * 16 + i * 4))
        L.mul(TB, TB, L.s(S_LDB, ldb_per_wave))
        L.or_(TC, TA, L.k(i))
        L.xor(TC, TC, DP)
        L.shl(TC, L.k(4), TC)
        L.add(V_DOFF + i, TB, TC)
    row_read_offsets(L, V_KOFF, (LANE, L32, HI), (TA, TB, TC))
    tr_read_offsets(L, V_VOFF, (LANE, L32, HI), (TA, TB, TC, V_PT + 9, V_PT + 10, V_PT + 11, V_PT + 12))
    _check_lanes(L, check_ldb)
    p.valu(f"v_mov_b32_e32 {vr(V_L32)}, {vr(L32)}", V(L32), V(V_L32))
    p.valu(f"v_lshlrev_b32_e32 {vr(V_HI4)}, 2, {vr(HI)}", V(HI), V(V_HI4))
    p.valu(f"v_mov_b32_e32 {vr(V_NINF)}, 0xff800000", [], V(V_NINF))
    # ------------------------------------------------------------------ first item
    # The wave's Q rows are requested first and K(0) next, so that S(0) waits only for those
    # while K(1) and V(0) are still arriving (every workgroup requests its first rows at once,
    # and HBM serves them roughly in order).
    for r in (S_KA, S_KD):
        sal(f"s_mov_b32 {sr(r)}, 0", [], S(r))
    sal(f"s_mov_b32 {sr(S_THR)}, {np.float32(RESCALE_LOG2).view(np.uint32):#x}", [], S(S_THR))
    b.item_index(S_KA, S_TMP + 15, S_TMP + 12)
    b.decode_a(S_TMP + 15, "p")
    b.q_loads(S_BA, S_HA, S_Q0, A_Q)                         # 16 loads
    b.decode_d("p0")
    b.stream_start(0, "p")                                   # K(0), K(1), V(0): 4 DMAs each
    b.reset_acc()
    p.waitcnt(vm=8)                                          # the Q rows, this wave's part of K(0)
    p.barrier()
    b.start_item(0, "p", drain=True)
    for u in range(2):
        _dispatch(b, u)
    for u in range(2):
        _boundary(b, u)
    p.label(".Lexit")
    p.waitcnt(vm=0, lgkm=0)
    p.emit("s_endpgm", BRANCH)
    return kernel_text(kernel_name(dt), p.finalize(), lds_bytes=LDS_BYTES, kernarg_bytes=KERNARG_BYTES,
                       next_free_sgpr=NEXT_FREE_SGPR, args=ARGS, wg_ids=(1, 0, 0))


def kernel_name(dt: str = "f16") -> str:
    return f"tkm_fa_fwd_d128_{dt}"


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


def _dispatch(b: Body, u: int):
    """Between bodies (the next tile has stream parity u): the stream's next item when its
    item is done (+16), the item's end (8), else the body variant by code."""
    p, s = b.p, b.s
    p.label(f".Ldisp{u}")
    s(f"s_bitcmp1_b32 {sr(S_CODE)}, 4", S(S_CODE), [("scc", 0)])
    p.branch(f"s_cbranch_scc0 .Lnod{u}", [("scc", 0)], skip_xdl=ACC)
    s(f"s_add_u32 {sr(S_KD)}, {sr(S_KD)}, 1", S(S_KD), S(S_KD))
    b.decode_d(f"d{u}")
    b.rsrc_k(S_TMP + 12)
    s(f"s_andn2_b32 {sr(S_CODE)}, {sr(S_CODE)}, 16", S(S_CODE), S(S_CODE))
    p.label(f".Lnod{u}")
    s(f"s_bitcmp1_b32 {sr(S_CODE)}, 3", S(S_CODE), [("scc", 0)])
    p.branch(f"s_cbranch_scc1 .Lbnd{u}", [("scc", 0)], skip_xdl=ACC)
    for lab, c in VARIANTS[:-1]:
        s(f"s_cmp_eq_u32 {sr(S_CODE)}, {c}", S(S_CODE), [("scc", 0)])
        p.branch(f"s_cbranch_scc1 .L{lab}{u}", [("scc", 0)], skip_xdl=ACC)
    for lab, _ in VARIANTS[::-1]:
        p.label(f".L{lab}{u}")
        b.body(u, lab)


def _boundary(b: Body, u: int):
    """End of the current item (the next tile has stream parity u): O and LSE out, then the
    next item (or stop): its Q, S(0) from K buffer u."""
    p, s = b.p, b.s
    I = S_TMP + 15
    p.label(f".Lbnd{u}")
    p.nop(16)
    p.waitcnt(lgkm=0)
    b.epilogue()
    s(f"s_add_u32 {sr(S_KA)}, {sr(S_KA)}, 1", S(S_KA), S(S_KA))
    b.item_index(S_KA, I, S_TMP + 12)
    s(f"s_cmp_ge_u32 {sr(I)}, {sr(S_NI)}", S(I) + S(S_NI), [("scc", 0)])
    p.branch("s_cbranch_scc1 .Lexit", [("scc", 0)], skip_xdl=ACC)
    p.comment("next q")
    b.decode_a(I, f"b{u}")
    b.start_item(u, f"b{u}", next_q=True)


def main(path: str) -> None:
    with open(path, "w") as f:
        f.write(build())


if __name__ == "__main__":
    import sys
    main(sys.argv[1])

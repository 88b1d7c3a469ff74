"""Scalar control flow of the generated persistent attention kernels, run on the CPU by
tests/asm_scalar_sim.py over whole launches: every workgroup ends, all four waves meet at
every barrier, each item is stored exactly once, descriptors stay inside their tensors, and
every K/V tile a body or an item start reads was requested earlier with the expected rows."""
import struct

import pytest

from tokamak_amd.asmgen import attn_fwd, gfx950

from asm_scalar_sim import M64, Fail, Sim

QKV, OUT, LSE, KVLEN = 0x10000000, 0x40000000, 0x70000000, 0x7F000000


def reciprocal(d, limit):
    if d == 1:
        return 0
    m = ((1 << 32) + d - 1) // d
    e = m * d - (1 << 32)
    assert m <= 0xFFFFFFFF and (limit - 1) * e < (1 << 32)
    return m


_lines = {}


def fwd_lines(dt="f16"):
    key = "fwd-" + dt
    if key not in _lines:
        captured = []
        orig = gfx950.Prog.finalize

        def finalize(self):
            out = orig(self)
            captured.append(out)
            return out
        gfx950.Prog.finalize = finalize
        try:
            attn_fwd.build(dt=dt)
        finally:
            gfx950.Prog.finalize = orig
        _lines[key] = captured[-1]
    return _lines[key]


def run_fwd(B, S, Hq, Hkv, causal, kv_len, n_wg, vcmp_lanes=M64, dt="f16"):
    n_qblk = (S + 255) // 256
    bhq, G = B * Hq, Hq // Hkv
    n_items = n_qblk * bhq
    n_wg = min(n_wg, n_items)
    ldb, ldo = (Hq + 2 * Hkv) * 256, Hq * 256
    kv = None if kv_len is None else [int(x) for x in kv_len]
    args = struct.pack("<QQQQIIIfIIIIIIIIIIII", QKV, OUT, LSE, KVLEN if kv else 0, S, Hq, Hkv,
                       0.127, int(causal), n_qblk, ldb, ldo, G, n_wg, n_items, bhq,
                       reciprocal(n_qblk, n_items), reciprocal(Hq, bhq), reciprocal(G, Hq), 0)
    assert len(args) == attn_fwd.KERNARG_BYTES
    mem = {"qkv": (QKV, B * S * ldb, ldb, 256), "out": (OUT, B * S * ldo, ldo, ldo),
           "lse": (LSE, B * Hq * S * 4, 4, 4), "kv_len": (KVLEN, 4 * B, 4, 4)}

    def kvl(b):
        return S if kv is None else max(0, min(kv[b], S))

    def kvend(b, qblk):
        return min(kvl(b), 256 * qblk + 256) if causal else kvl(b)

    def tile(b, kvh, qblk, t, v):
        col = (Hq + (Hkv if v else 0) + kvh) * 256
        rows = max(0, min(64, kvend(b, qblk) - 64 * t))
        return QKV + (b * S + 64 * t) * ldb + col, (rows - 1) * ldb + 256 if rows else 0

    def item_of(w):
        s = w.s
        b, h, kvh, q0 = s[attn_fwd.S_BA], s[attn_fwd.S_HA], s[attn_fwd.S_KVHA], s[attn_fwd.S_Q0]
        return b, h, kvh, q0, q0 >> 8

    def expect(w, words):
        b, h, kvh, q0, qblk = item_of(w)
        s = w.s
        if words[0] == "start":
            assert kvh == h // G
            nt = max(1, -(-kvend(b, qblk) // 64))
            act = 0 if kvl(b) == 0 else (min(nt, q0 // 64 + 1) if causal else nt)
            maskb = min(kvl(b) // 64, q0 // 64 if causal else nt)
            got = (s[attn_fwd.S_NT], s[attn_fwd.S_ACTEND], s[attn_fwd.S_MASKB], s[attn_fwd.S_IT])
            if got != (nt, act, maskb, 0):
                raise Fail(f"item (b {b}, h {h}, q0 {q0}): NT/ACTEND/MASKB/IT {got}, expected {(nt, act, maskb, 0)}")
            u = int(words[1])
            return [(attn_fwd.LDS_K[u], *tile(b, kvh, qblk, 0, False))] if act else []
        if words[0] == "body":
            variant, u, t = words[1], int(words[2]), s[attn_fwd.S_IT]
            code = s[attn_fwd.S_CODE] & ~16
            if dict(attn_fwd.VARIANTS).get(variant) not in (code, code & ~1 if variant == "idle" else code):
                raise Fail(f"body {variant} entered with code {code}")
            if variant == "full":
                return [(attn_fwd.LDS_K[u ^ 1], *tile(b, kvh, qblk, t + 1, False)),
                        (attn_fwd.LDS_V[u], *tile(b, kvh, qblk, t, True))]
            if variant in ("last", "lastm"):
                return [(attn_fwd.LDS_V[u], *tile(b, kvh, qblk, t, True))]
        return []

    stored = {}
    next_q = {}
    checked = [0]

    def on_event(w, words):
        if words[0] == "epilogue":
            b, h, _, q0, _ = item_of(w)
            key = (b, h, q0)
            stored[key] = stored.get(key, 0) + 1
        elif words[0] == "next" and words[1] == "q":
            # the next item's Q, loaded into the next-item AGPRs during this item
            next_q[(w.wg, w.wave)] = [(o, base) for o, base in w.loads
                                      if o[0] == "a" and attn_fwd.A_QN <= o[1] < attn_fwd.A_QN + 64]
            w.loads.clear()
        elif words[0] == "start" and (w.wg, w.wave) in next_q:
            b, h, _, _, _ = item_of(w)
            loads = next_q.pop((w.wg, w.wave))
            regs = sorted(o[1] for o, _ in loads)
            if regs != list(range(attn_fwd.A_QN, attn_fwd.A_QN + 64, 4)):
                raise Fail(f"next-item Q loads into {regs}")
            if {base for _, base in loads} != {QKV + b * S * ldb + h * 256}:
                raise Fail(f"next-item Q loads of another head: {sorted({base for _, base in loads})}")
            checked[0] += 1

    sim = Sim(fwd_lines(dt), args, mem, kv, n_wg, expect, on_event, vcmp_lanes=vcmp_lanes, max_steps=8_000_000)
    sim.run()
    want = {(b, h, 256 * z + 64 * wv) for b in range(B) for h in range(Hq) for z in range(n_qblk) for wv in range(4)}
    assert set(stored) == want and all(c == 1 for c in stored.values()), \
        (len(stored), len(want), [k for k, c in stored.items() if c != 1][:4])
    # O and LSE stores of each wave target its item's rows
    assert {m for _, _, m, _, _ in sim.stores} <= {"out", "lse", None}
    # every item after a workgroup's first found its Q loaded during the previous item
    assert checked[0] == 4 * (n_items - n_wg) and not next_q, (checked[0], n_items, n_wg)
    return sim


@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", [
    (1, 512, 2, 1, True, None, 3),
    (2, 700, 4, 2, True, None, 5),
    (2, 700, 4, 2, False, None, 4),
    (2, 1000, 2, 2, False, [1000, 333], 3),
    (3, 600, 2, 1, True, [0, 65, 600], 2),
    (1, 64, 1, 1, True, None, 1),
    (1, 1, 1, 1, False, None, 1),
    (2, 2048, 4, 4, True, None, 7),
    (1, 512, 4, 2, True, None, 8),          # one item per workgroup: the DMA stream runs past the last item
    (1, 300, 3, 1, True, [129], 256),
    (2, 2048, 4, 2, True, None, 20),        # 20 places over the 8 XCDs: 3, 3, 3, 3, 2, 2, 2, 2
])
def test_fwd_scalar_flow(B, S, Hq, Hkv, causal, kv_len, n_wg):
    run_fwd(B, S, Hq, Hkv, causal, kv_len, n_wg)


@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", [
    (2, 700, 4, 2, True, None, 5),
    (2, 1000, 2, 2, False, [1000, 333], 3),
    (1, 512, 4, 2, True, None, 8),
])
def test_fwd_bf16_scalar_flow(B, S, Hq, Hkv, causal, kv_len, n_wg):
    """The bf16 kernel (96-slot bodies, P in two halves) has the fp16 kernel's scalar flow."""
    run_fwd(B, S, Hq, Hkv, causal, kv_len, n_wg, dt="bf16")
    run_fwd(B, S, Hq, Hkv, causal, kv_len, n_wg, vcmp_lanes=0, dt="bf16")


def test_fwd_scalar_flow_without_rescale():
    """The rescale test failing everywhere (no lane ever needs a larger m) leaves the same
    flow: every tile arrives as expected and each item is stored once (the other tests run
    with every test passing, so every body takes the rescale)."""
    run_fwd(2, 700, 4, 2, True, None, 3, vcmp_lanes=0)
    run_fwd(1, 512, 2, 1, False, [300], 2, vcmp_lanes=0)


# ---------------------------------------------------------------- backward kernels
from tokamak_amd.asmgen import attn_dkdv, attn_dq  # noqa: E402

O_, DOUT, QUADS, DELTA, DQKV = 0x20000000, 0x30000000, 0x50000000, 0x60000000, 0x80000000


def _gen_lines(gen, dt="f16"):
    key = gen.NAME if dt == "f16" else gen.NAME + "-" + dt
    if key not in _lines:
        captured = []
        orig = gfx950.Prog.finalize

        def finalize(self):
            out = orig(self)
            captured.append(out)
            return out
        gfx950.Prog.finalize = finalize
        try:
            gen.build() if dt == "f16" else gen.build(dt=dt)
        finally:
            gfx950.Prog.finalize = orig
        _lines[key] = captured[-1]
    return _lines[key]


def _bwd_mem(B, S, Hq, Hkv, kv):
    ldb, ldo = (Hq + 2 * Hkv) * 256, Hq * 256
    sp = (S + 31) // 32 * 32
    return {"qkv": (QKV, B * S * ldb, ldb, 256), "dqkv": (DQKV, B * S * ldb, ldb, 256),
            "o": (O_, B * S * ldo, ldo, 256), "dout": (DOUT, B * S * ldo, ldo, 256),
            "lse": (LSE, B * Hq * S * 4, 4, 4), "delta": (DELTA, B * Hq * S * 4, 4, 4),
            "quads": (QUADS, B * Hq * sp * 8, 16, 16), "kv_len": (KVLEN, 4 * B, 4, 4)}


def run_dkdv(B, S, Hq, Hkv, causal, kv_len, n_wg, dt="f16"):
    n_kblk, bh = (S + 127) // 128, B * Hkv
    n_items = n_kblk * bh
    n_wg = min(n_wg, n_items)
    ldb, ldo = (Hq + 2 * Hkv) * 256, Hq * 256
    kv = None if kv_len is None else [int(x) for x in kv_len]
    args = struct.pack("<QQQQQIIIfIIIIfIIIIIII", QKV, DOUT, QUADS, DQKV, KVLEN if kv else 0, S, Hq, Hkv,
                       0.127, int(causal), ldb, ldo, Hq // Hkv, 0.088, n_kblk, (S + 31) // 32 * 32, n_wg,
                       n_items, bh, reciprocal(n_kblk, n_items), reciprocal(Hkv, bh))
    assert len(args) == attn_dkdv.KERNARG_BYTES
    stored = {}
    next_kv = {}
    checked = [0]
    spare = range(attn_dkdv.A_NK, attn_dkdv.A_NV + 32)

    def on_event(w, words):
        if words[0] == "epilogue":
            key = (w.s[attn_dkdv.S_BA], w.s[attn_dkdv.S_KVHA], w.s[attn_dkdv.S_KW0])
            stored[key] = stored.get(key, 0) + 1
        elif words[0] == "next" and words[1] == "kv":
            # the next item's K and V, loaded into the spare AGPRs before this boundary
            next_kv[(w.wg, w.wave)] = [(o, base) for o, base in w.loads if o[0] == "a" and o[1] in spare]
            w.loads.clear()
        elif words[0] == "item":
            b, kvh, kw0 = w.s[attn_dkdv.S_BA], w.s[attn_dkdv.S_KVHA], w.s[attn_dkdv.S_KW0]
            # the stream's Q / dO descriptors end at the last row's last head of the kv group
            G = Hq // Hkv
            got = (w.s[attn_dkdv.S_RQ + 2], w.s[attn_dkdv.S_RO + 2])
            if got != ((S - 1) * ldb + G * 256, (S - 1) * ldo + G * 256):
                raise Fail(f"Q / dO descriptor sizes {got}")
            loads = next_kv.pop((w.wg, w.wave))
            if sorted(o[1] for o, _ in loads) != list(range(attn_dkdv.A_NK, attn_dkdv.A_NV + 32, 4)):
                raise Fail(f"next-item K/V loads into {sorted(o[1] for o, _ in loads)}")
            k_base = QKV + (b * S + kw0) * ldb + (Hq + kvh) * 256
            for o, base in loads:
                want = k_base + (Hkv * 256 if o[1] >= attn_dkdv.A_NV else 0)
                if base != want:
                    raise Fail(f"next-item {'V' if o[1] >= attn_dkdv.A_NV else 'K'} load from {base:#x}, expected {want:#x}")
            checked[0] += 1

    # largest lane offset of each DMA address register: rows wave*8 + 4i + 0..3 of a tile, 256 B
    reach = {attn_dkdv.V_LOFF: 255}
    for i in range(2):
        reach[attn_dkdv.V_DOFF + i] = tuple((8 * w + 4 * i + 3) * ldb + 255 for w in range(4))
        reach[attn_dkdv.V_DOFF + 2 + i] = tuple((8 * w + 4 * i + 3) * ldo + 255 for w in range(4))
    sim = Sim(_gen_lines(attn_dkdv, dt), args, _bwd_mem(B, S, Hq, Hkv, kv), kv, n_wg, None, on_event,
              wave_vgpr=attn_dkdv.V_PT, lane_max=reach)
    sim.run()
    want = {(b, h, 128 * z + 32 * w) for b in range(B) for h in range(Hkv) for z in range(n_kblk) for w in range(4)}
    assert set(stored) == want and all(c == 1 for c in stored.values()), \
        (len(stored), len(want), [k for k, c in stored.items() if c != 1][:4])
    # every item after a workgroup's first found its K, V loaded during the previous item
    assert checked[0] == 4 * (n_items - n_wg) and not next_kv, (checked[0], n_items, n_wg)
    return sim


def run_dq(B, S, Hq, Hkv, causal, kv_len, n_wg, compute_d, dt="f16"):
    n_qblk, bhq, G = (S + 255) // 256, B * Hq, Hq // Hkv
    n_items = n_qblk * bhq
    n_wg = min(n_wg, n_items)
    ldb, ldo = (Hq + 2 * Hkv) * 256, Hq * 256
    kv = None if kv_len is None else [int(x) for x in kv_len]
    args = struct.pack("<QQQQQQQQIIIfIIIIfIIIIIIIII", QKV, O_, DOUT, LSE, DELTA, QUADS, DQKV,
                       KVLEN if kv else 0, S, Hq, Hkv, 0.127, int(causal), ldb, ldo, G, 0.088, n_qblk,
                       (S + 31) // 32 * 32, n_wg, n_items, bhq, reciprocal(n_qblk, n_items),
                       reciprocal(Hq, bhq), reciprocal(G, Hq), int(compute_d))
    assert len(args) == attn_dq.KERNARG_BYTES
    stored = {}
    checked = [0]

    def on_event(w, words):
        if words[0] == "epilogue":
            key = (w.s[attn_dq.S_BA], w.s[attn_dq.S_HA], w.s[attn_dq.S_Q0])
            stored[key] = stored.get(key, 0) + 1
        elif words[0] == "next" and words[1] == "rows":
            w.loads.clear()
        elif words[0] == "item":
            # the rows requested before the epilogue are the new item's: Q -> v0..63,
            # dO -> its AGPRs, O -> v64..127 (computing D), LSE -> two VGPRs
            b, h = w.s[attn_dq.S_BA], w.s[attn_dq.S_HA]
            row, col = b * S, h * 256
            want = sorted([(("v", 4 * k, 4), QKV + row * ldb + col) for k in range(16)] +
                          [(("a", attn_dq.A_O + 4 * k, 4), DOUT + row * ldo + col) for k in range(16)] +
                          [(("v", attn_dq.V_T + 5 + k, 1), LSE + (b * Hq + h) * S * 4) for k in range(2)] +
                          ([(("v", 64 + 4 * k, 4), O_ + row * ldo + col) for k in range(16)] if compute_d else []))
            got = sorted(w.loads)
            if got != want:
                raise Fail(f"next-item row loads {got[:3]}..., expected {want[:3]}...")
            # each row descriptor ends at the batch's last row of the head
            for base, ld in ((QKV + row * ldb + col, ldb), (DOUT + row * ldo + col, ldo)):
                if w.load_nrec[base] != (S - 1) * ld + 256:
                    raise Fail(f"row descriptor at {base:#x}: {w.load_nrec[base]} bytes")
            w.loads.clear()
            checked[0] += 1

    sim = Sim(_gen_lines(attn_dq, dt), args, _bwd_mem(B, S, Hq, Hkv, kv), kv, n_wg, None, on_event,
              wave_vgpr=attn_dq.V_PT)
    sim.run()
    want = {(b, h, 256 * z + 64 * w) for b in range(B) for h in range(Hq) for z in range(n_qblk) for w in range(4)}
    assert set(stored) == want and all(c == 1 for c in stored.values()), \
        (len(stored), len(want), [k for k, c in stored.items() if c != 1][:4])
    # every item after a workgroup's first found its rows requested before the epilogue
    assert checked[0] == 4 * (n_items - n_wg), (checked[0], n_items, n_wg)
    return sim


BWD_CASES = [(1, 512, 2, 1, True, None, 3), (2, 700, 4, 2, True, None, 5), (2, 700, 4, 2, False, None, 4),
             (2, 1024, 8, 8, True, None, 16),
             (2, 1000, 2, 2, False, [1000, 333], 3), (3, 600, 2, 1, True, [0, 65, 600], 2),
             (1, 64, 1, 1, True, None, 1), (1, 1, 1, 1, False, None, 1), (1, 300, 3, 1, True, [129], 256),
             (2, 1024, 4, 2, True, None, 12)]


# GQA shapes whose last items have one visible query tile per head: past its last item the
# unfixed dK/dV stream advanced one head per request, past the group's last, and read 256
# bytes past the end of dO
DKDV_PAST_END = [(1, 6, 4, 2, True, [2], 1), (2, 800, 4, 2, True, None, 8), (3, 131, 4, 2, True, None, 3)]


@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", [BWD_CASES[1], BWD_CASES[4], DKDV_PAST_END[0],
                                                          DKDV_PAST_END[1]])
def test_dkdv_bf16_scalar_flow(B, S, Hq, Hkv, causal, kv_len, n_wg):
    """The bf16 kernel (48-slot bodies, P and dS in two halves) has the fp16 kernel's flow."""
    run_dkdv(B, S, Hq, Hkv, causal, kv_len, n_wg, dt="bf16")


@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", BWD_CASES + DKDV_PAST_END)
def test_dkdv_scalar_flow(B, S, Hq, Hkv, causal, kv_len, n_wg):
    """Every workgroup ends, waves meet at every barrier, DMA and stores stay in their tensors,
    and each (key block, batch, kv head) item's dK and dV rows are stored."""
    sim = run_dkdv(B, S, Hq, Hkv, causal, kv_len, n_wg)
    assert {m for _, _, m, _, _ in sim.stores} <= {"dqkv", None}
    ldb = (Hq + 2 * Hkv) * 256
    heads = {(base - DQKV) % ldb // 256 for _, _, m, base, _ in sim.stores if m}
    assert heads == set(range(Hq, Hq + 2 * Hkv))


@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", [BWD_CASES[1], BWD_CASES[4], BWD_CASES[5]])
def test_dq_bf16_scalar_flow(B, S, Hq, Hkv, causal, kv_len, n_wg):
    """The bf16 kernel (64-slot bodies, dS^T in two halves) has the fp16 kernel's flow."""
    run_dq(B, S, Hq, Hkv, causal, kv_len, n_wg, True, dt="bf16")
    run_dq(B, S, Hq, Hkv, causal, kv_len, n_wg, False, dt="bf16")


@pytest.mark.parametrize("compute_d", [True, False])
@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", BWD_CASES)
def test_dq_scalar_flow(B, S, Hq, Hkv, causal, kv_len, n_wg, compute_d):
    sim = run_dq(B, S, Hq, Hkv, causal, kv_len, n_wg, compute_d)
    stored = {m for _, _, m, _, _ in sim.stores}
    assert stored <= ({"dqkv", "delta", "quads", None} if compute_d else {"dqkv", None})
    # D and the row values of every item go to its (batch, head)'s own rows: one descriptor
    # per (b, h) covering exactly S floats of delta / SP*2 floats of row values
    sp = (S + 31) // 32 * 32
    for _, _, m, base, nrec in sim.stores:
        if m == "delta":
            assert nrec == 4 * S and (base - DELTA) % (4 * S) == 0, (hex(base), nrec)
        elif m == "quads":
            assert nrec == 8 * sp and (base - QUADS) % (8 * sp) == 0, (hex(base), nrec)
    if compute_d:
        heads = {(base - DELTA) // (4 * S) for _, _, m, base, _ in sim.stores if m == "delta"}
        assert heads == set(range(B * Hq))
    ldb = (Hq + 2 * Hkv) * 256
    heads = {(base - DQKV) % ldb // 256 for _, _, m, base, _ in sim.stores if m == "dqkv"}
    assert heads == set(range(Hq))


# ---------------------------------------------------------------- seeded random shapes
def _random_shapes(seed, n):
    """Shapes the fixed cases above do not pin down: GQA ratios up to 8, ragged S, per-batch
    key lengths (0 and S included), and workgroup counts from 1 to a full MI355X."""
    import random
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        B = rng.randint(1, 3)
        Hkv = rng.randint(1, 2)
        Hq = Hkv * rng.choice((1, 2, 3, 4, 8))
        if B * Hq > 12:
            continue
        S = rng.choice((rng.randint(1, 300), rng.randint(300, 1200)))
        causal = rng.random() < 0.6
        kv_len = None
        if rng.random() < 0.4:
            kv_len = [rng.choice((0, S, rng.randint(0, S))) for _ in range(B)]
        n_wg = rng.choice((1, 2, 3, 5, 8, 9, 13, 256))
        out.append((B, S, Hq, Hkv, causal, kv_len, n_wg))
    return out


@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", _random_shapes(1, 8))
def test_fwd_scalar_flow_random(B, S, Hq, Hkv, causal, kv_len, n_wg):
    run_fwd(B, S, Hq, Hkv, causal, kv_len, n_wg)


@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", _random_shapes(2, 8))
def test_dkdv_scalar_flow_random(B, S, Hq, Hkv, causal, kv_len, n_wg):
    run_dkdv(B, S, Hq, Hkv, causal, kv_len, n_wg)


@pytest.mark.parametrize("B,S,Hq,Hkv,causal,kv_len,n_wg", _random_shapes(3, 8))
def test_dq_scalar_flow_random(B, S, Hq, Hkv, causal, kv_len, n_wg):
    run_dq(B, S, Hq, Hkv, causal, kv_len, n_wg, compute_d=(S % 2 == 0))


# ---------------------------------------------------------------- descriptor reach
@pytest.mark.parametrize("gen", ["fwd", "dq", "dkdv"])
def test_descriptors_end_at_the_tensor_end(monkeypatch, gen):
    """Every descriptor ends at or before the end of its tensor (Sim._inside): a descriptor
    over whole rows of the packed pitch (rows * stride bytes, the earlier form) reaches up to
    stride - 256 bytes past the tensor for the last batch's rows, and the check must catch it
    for each kernel; the kernels as built pass the same shape."""
    mod = {"fwd": attn_fwd, "dq": attn_dq, "dkdv": attn_dkdv}[gen]
    shape = (2, 300, 4, 2, True, None, 5)
    run = {"fwd": lambda: run_fwd(*shape), "dq": lambda: run_dq(*shape, compute_d=True),
           "dkdv": lambda: run_dkdv(*shape)}[gen]
    run()

    def whole_rows(self, dst, rows, stride, *width):
        self.s(f"s_mul_i32 {gfx950.sr(dst)}, {gfx950.sr(rows)}, {gfx950.sr(stride)}",
               gfx950.S(rows) + gfx950.S(stride), gfx950.S(dst))
    monkeypatch.setattr(mod.Body, "nrec_rows", whole_rows)
    key = "fwd-f16" if gen == "fwd" else mod.NAME
    good = _lines.pop(key)
    try:
        # (the forward's tile check, which compares each K/V tile's descriptor with the
        # expected one, may see the longer descriptor first)
        with pytest.raises(Fail, match="outside every tensor" if gen != "fwd" else "outside every tensor|holds"):
            run()
    finally:
        _lines[key] = good

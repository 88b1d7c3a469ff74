"""Pins of the CPU oracle (oracle/attn_ref.c) -- runs without a GPU.

The reference ships no CPU attention and no test or golden vector for this path, so the
oracle is pinned by: the published PCG32 known-answer vector (its input generator),
IEEE rounding against numpy/torch, closed forms, an independent float64 brute force that
uses the textbook softmax gradient (rowsum(P*dP) rather than the oracle's <O, dO>),
torch-generated golden fixtures (tests/golden/attn_golden.npz), finite differences,
invariants, GQA <-> MHA equivalence, and planted mistakes that these checks must catch.
"""
import math
import os

import numpy as np
import pytest

import oracle

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden", "attn_golden.npz")


def scale_of(D):
    return float(np.float32(1.0) / np.sqrt(np.float32(D)))


# ----------------------------------------------------------------------------- inputs
def test_pcg32_known_answer():
    # pcg32-demo (O'Neill, pcg-c-basic): pcg32_srandom_r(&rng, 42u, 54u), first six outputs
    got = [int(x) for x in oracle.pcg32_sequence(42, 54, 6)]
    assert got == [0xa15c02b7, 0x7b47f409, 0xba1d3330, 0x83d2f293, 0xbfa4784b, 0xcbed606e]


def test_box_muller_matches_formula():
    r = oracle.pcg32_sequence(3, 2, 64).astype(np.float64)
    u1 = (np.floor(r[0::2] / 256.0) + 1.0) / 16777216.0
    u2 = np.floor(r[1::2] / 256.0) / 16777216.0
    rad = np.sqrt(-2.0 * np.log(u1))
    want = np.empty(64)
    want[0::2] = rad * np.cos(2 * np.pi * u2)
    want[1::2] = rad * np.sin(2 * np.pi * u2)
    got = oracle.normal(64, 3, 2)
    np.testing.assert_allclose(got, want.astype(np.float32), rtol=2e-7, atol=1e-7)
    z = oracle.normal(200000, 0, 1)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01


def test_round_f16_matches_numpy():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * s for s in (1e-6, 1e-3, 1, 300, 7e4)])
    x = np.concatenate([x, np.array([0.0, -0.0, 65504, 65520, -65519.9, 6.1e-5, 5.96e-8, 2.98e-8,
                                     1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, np.inf, -np.inf], dtype=np.float32)])
    got, bits = oracle.round_to(x, "f16")
    with np.errstate(over="ignore"):
        want = x.astype(np.float16)
    np.testing.assert_array_equal(bits, want.view(np.uint16))
    np.testing.assert_array_equal(got, want.astype(np.float32))
    np.testing.assert_array_equal(oracle.widen(bits, "f16"), want.astype(np.float32))


def test_round_bf16_matches_torch():
    import torch
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(20000).astype(np.float32) * s for s in (1e-30, 1e-3, 1, 1e30)])
    x = np.concatenate([x, np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 3.4e38, -np.inf], dtype=np.float32)])
    got, bits = oracle.round_to(x, "bf16")
    want = torch.from_numpy(x).to(torch.bfloat16)
    np.testing.assert_array_equal(bits, want.view(torch.int16).numpy().view(np.uint16))
    np.testing.assert_array_equal(got, want.float().numpy())


# ------------------------------------------------------------------------- brute force
def brute(qkv, dout, B, S, Hq, Hkv, D, causal, kv_len=None):
    """Textbook float64 attention and gradient: explicit P, dS = P*(dP - rowsum(P*dP))."""
    g = Hq // Hkv
    sc = scale_of(D)
    x = qkv.astype(np.float64).reshape(B, S, Hq + 2 * Hkv, D)
    q, k, v = x[:, :, :Hq], x[:, :, Hq:Hq + Hkv], x[:, :, Hq + Hkv:]
    do = dout.astype(np.float64).reshape(B, S, Hq, D)
    o = np.zeros((B, S, Hq, D))
    lse = np.full((B, Hq, S), -np.inf)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b in range(B):
        kvl = S if kv_len is None else max(0, min(S, kv_len[b]))
        vis = np.zeros((S, S), dtype=bool)
        vis[:, :kvl] = True
        if causal:
            vis &= np.tril(np.ones((S, S), dtype=bool))
        for h in range(Hq):
            kh = h // g
            s = sc * q[b, :, h] @ k[b, :, kh].T
            s = np.where(vis, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            has = np.isfinite(m[:, 0])
            e = np.where(vis, np.exp(s - np.where(has[:, None], m, 0.0)), 0.0)
            l = e.sum(axis=1, keepdims=True)
            P = np.where(has[:, None], e / np.where(l > 0, l, 1.0), 0.0)
            o[b, :, h] = P @ v[b, :, kh]
            lse[b, h] = np.where(has, (m[:, 0] + np.log(np.where(l[:, 0] > 0, l[:, 0], 1.0))), -np.inf)
            dP = do[b, :, h] @ v[b, :, kh].T
            dS = P * (dP - (P * dP).sum(axis=1, keepdims=True))
            dq[b, :, h] = sc * dS @ k[b, :, kh]
            dk[b, :, kh] += sc * dS.T @ q[b, :, h]
            dv[b, :, kh] += P.T @ do[b, :, h]
    dqkv = np.concatenate([dq, dk, dv], axis=2).reshape(B, S, -1)
    return o.reshape(B, S, Hq * D), lse, dqkv


CASES = [
    # B, S, Hq, Hkv, D, causal, kv_len
    (1, 1, 1, 1, 64, True, None),
    (2, 23, 4, 2, 64, True, None),
    (1, 31, 4, 1, 128, False, None),
    (2, 19, 2, 2, 64, False, [19, 7]),
    (2, 26, 6, 3, 128, True, [11, 26]),
    (2, 9, 2, 1, 64, False, [0, 4]),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}S{}Hq{}Hkv{}D{}c{}kv{}".format(*c))
@pytest.mark.parametrize("f64", [True, False], ids=["acc64", "acc32"])
def test_oracle_vs_brute_force(case, f64):
    B, S, Hq, Hkv, D, causal, kv_len = case
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f32", seed_qkv=S, seed_do=S + 1)
    o, lse = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=causal, kv_len=kv_len, f64=f64)
    d = oracle.bwd(inp["qkv"], o, inp["dout"], lse, B, S, Hq, Hkv, D, causal=causal, kv_len=kv_len, f64=f64)
    ob, lb, db = brute(inp["qkv"], inp["dout"], B, S, Hq, Hkv, D, causal, kv_len)
    tol = 2e-6 if f64 else 2e-5
    np.testing.assert_allclose(o, ob, rtol=tol, atol=tol)
    np.testing.assert_array_equal(np.isinf(lse), np.isinf(lb))
    np.testing.assert_allclose(lse[np.isfinite(lb)], lb[np.isfinite(lb)], rtol=tol, atol=tol)
    np.testing.assert_allclose(d, db, rtol=10 * tol, atol=10 * tol)


# ------------------------------------------------------------------------ golden (torch)
GOLD_CASES = {
    "cfg1": (2, 128, 4, 4, 64, "f32", True, None, 0, 1),
    "tiny_gqa_causal": (1, 17, 2, 1, 64, "f16", True, None, 5, 6),
    "gqa_kvlen": (2, 40, 4, 2, 128, "f16", False, [40, 23], 7, 8),
    "bf16_causal_kvlen": (2, 33, 3, 3, 64, "bf16", True, [33, 9], 9, 10),
    "s1": (2, 1, 2, 2, 128, "f16", False, None, 11, 12),
}


@pytest.mark.parametrize("name", sorted(GOLD_CASES))
@pytest.mark.parametrize("f64", [True, False], ids=["acc64", "acc32"])
def test_oracle_vs_torch_golden(name, f64):
    gold = np.load(GOLDEN)
    B, S, Hq, Hkv, D, dt, causal, kv_len, s1, s2 = GOLD_CASES[name]
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, dt, seed_qkv=s1, seed_do=s2)
    x = inp["qkv"].astype(np.float64)
    np.testing.assert_allclose([x.sum(), np.abs(x).sum()], gold[f"{name}/qkv_sum"], rtol=1e-12)
    o, lse = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=causal, kv_len=kv_len, f64=f64)
    d = oracle.bwd(inp["qkv"], o, inp["dout"], lse, B, S, Hq, Hkv, D, causal=causal, kv_len=kv_len, f64=f64)
    tol = 1e-5 if f64 else 5e-5
    glse = gold[f"{name}/lse"]
    fin = np.isfinite(glse)
    np.testing.assert_array_equal(np.isfinite(lse), fin)
    np.testing.assert_allclose(lse[fin], glse[fin], rtol=tol, atol=tol)
    for key, arr in (("o", o), ("dqkv", d)):
        if f"{name}/{key}" in gold:
            np.testing.assert_allclose(arr, gold[f"{name}/{key}"], rtol=tol, atol=tol)
        else:
            idx = gold[f"{name}/{key}_idx"]
            np.testing.assert_allclose(arr.reshape(-1)[idx], gold[f"{name}/{key}_val"], rtol=tol, atol=tol)
            hs = arr.reshape(B, S, -1, D).sum(axis=(1, 3))
            np.testing.assert_allclose(hs, gold[f"{name}/{key}_headsum"], rtol=1e-4, atol=1e-3)


# ------------------------------------------------------------------------ closed forms
def test_closed_form_causal_first_row():
    B, S, H, D = 2, 16, 3, 64
    inp = oracle.make_inputs(B, S, H, H, D, "f32", seed_qkv=21)
    o, lse = oracle.fwd(inp["qkv"], B, S, H, H, D, causal=True, f64=True)
    x = inp["qkv"].reshape(B, S, 3 * H, D).astype(np.float64)
    for b in range(B):
        for h in range(H):
            np.testing.assert_allclose(o.reshape(B, S, H, D)[b, 0, h], x[b, 0, 2 * H + h], rtol=1e-6, atol=1e-7)
            assert abs(lse[b, h, 0] - scale_of(D) * x[b, 0, h] @ x[b, 0, H + h]) < 1e-5


def test_closed_form_zero_keys_uniform():
    B, S, H, D = 1, 20, 2, 128
    inp = oracle.make_inputs(B, S, H, H, D, "f32", seed_qkv=22)
    x = inp["qkv"].reshape(B, S, 3 * H, D)
    x[:, :, H:2 * H] = 0.0
    for causal in (True, False):
        o, lse = oracle.fwd(x, B, S, H, H, D, causal=causal, f64=True)
        v = x[0, :, 2 * H:].astype(np.float64)
        for i in range(S):
            n = i + 1 if causal else S
            np.testing.assert_allclose(o.reshape(B, S, H, D)[0, i], v[:n].mean(axis=0), rtol=1e-6, atol=1e-6)
            np.testing.assert_allclose(lse[0, :, i], math.log(n), rtol=1e-7)


def test_closed_form_kv_len_one_and_zero():
    B, S, H, D = 2, 12, 2, 64
    inp = oracle.make_inputs(B, S, H, H, D, "f32", seed_qkv=23)
    o, lse = oracle.fwd(inp["qkv"], B, S, H, H, D, causal=False, kv_len=[1, 0], f64=True)
    d = oracle.bwd(inp["qkv"], o, inp["dout"], lse, B, S, H, H, D, causal=False, kv_len=[1, 0], f64=True)
    x = inp["qkv"].reshape(B, S, 3 * H, D)
    o4 = o.reshape(B, S, H, D)
    for i in range(S):
        np.testing.assert_allclose(o4[0, i], x[0, 0, 2 * H:], rtol=1e-6, atol=1e-7)
    assert np.all(o4[1] == 0.0) and np.all(np.isneginf(lse[1]))
    assert np.all(d.reshape(B, S, 3 * H, D)[1] == 0.0)
    # with one visible key P == 1, so dQ = dK = 0 and dV_0 = sum_i dO_i
    d4 = d.reshape(B, S, 3 * H, D)
    np.testing.assert_allclose(d4[0, :, :2 * H], 0.0, atol=1e-7)
    do = inp["dout"].reshape(B, S, H, D).astype(np.float64)
    np.testing.assert_allclose(d4[0, 0, 2 * H:], do[0].sum(axis=0), rtol=1e-6, atol=1e-6)


# ---------------------------------------------- the reference's order of work with fp16 P
def test_pround_two_keys_closed_form():
    """Two visible keys.  In one 16-key tile the larger score's p is exactly 1 and the other's
    exp(-|ds|) is rounded to fp16 for PV while the row sum keeps it unrounded
    (tkm_gpu.cu:399-409): O = (v_big + r(p) v_small) / (1 + p), LSE = s_big + ln(1 + p).
    With the keys in different tiles (0 and 17, the keys between scored far below) the
    rounding follows the running max: if key 17 scores higher, key 0 was stored with p = 1
    and is rescaled by the unrounded alpha = exp(s_0 - s_17), so O = (alpha v_0 + v_17) /
    (1 + alpha) with no rounding at all; if key 0 scores higher, key 17's p is rounded as in
    one tile."""
    B, S, H, D = 1, 24, 2, 64
    sc = scale_of(D)
    seen = set()
    for kvl, keys in ((2, (0, 1)), (18, (0, 17))):
        inp = oracle.make_inputs(B, S, H, H, D, "f32", seed_qkv=31)
        x = inp["qkv"].reshape(B, S, 3 * H, D).astype(np.float32)
        # every key other than the two: k = -40 q-direction, so its score is hugely negative
        for j in range(S):
            if j not in keys:
                for h in range(H):
                    x[0, j, H + h] = -40.0 * x[0, S - 1, h] / np.linalg.norm(x[0, S - 1, h])
        o, lse = oracle.fwd(x, B, S, H, H, D, causal=False, kv_len=[kvl], p_f16=True)
        o4 = o.reshape(B, S, H, D)
        i = S - 1
        for h in range(H):
            q = x[0, i, h].astype(np.float64)
            (s0, v0), (s1, v1) = [(sc * q @ x[0, j, H + h].astype(np.float64), x[0, j, 2 * H + h].astype(np.float64))
                                  for j in keys]
            p = math.exp(-abs(s1 - s0))
            if kvl == 18 and s1 > s0:          # key 0 stored first with p = 1, then rescaled
                want, seen_case = (p * v0 + v1) / (1.0 + p + 1e-8), "rescaled"
            else:                              # the lower key's p rounded to fp16
                p16 = float(np.float16(np.float32(p)))
                assert p16 != p
                v_hi, v_lo = (v0, v1) if s0 >= s1 else (v1, v0)
                want, seen_case = (v_hi + p16 * v_lo) / (1.0 + p + 1e-8), "rounded"
            seen.add((kvl, seen_case))
            np.testing.assert_allclose(o4[0, i, h], want, rtol=2e-6, atol=2e-7)
            assert abs(lse[0, h, i] - (max(s0, s1) + math.log(1.0 + p + 1e-8))) < 2e-6
    assert seen == {(2, "rounded"), (18, "rounded"), (18, "rescaled")}, seen


def test_pround_uniform_and_single_key():
    """K = 0: every p is exactly 1 in every tile (alpha 1 after the first), so O is the exact
    mean of the visible V over several tiles and LSE = ln(#visible); one visible key gives
    O = v_0."""
    B, S, H, D = 1, 40, 2, 128
    inp = oracle.make_inputs(B, S, H, H, D, "f32", seed_qkv=32)
    x = inp["qkv"].reshape(B, S, 3 * H, D)
    x[:, :, H:2 * H] = 0.0
    o, lse = oracle.fwd(x, B, S, H, H, D, causal=True, p_f16=True)
    v = x[0, :, 2 * H:].astype(np.float64)
    for i in range(S):
        np.testing.assert_allclose(o.reshape(B, S, H, D)[0, i], v[:i + 1].mean(axis=0), rtol=1e-6, atol=1e-6)
        # (the reference's +1e-8 guard on the row sum: ln(n + 1e-8))
        np.testing.assert_allclose(lse[0, :, i], math.log(i + 1), rtol=1e-7, atol=2e-8)
    inp = oracle.make_inputs(2, 12, 2, 2, 64, "f32", seed_qkv=33)
    o, lse = oracle.fwd(inp["qkv"], 2, 12, 2, 2, 64, causal=False, kv_len=[1, 0], p_f16=True)
    o4 = o.reshape(2, 12, 2, 64)
    x = inp["qkv"].reshape(2, 12, 6, 64)
    for i in range(12):
        np.testing.assert_allclose(o4[0, i], x[0, 0, 4:], rtol=1e-6, atol=1e-7)
    assert np.all(o4[1] == 0.0) and np.all(np.isneginf(lse[1]))


@pytest.mark.parametrize("growth", [0.0, 0.05])
def test_pround_within_rounding_of_exact(growth):
    """Against the float64 forward, the only difference is P's fp16 rounding (relative 2^-11
    per term): |O - O_exact| <= 2^-11 max|v| per row, LSE equal to float resolution.  With
    scores growing along the keys (growth > 0) the running max moves every tile, so a wrong
    or missing rescale would break the bound."""
    B, S, Hq, Hkv, D = 2, 160, 4, 2, 128
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f16", seed_qkv=34)
    x = inp["qkv"].reshape(B, S, Hq + 2 * Hkv, D).copy()
    # scores rise with the key index: add growth * j * (q-direction mean) to every key
    qdir = x[:, :, :Hq].mean(axis=(1, 2))
    for j in range(S):
        x[:, j, Hq:Hq + Hkv] += growth * j * qdir[:, None, :] / max(1e-6, float(np.abs(qdir).max()))
    for causal, kvl in ((True, None), (False, [160, 37])):
        o_e, l_e = oracle.fwd(x, B, S, Hq, Hkv, D, causal=causal, kv_len=kvl, f64=True)
        o_p, l_p = oracle.fwd(x, B, S, Hq, Hkv, D, causal=causal, kv_len=kvl, p_f16=True)
        vmax = float(np.abs(x[:, :, Hq + Hkv:]).max())
        err = float(np.abs(o_p - o_e).max())
        assert err <= 2 ** -11 * vmax + 1e-6, err
        assert err > 0.0                       # the rounding is there
        np.testing.assert_allclose(l_p, l_e, rtol=1e-6, atol=1e-5)


# ----------------------------------------------------------------- finite differences
def test_finite_differences_fp64():
    B, S, Hq, Hkv, D = 1, 10, 2, 1, 64
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f32", seed_qkv=31, seed_do=32)
    x = inp["qkv"].astype(np.float64)
    w = inp["dout"].astype(np.float64)
    rng = np.random.default_rng(3)

    def loss(xx):
        o, _ = oracle.fwd(xx.astype(np.float32), B, S, Hq, Hkv, D, causal=True, f64=True)
        return float((o.astype(np.float64) * w).sum())

    o, lse = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=True, f64=True)
    g = oracle.bwd(inp["qkv"], o, inp["dout"], lse, B, S, Hq, Hkv, D, causal=True, f64=True).astype(np.float64)
    for part in range(3):  # directions confined to Q, K and V in turn
        u = np.zeros_like(x).reshape(B, S, Hq + 2 * Hkv, D)
        sl = [slice(0, Hq), slice(Hq, Hq + Hkv), slice(Hq + Hkv, Hq + 2 * Hkv)][part]
        u[:, :, sl] = rng.standard_normal(u[:, :, sl].shape)
        u = u.reshape(x.shape)
        eps = 1e-2
        fd = (loss(x + eps * u) - loss(x - eps * u)) / (2 * eps)
        an = float((g * u).sum())
        assert abs(fd - an) <= 2e-3 * max(1.0, abs(an)), (part, fd, an)


def test_finite_differences_config1():
    """BASELINE config 1 (fp32 B2 H4 S128 D64, causal, Q/K/V seed 0, dO seed 1): the oracle's
    dQ, dK, dV against central differences of L = sum(O * dO) in float64, along random
    directions confined to Q, K and V of each batch, and at 48 single coordinates drawn from
    every part (the first query row, the last key row, a masked-out-early key).  The oracle
    takes and returns fp32, so L carries about 1e-5 of rounding noise: eps = 1e-2 keeps the
    truncation error (~eps^2) and that noise (~1e-5 / eps) below the bars."""
    B, S, Hq, Hkv, D = 2, 128, 4, 4, 64
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f32", seed_qkv=0, seed_do=1)
    x = inp["qkv"].astype(np.float64)
    w = inp["dout"].astype(np.float64)

    def loss(xx):
        o, _ = oracle.fwd(xx, B, S, Hq, Hkv, D, causal=True, f64=True)
        return float((o.astype(np.float64) * w).sum())

    o, lse = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=True, f64=True)
    g = oracle.bwd(inp["qkv"], o, inp["dout"], lse, B, S, Hq, Hkv, D, causal=True,
                   f64=True).astype(np.float64)
    rng = np.random.default_rng(11)
    x4 = x.reshape(B, S, Hq + 2 * Hkv, D)
    parts = [slice(0, Hq), slice(Hq, Hq + Hkv), slice(Hq + Hkv, Hq + 2 * Hkv)]
    eps = 1e-2
    for b in range(B):
        for part in parts:
            u = np.zeros_like(x4)
            u[b, :, part] = rng.standard_normal(u[b, :, part].shape)
            u = u.reshape(x.shape)
            fd = (loss(x + eps * u) - loss(x - eps * u)) / (2 * eps)
            an = float((g * u).sum())
            assert abs(fd - an) <= 2e-3 * max(1.0, abs(an)), (b, part, fd, an)
    coords = [(0, 0, 0, 3), (1, S - 1, Hq, 5), (0, 0, Hq + 1, 7), (1, 64, Hq + Hkv + 2, 1)]
    coords += [(int(rng.integers(B)), int(rng.integers(S)), int(rng.integers(Hq + 2 * Hkv)),
                int(rng.integers(D))) for _ in range(44)]
    g4 = g.reshape(x4.shape)
    for c in coords:
        e = np.zeros_like(x4)
        e[c] = 1.0
        e = e.reshape(x.shape)
        fd = (loss(x + eps * e) - loss(x - eps * e)) / (2 * eps)
        assert abs(fd - g4[c]) <= 1e-4 + 2e-3 * abs(g4[c]), (c, fd, g4[c])


# -------------------------------------------------------------------------- invariants
def test_invariants():
    B, S, H, D = 2, 24, 2, 64
    inp = oracle.make_inputs(B, S, H, H, D, "f32", seed_qkv=41, seed_do=42)
    x = inp["qkv"].reshape(B, S, 3 * H, D).astype(np.float32)
    sc = scale_of(D)
    for causal in (True, False):
        o, lse = oracle.fwd(x, B, S, H, H, D, causal=causal, f64=True)
        d = oracle.bwd(x, o, inp["dout"], lse, B, S, H, H, D, causal=causal, f64=True).reshape(B, S, 3 * H, D)
        # sum_j dS_ij = 0  =>  sum_j dK_j = 0 per kv head
        np.testing.assert_allclose(d[:, :, H:2 * H].sum(axis=1), 0.0, atol=1e-5)
        # key shift: O unchanged, LSE += scale <q_i, c>
        c = np.linspace(-1, 1, D).astype(np.float32)
        xs = x.copy()
        xs[:, :, H:2 * H] += c
        o2, lse2 = oracle.fwd(xs, B, S, H, H, D, causal=causal, f64=True)
        np.testing.assert_allclose(o2, o, atol=1e-5)
        qc = sc * np.einsum("bshd,d->bhs", x[:, :, :H].astype(np.float64), c.astype(np.float64))
        np.testing.assert_allclose(lse2, lse + qc, atol=1e-4)
        # value shift: O += c, dV unchanged
        xv = x.copy()
        xv[:, :, 2 * H:] += c
        o3, lse3 = oracle.fwd(xv, B, S, H, H, D, causal=causal, f64=True)
        np.testing.assert_allclose(o3.reshape(B, S, H, D), o.reshape(B, S, H, D) + c, atol=1e-5)
        d3 = oracle.bwd(xv, o3, inp["dout"], lse3, B, S, H, H, D, causal=causal, f64=True).reshape(B, S, 3 * H, D)
        np.testing.assert_allclose(d3[:, :, 2 * H:], d[:, :, 2 * H:], atol=1e-5)
    # non-causal key/value permutation: O unchanged, dK/dV permuted
    perm = np.random.default_rng(5).permutation(S)
    xp = x.copy()
    xp[:, :, H:] = x[:, perm, H:]
    o, lse = oracle.fwd(x, B, S, H, H, D, causal=False, f64=True)
    op, lsep = oracle.fwd(xp, B, S, H, H, D, causal=False, f64=True)
    np.testing.assert_allclose(op, o, atol=1e-5)
    d = oracle.bwd(x, o, inp["dout"], lse, B, S, H, H, D, causal=False, f64=True).reshape(B, S, 3 * H, D)
    dp = oracle.bwd(xp, op, inp["dout"], lsep, B, S, H, H, D, causal=False, f64=True).reshape(B, S, 3 * H, D)
    np.testing.assert_allclose(dp[:, :, H:], d[:, perm, H:], atol=1e-5)


def test_gqa_equals_repeated_mha():
    B, S, Hq, Hkv, D = 2, 21, 6, 2, 64
    g = Hq // Hkv
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f32", seed_qkv=51, seed_do=52)
    x = inp["qkv"].reshape(B, S, Hq + 2 * Hkv, D)
    xm = np.concatenate([x[:, :, :Hq], np.repeat(x[:, :, Hq:Hq + Hkv], g, axis=2),
                         np.repeat(x[:, :, Hq + Hkv:], g, axis=2)], axis=2)
    for causal in (True, False):
        o, lse = oracle.fwd(x, B, S, Hq, Hkv, D, causal=causal, f64=True)
        om, lsem = oracle.fwd(xm, B, S, Hq, Hq, D, causal=causal, f64=True)
        np.testing.assert_allclose(o, om, atol=1e-6)
        d = oracle.bwd(x, o, inp["dout"], lse, B, S, Hq, Hkv, D, causal=causal, f64=True).reshape(B, S, -1, D)
        dm = oracle.bwd(xm, om, inp["dout"], lsem, B, S, Hq, Hq, D, causal=causal, f64=True).reshape(B, S, -1, D)
        np.testing.assert_allclose(d[:, :, :Hq], dm[:, :, :Hq], atol=1e-6)
        np.testing.assert_allclose(d[:, :, Hq:Hq + Hkv], dm[:, :, Hq:2 * Hq].reshape(B, S, Hkv, g, D).sum(3), atol=1e-5)
        np.testing.assert_allclose(d[:, :, Hq + Hkv:], dm[:, :, 2 * Hq:].reshape(B, S, Hkv, g, D).sum(3), atol=1e-5)


# ---------------------------------------------------------------- planted mistakes
def test_checks_catch_planted_mistakes():
    """Each plausible oracle mistake, planted on the CPU, must fail the brute-force check."""
    B, S, Hq, Hkv, D = 2, 17, 4, 2, 64
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f32", seed_qkv=61, seed_do=62)
    ob, lb, db = brute(inp["qkv"], inp["dout"], B, S, Hq, Hkv, D, True)

    def close(a, b):
        return np.allclose(a, b, rtol=1e-4, atol=1e-4)

    o, lse = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=True, f64=True)
    d = oracle.bwd(inp["qkv"], o, inp["dout"], lse, B, S, Hq, Hkv, D, causal=True, f64=True)
    assert close(o, ob) and close(d, db)
    # wrong scale (1/D instead of 1/sqrt(D))
    o1, _ = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, scale=1.0 / D, causal=True, f64=True)
    assert not close(o1, ob)
    # causal mask dropped
    o2, _ = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=False, f64=True)
    assert not close(o2, ob)
    # K and V heads swapped in the packing
    x = inp["qkv"].reshape(B, S, Hq + 2 * Hkv, D).copy()
    x[:, :, Hq:] = np.concatenate([x[:, :, Hq + Hkv:], x[:, :, Hq:Hq + Hkv]], axis=2)
    o3, _ = oracle.fwd(x, B, S, Hq, Hkv, D, causal=True, f64=True)
    assert not close(o3, ob)
    # wrong GQA head map (h % Hkv instead of h / (Hq/Hkv)) == permuting q-heads' kv partner
    xq = inp["qkv"].reshape(B, S, Hq + 2 * Hkv, D).copy()
    xq[:, :, :Hq] = xq[:, :, [0, 2, 1, 3]]
    o4, _ = oracle.fwd(xq, B, S, Hq, Hkv, D, causal=True, f64=True)
    assert not close(o4.reshape(B, S, Hq, D)[:, :, [0, 2, 1, 3]].reshape(o4.shape), ob)
    # dK and dV swapped, or dK = dQ as in the reference kernel (tkm_gpu.cu:593-594)
    d5 = d.reshape(B, S, Hq + 2 * Hkv, D).copy()
    d5[:, :, Hq:] = np.concatenate([d5[:, :, Hq + Hkv:], d5[:, :, Hq:Hq + Hkv]], axis=2)
    assert not close(d5.reshape(d.shape), db)
    d6 = d.reshape(B, S, Hq + 2 * Hkv, D).copy()
    d6[:, :, Hq:Hq + Hkv] = d6[:, :, 0:Hq:Hq // Hkv]
    assert not close(d6.reshape(d.shape), db)
    # backward fed with LSE off by one unit
    d7 = oracle.bwd(inp["qkv"], o, inp["dout"], lse + 1.0, B, S, Hq, Hkv, D, causal=True, f64=True)
    assert not close(d7, db)


# ----------------------------------------------------------------------------- Drop's generators
def test_drop_xorshift32_known_answer():
    """Generator 1 is Marsaglia's xorshift32 (13, 17, 5) ("Xorshift RNGs", J. Stat. Softw. 2003):
    from y = 2463534242 its first output is 723471715.  rng_init(seed, idx) starts it at
    seed ^ (idx * 0x9E3779B9 + 0x7F4A7C15), so idx 0 and seed = y ^ 0x7F4A7C15 start it at y."""
    got = oracle.rng_u32(1, 2463534242 ^ 0x7F4A7C15, 0, 3)
    assert int(got[0]) == 723471715
    y, want = 2463534242, []
    for _ in range(3):
        y ^= (y << 13) & 0xFFFFFFFF
        y ^= y >> 17
        y ^= (y << 5) & 0xFFFFFFFF
        want.append(y)
    assert [int(v) for v in got] == want


def test_drop_pcg32_is_pcg32_srandom():
    """Generator 3 (what the shipped models select with `prng: pcg32`) is
    pcg32_srandom(seed ^ 0x853C49E6748FEA9B, idx); the oracle's PCG32 stream is pinned to
    O'Neill's demo vector above."""
    for seed, idx in ((0, 0), (1234, 77), (0x13579BDF, 123456)):
        got = oracle.rng_u32(3, seed, idx, 8)
        want = oracle.pcg32_sequence(seed ^ 0x853C49E6748FEA9B, idx, 8)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("rng_type", [1, 2, 3, 4])
def test_drop_generators_match_the_reference(rng_type):
    """All four generators, bit for bit, against the reference's own generator code
    (src/tkm_gpu.cu:751-794, run on the GPU by oracle/ref_rng_harness.hip; vectors written by
    tests/golden/make_rng_vectors.py): 80 streams (seeds 0, 1, 2^32-1, the runtime's Drop
    seeds and others; stream indices up to 2^32-1) x 16 draws of rng_u32, and rng_uniform's
    24-bit float of each draw.  Generator 2 (Wang hash + xorshift32) is the front end's
    default when a model names no `prng` (src/tkm_core.c:252)."""
    v = np.load(os.path.join(HERE, "golden", "rng_vectors.npz"))
    u32 = v[f"u32_{rng_type}"]
    for k in range(v["seeds"].size):
        got = oracle.rng_u32(rng_type, int(v["seeds"][k]), int(v["idxs"][k]), u32.shape[1])
        assert np.array_equal(np.asarray(got, np.uint32), u32[k]), (rng_type, k)
    uni = (u32 >> 8).astype(np.float32) * np.float32(1.0 / 16777216.0)
    assert np.array_equal(uni, v[f"uni_{rng_type}"])


@pytest.mark.parametrize("rng_type", [1, 2, 3, 4])
def test_drop_keep_rate_and_pairs(rng_type):
    """The keep fraction is 1 - p within 5 sigma for every generator, and the two channels of a
    pair come from consecutive draws of one stream."""
    rows, C, p = 256, 64, 0.3
    keep = oracle.drop_keep(rows, C, 0x13579BDF, 17, rng_type, p)
    n = keep.size
    assert abs(keep.mean() - (1 - p)) < 5 * np.sqrt(p * (1 - p) / n)
    sd = (0x13579BDF ^ (17 * 19937 + 1)) & 0xFFFFFFFF
    for r, t in ((0, 0), (3, 5), (255, 31)):
        u = (oracle.rng_u32(rng_type, sd, r * (C // 2) + t, 2) >> 8).astype(np.float64) / 16777216.0
        assert list(keep[r, 2 * t:2 * t + 2]) == [int(v < 1 - p) for v in u]
    # another node or step seed gives another mask
    assert not np.array_equal(keep, oracle.drop_keep(rows, C, 0x13579BDF, 18, rng_type, p))
    assert not np.array_equal(keep, oracle.drop_keep(rows, C, 0x13579BDF + 0x9E3779B9, 17, rng_type, p))

"""Shared helpers for the attention parity tests: seeded inputs, upload, comparison.

Tolerances (element-wise, numpy allclose form |x - ref| <= atol + rtol*|ref|):
  O, LSE      : atol 2e-3, rtol 1e-2
  dQ, dK, dV  : atol 5e-3, rtol 2e-2
against the CPU oracle run on the same rounded inputs.
"""
from __future__ import annotations

import sys

import numpy as np

import oracle
from parity_checks import compare  # noqa: F401  (NaN-safe; re-exported for the tests)

TOL_FWD = (2e-3, 1e-2)
TOL_BWD = (5e-3, 2e-2)


def log(msg: str) -> None:
    print(msg, flush=True)
    sys.stdout.flush()


def to_device(bits: np.ndarray, dtype: str, device):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16))
    return t.view(torch.float16 if dtype == "f16" else torch.bfloat16).to(device)


def from_device(t) -> np.ndarray:
    import torch
    return t.detach().to(torch.float32).cpu().numpy()


def split_dqkv(dqkv: np.ndarray, B, S, Hq, Hkv, D):
    x = dqkv.reshape(B, S, Hq + 2 * Hkv, D)
    return x[:, :, :Hq], x[:, :, Hq:Hq + Hkv], x[:, :, Hq + Hkv:]


def run_gpu_case(device, B, S, Hq, Hkv, D, dtype="f16", causal=True, kv_len=None, mul=1.0,
                 bwd=True, seed=0, f64=None, transform=None):
    """Runs the HIP forward (and backward) and the oracle; returns a list of compare() stats."""
    import torch
    from tokamak_amd import attn

    tag = f"B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} {dtype} causal={int(causal)} kv_len={kv_len} seed={seed}"
    log(f"[case] {tag}")
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, dtype, seed_qkv=seed, seed_do=seed + 1, mul=mul,
                             with_dout=bwd, transform=transform)
    qkv = to_device(inp["qkv_bits"], dtype, device)
    kvl = None if kv_len is None else torch.tensor(kv_len, dtype=torch.int32, device=device)
    o, lse = attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=causal, kv_len=kvl)
    if f64 is None:
        f64 = B * Hq * S * S * D < 2e9
    o_ref, lse_ref = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=causal, kv_len=kv_len, f64=f64)
    res = [compare("O", from_device(o), o_ref, TOL_FWD), compare("LSE", from_device(lse), lse_ref, TOL_FWD)]
    if bwd:
        dout = to_device(inp["dout_bits"], dtype, device)
        dqkv = attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, causal=causal, kv_len=kvl)
        torch.cuda.synchronize()
        o_stored, _ = oracle.round_to(o_ref, dtype)  # the O a 16-bit forward stores
        d_ref = oracle.bwd(inp["qkv"], o_stored, inp["dout"], lse_ref, B, S, Hq, Hkv, D,
                           causal=causal, kv_len=kv_len, f64=f64)
        got = split_dqkv(from_device(dqkv), B, S, Hq, Hkv, D)
        ref = split_dqkv(d_ref, B, S, Hq, Hkv, D)
        for nm, g, r in zip(("dQ", "dK", "dV"), got, ref):
            res.append(compare(nm, g, r, TOL_BWD))
    for st in res:
        log(f"    {st['name']:>3}: max_abs={st['max_abs']:.3e} max_rel={st['max_rel']:.3e} "
            f"bad={st['n_bad']}/{st['n']}" + (f" e.g. {st.get('examples')}" if st["n_bad"] else ""))
    return res


def gradient_term_rms(qkv, o_stored, dout, lse, B, S, Hq, Hkv, D, causal=True, kv_len=None,
                      scale=None):
    """Root of the sum of squares of the terms each gradient element sums (float64, from the
    oracle's state): dV_jd = sum_i P_ij dO_id, dK_jd = scale sum_i dS_ij q_id (both over the
    q-heads of the kv group), dQ_id = scale sum_j dS_ij k_jd.  A 16-bit kernel rounds P and dS
    to its storage type before these products (as the reference rounds P and dS,
    tkm_gpu.cu:402, 552), so each term carries an independent relative error of about one
    rounding unit u, and the sum's error is of order u * sqrt(sum of squared terms), whatever
    the sum's own size: the scale of the rounding error where the terms cancel.  Small shapes
    only (S x S per head)."""
    scale = 1.0 / np.sqrt(np.float32(D)) if scale is None else scale
    g = Hq // Hkv
    x = qkv.reshape(B, S, Hq + 2 * Hkv, D).astype(np.float64)
    o = o_stored.reshape(B, S, Hq, D).astype(np.float64)
    do = dout.reshape(B, S, Hq, D).astype(np.float64)
    rq = np.zeros((B, S, Hq, D))
    rk = np.zeros((B, S, Hkv, D))
    rv = np.zeros((B, S, Hkv, D))
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    for b in range(B):
        kvl = S if kv_len is None else max(0, min(int(kv_len[b]), S))
        vis = (j < kvl) & ((j <= i) if causal else True)
        for h in range(Hq):
            kh = h // g
            q, k, v = x[b, :, h], x[b, :, Hq + kh], x[b, :, Hq + Hkv + kh]
            L = lse[b, h].astype(np.float64)[:, None]
            with np.errstate(invalid="ignore", over="ignore"):
                P = np.where(vis, np.exp(scale * (q @ k.T) - np.where(np.isfinite(L), L, 0.0)), 0.0)
            dP = do[b, :, h] @ v.T
            Dv = (o[b, :, h] * do[b, :, h]).sum(axis=1, keepdims=True)
            dS = P * (dP - Dv)
            rv[b, :, kh] += (P ** 2).T @ (do[b, :, h] ** 2)
            rk[b, :, kh] += scale ** 2 * (dS ** 2).T @ (q ** 2)
            rq[b, :, h] = scale ** 2 * (dS ** 2) @ (k ** 2)
    return np.sqrt(rq), np.sqrt(rk), np.sqrt(rv)


def fp16_forward_repeats(qkv, B, S, Hq, Hkv, D, causal):
    """The fp16 D = 128 assembly forward's overflow test (tokamak_amd/asmgen/attn_fwd.py:
    overflow_vote), evaluated on the CPU for every item (b, h, block of
    256 query rows): per row, m = max over the item's first tile (keys 0..63, visible ones) of
    s' = (q . k) * sl2 (fp32, sl2 = scale * log2 e); for every tile, each lane sums exp2(s' - m) over its 32 keys
    of the tile (the keys whose index mod 8 is in the lane's half); the item repeats if any
    such sum reaches 65504.  Returns (number of items, items that repeat, largest
    max_j(s') - m over all rows in log2 units; the repeat needs about 16)."""
    sl2 = np.float32(np.float32(1.0) / np.sqrt(np.float32(D)) * np.float32(1.4426950408889634))
    x = qkv.reshape(B, S, Hq + 2 * Hkv, D)
    g = Hq // Hkv
    n_items = n_redo = 0
    growth = -np.inf
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    vis = (j <= i) if causal else np.ones((S, S), bool)
    half = (np.arange(S) % 8) // 4          # the lane half that holds key j
    tile = np.arange(S) // 64
    nt = (S + 63) // 64
    for b in range(B):
        for h in range(Hq):
            q = x[b, :, h].astype(np.float32)
            k = x[b, :, Hq + h // g].astype(np.float32)
            s = (q @ k.T) * sl2                                   # fp32, log2 units
            s = np.where(vis, s, -np.inf)
            first = np.where(tile[None, :] == 0, s, -np.inf).max(axis=1)
            m = np.where(np.isfinite(first), first, 0.0)
            growth = max(growth, float(np.nanmax(np.where(vis, s - m[:, None], -np.inf))))
            with np.errstate(over="ignore"):
                p = np.where(vis, np.exp2(np.minimum(s - m[:, None], 126.0)), 0.0)
            sums = np.zeros((S, nt, 2))
            np.add.at(sums, (slice(None), tile, half), p)       # per row, tile, lane half
            bad_row = (sums >= 65504.0).any(axis=(1, 2))
            for z in range((S + 255) // 256):
                n_items += 1
                n_redo += bool(bad_row[256 * z:256 * z + 256].any())
    return n_items, n_redo, growth

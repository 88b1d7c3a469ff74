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


def fp16_forward_rescales(qkv, B, S, Hq, Hkv, D, causal, threshold=None):
    """The D = 128 assembly forwards' lazy rescale (tokamak_amd/asmgen/attn_fwd.py:
    rescale_test, rescale_if), evaluated on the CPU.  Per wave (64 query rows of one q-head):
    m_row starts as the row max over the first 64-key tile of s' = (q . k) * sl2 (fp32, log2
    units, visible keys only; 0 for a row with none there); each later tile the wave uses is
    tested, and if any of the wave's rows has a visible s' above m_row + threshold, every row
    takes m_row = max(m_row, its max over the tile).  Returns (tiles tested, tiles rescaled,
    largest max_j(s') - (first tile's max) over all rows, in log2 units).  The threshold is the
    kernel's RESCALE_LOG2 unless given."""
    if threshold is None:
        from tokamak_amd.asmgen.attn_fwd import RESCALE_LOG2 as threshold
    sl2 = np.float32(np.float32(1.0) / np.sqrt(np.float32(D)) * np.float32(1.4426950408889634))
    x = qkv.reshape(B, S, Hq + 2 * Hkv, D)
    g = Hq // Hkv
    tested = rescaled = 0
    growth = -np.inf
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    vis = (j <= i) if causal else np.ones((S, S), bool)
    nt = (S + 63) // 64
    for b in range(B):
        for h in range(Hq):
            q = x[b, :, h].astype(np.float32)
            k = x[b, :, Hq + h // g].astype(np.float32)
            s = np.where(vis, (q @ k.T) * sl2, -np.inf)            # fp32, log2 units
            tmax = np.stack([s[:, 64 * t:64 * t + 64].max(axis=1) for t in range(nt)], axis=1)
            m0 = np.where(np.isfinite(tmax[:, 0]), tmax[:, 0], 0.0)
            growth = max(growth, float(np.max(np.where(np.isfinite(tmax), tmax - m0[:, None], -np.inf))))
            for r0 in range(0, S, 64):
                m = m0[r0:r0 + 64].copy()
                last = min(nt, r0 // 64 + 1) if causal else nt
                for t in range(1, last):
                    tm = tmax[r0:r0 + 64, t]
                    tested += 1
                    if np.any(tm > m + threshold):
                        rescaled += 1
                        m = np.maximum(m, tm)
    return tested, rescaled, growth

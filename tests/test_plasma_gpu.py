"""GPU parity of the generated plasma epilogues (hipRTC, launched through include/tkm_plasma.h)
against the CPU oracle oracle/plasma_ref.c.

Bars, element-wise against the oracle on the same rounded inputs:
  out, xhat, din, dbranch (16-bit)  |gpu - ref| <= 2 ulp of the storage type at |ref| + 1e-4 * max(1, |ref|max)
  istd (fp32)                       relative 1e-5
  parameter gradients (fp32 sums)   |gpu - ref| <= 1e-4 * |ref| + 1e-6 * rows * max(1, |ref|max)
The oracle computes in double and rounds once.  The kernels compute in fp32 with the
registry's fast intrinsics (__expf, __sinf, tanhf, ...), and a chain of up to 8 ops
accumulates a few fp32 ulps before the final rounding, hence 2 ulps.  The backward is
checked on the state the GPU forward saved (xhat, istd).
"""
import numpy as np
import pytest

import oracle
from attn_cases import from_device, log, to_device
from parity_checks import check16_mask

pytestmark = pytest.mark.gpu


def check16(name, got, ref, dtype):
    bad = check16_mask(got, ref, dtype, n_ulp=2, rel_floor=1e-4)
    fin = np.isfinite(np.asarray(ref, np.float64))   # matching infinities are checked by the mask
    diff = np.abs(np.asarray(got, np.float64)[fin] - np.asarray(ref, np.float64)[fin])
    log(f"    {name}: max_abs={np.nanmax(diff, initial=0.0):.3e} n_bad={int(bad.sum())}/{bad.size}")
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        pytest.fail(f"{name}: {int(bad.sum())} elements off, e.g. {i}: gpu {got[i]} ref {ref[i]}")


CHAINS = [
    dict(C=512, chain=["Bias", "Add", "RMSNorm"], acc=7),
    dict(C=64, chain=["RMSNorm", ("SoftCap", 4.0), "LayerScale"], acc=7),
    dict(C=96, chain=["LN", "GELU", "DyT", "PReLU", "xATLU"], acc=0),
    dict(C=24, chain=["Bias", "L2Norm", "Mish", ("Snake", 1.2), "Softplus", "BN"], acc=3),
    dict(C=128, chain=["SiLU", "ReLU2", ("LeakyReLU", 0.1), "ELU", "HardSwish", "HardSigmoid", "Tanh", "Sigmoid"],
         acc=1),
    dict(C=64, chain=[("SwishBeta", 1.5), ("Sin", 1.3), "CosGate", ("Clamp", 1.5), ("Scale", 0.7), "ReLU", "Add"],
         acc=4),
    dict(C=1536, twin=True, left=["SiLU"], right=[], chain=[("Scale", 0.5), "Add"], acc=6),
    dict(C=64, twin=True, left=["Bias", "GELU"], right=["Bias", "LayerScale"], chain=["RMSNorm"], acc=2),
    dict(C=32, twin=True, left=["Sigmoid"], right=["Tanh"], chain=[], acc=0),
    # a Drop between a gate and a residual add that a norm closes (exotic_llama's group shape)
    dict(C=512, chain=["Bias", ("DyT", 0.5), ("Drop", 0.1, 3, 131), "Add", "RMSNorm"], acc=7),
    dict(C=64, twin=True, left=["Bias", ("Drop", 0.2, 1, 7)], right=["SiLU"], chain=[("Drop", 0.3, 4, 9), "LN"], acc=3),
    # Softplus past ln(FLT_MAX): the reference's float formula gives +inf there, as this build does
    dict(C=64, chain=[("Scale", 100.0), "Softplus"], acc=0),
]


DROP_SEED = 0x2468ACE1


def _nodes(c):
    from tokamak_amd import plasma
    def norm(lst):
        return [(x, None) if isinstance(x, str) else tuple(x[:2]) for x in lst]
    items = (norm(c["left"]) + norm(c["right"]) + norm(c["chain"])) if c.get("twin") else norm(c["chain"])
    L = plasma.lib()
    return [(plasma.OPS[n], float(L.tkm_plasma_default_fval(plasma.OPS[n])) if fv is None else float(fv))
            for n, fv in items]


def run_chain(dev, c, rows, dtype, seed, guard=False):
    """One chain's forward and backward against the oracle.  guard: every tensor is moved into
    an all-ones (NaN) guarded buffer, the forward's outputs and the backward workspace start
    as NaN, and the guards must be intact after each call."""
    import torch
    from tokamak_amd import plasma
    C, twin = c["C"], bool(c.get("twin"))
    nl, nr = (len(c["left"]), len(c["right"])) if twin else (0, 0)
    acc = c["acc"]
    log(f"[case] plasma C{C} twin={int(twin)} chain={c.get('left', [])}|{c.get('right', [])}|{c['chain']} "
        f"{dtype} rows={rows} acc={acc} seed={seed}")
    nodes = _nodes(c)
    items = (list(c["left"]) + list(c["right"]) + list(c["chain"])) if twin else list(c["chain"])
    P = plasma.Plasma(C, c["chain"], twin, c.get("left", ()), c.get("right", ()), dtype, group_id=seed)
    rng = np.random.default_rng(seed)
    W = 2 * C if twin else C
    x_r, x_b = oracle.round_to(rng.standard_normal((rows, W)).astype(np.float32), dtype)
    g_r, g_b = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
    t16 = torch.float16 if dtype == "f16" else torch.bfloat16
    params, tens = {}, {"in": to_device(x_b, dtype, dev), "dout": to_device(g_b, dtype, dev)}
    NG = (C + 63) // 64
    for k, (op, _) in enumerate(nodes):
        fl = oracle.plasma_flags(op)
        for key, bit, scale in (("w", oracle.PR_W, 0.3), ("beta", oracle.PR_BETA, 0.2), ("bias", oracle.PR_BIAS, 0.2)):
            if fl & bit:
                a = ((1.0 if key == "w" else 0.0) + scale * rng.standard_normal(C)).astype(np.float32)
                params[(key, k)] = a
                tens[(key, k)] = torch.from_numpy(a).to(dev)
        if fl & oracle.PR_BRANCH:
            b_r, b_b = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
            params[("branch", k)] = b_r
            tens[("branch", k)] = to_device(b_b, dtype, dev)
            p_r, p_b = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
            params[("dbranch_prev", k)] = p_r
            tens[("dbranch", k)] = to_device(p_b, dtype, dev)
        if fl & oracle.PR_MASK:
            _, p, rng_type, node_id = items[k]
            params[("keep", k)] = oracle.drop_keep(rows, C, DROP_SEED, node_id, rng_type, p)
            tens[("mask", k)] = torch.zeros(rows * C, dtype=torch.uint8, device=dev)
            tens[("seed", k)] = torch.from_numpy(np.array([DROP_SEED], np.uint32).view(np.int32)).to(dev)
        if fl & oracle.PR_NORM:
            tens[("xhat", k)] = torch.empty((rows, C), dtype=t16, device=dev)
            tens[("istd", k)] = torch.empty((rows, NG), dtype=torch.float32, device=dev)
        for key, bit in (("dw", oracle.PR_W), ("dbeta", oracle.PR_BETA), ("dbias", oracle.PR_BIAS)):
            if fl & bit:
                prev = (0.1 * rng.standard_normal(C)).astype(np.float32)
                params[(key + "_prev", k)] = prev
                tens[(key, k)] = torch.from_numpy(prev).to(dev)
    tens["out"] = torch.empty((rows, C), dtype=t16, device=dev)
    dp_r, dp_b = oracle.round_to(rng.standard_normal((rows, W)).astype(np.float32), dtype)
    tens["din"] = to_device(dp_b, dtype, dev)

    guards, ws = [], None
    if guard:
        from guarded import Guarded
        fwd_outs = {k for k in tens if k == "out" or (isinstance(k, tuple) and k[0] in ("xhat", "istd", "mask"))}
        for k, v in list(tens.items()):
            g = Guarded(v.numel(), v.dtype, dev)
            if k not in fwd_outs:
                g.t.copy_(v.reshape(-1))
            tens[k] = g.t.view(v.shape)
            guards.append(g)
        ws = Guarded(max(P.bwd_workspace_bytes(rows), 1), torch.uint8, dev)
        guards.append(ws)
    P.fwd(tens, rows)
    torch.cuda.synchronize()
    assert all(g.intact() for g in guards)
    plain = {k: v for k, v in params.items() if k[0] in ("w", "beta", "bias", "branch", "keep")}
    ro, rxh, ris = oracle.plasma_fwd(x_r, rows, C, nodes, plain, twin, nl, nr, dtype)
    check16("out", from_device(tens["out"]), ro, dtype)
    gxh, gis = {}, {}
    for k in rxh:
        check16(f"xhat{k}", from_device(tens[("xhat", k)]), rxh[k], dtype)
        gis[k] = tens[("istd", k)].cpu().numpy()
        np.testing.assert_allclose(gis[k], ris[k], rtol=1e-5)
        gxh[k] = from_device(tens[("xhat", k)])

    P.bwd(tens, rows, acc, workspace=None if ws is None else ws.t)
    torch.cuda.synchronize()
    assert all(g.intact() for g in guards)
    din, dbr, grads = oracle.plasma_bwd(
        g_r, x_r, rows, C, nodes, plain, gxh, gis, twin, nl, nr, dtype, acc_flags=acc, din_prev=dp_r,
        dbranch_prev={k[1]: v for k, v in params.items() if k[0] == "dbranch_prev"},
        grads_prev={(k[0][:-5], k[1]): v for k, v in params.items() if k[0].endswith("_prev") and k[0] != "dbranch_prev"})
    check16("din", from_device(tens["din"]), din, dtype)
    for k, v in dbr.items():
        check16(f"dbranch{k}", from_device(tens[("dbranch", k)]), v, dtype)
    for (kind, k), ref in grads.items():
        got = tens[(kind, k)].cpu().numpy().astype(np.float64)
        bound = 1e-4 * np.abs(ref) + 1e-6 * rows * max(1.0, float(np.abs(ref).max()))
        diff = np.abs(got - ref)
        log(f"    {kind}{k}: max_abs={diff.max():.3e}")
        assert np.all(diff <= bound), (kind, k, float(diff.max()))
    P.close()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("ci", range(len(CHAINS)), ids=lambda i: f"chain{i}_C{CHAINS[i]['C']}")
def test_plasma_chain_parity(gpu, ci, dtype):
    rows = {512: 300, 1536: 130}.get(CHAINS[ci]["C"], 777)
    run_chain(gpu, CHAINS[ci], rows, dtype, seed=ci + 1)


@pytest.mark.parametrize("ci", [0, 3, 6, 9, 10], ids=lambda i: f"chain{i}_C{CHAINS[i]['C']}")
def test_plasma_guarded_buffers(gpu, ci):
    """The chains' kernels write nothing outside their tensors and every forward output and
    workspace byte they own (tests/guarded.py); results as in test_plasma_chain_parity."""
    run_chain(gpu, CHAINS[ci], 131, "f16" if ci % 2 else "bf16", 100 + ci, guard=True)


def test_plasma_config4_pre_attention(gpu):
    """Config 4's residual + pre-norm group (d_model 512, 4096 rows): Add then RMSNorm (F7 groups)."""
    run_chain(gpu, dict(C=512, chain=["Add", "RMSNorm"], acc=7), 4096, "f16", seed=40)


def test_plasma_config4_swiglu(gpu):
    """Config 4's gated FFN epilogue: SiLU(gate) * up over 4096 rows of 2 x 1536."""
    run_chain(gpu, dict(C=1536, twin=True, left=["SiLU"], right=[], chain=[], acc=2), 4096, "f16", seed=41)


def test_plasma_deterministic(gpu):
    import torch
    from tokamak_amd import plasma
    C, rows = 512, 1000
    P = plasma.Plasma(C, ["Bias", "RMSNorm", "LayerScale"])
    rng = np.random.default_rng(0)
    _, xb = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), "f16")
    _, gb = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), "f16")
    t = {"in": to_device(xb, "f16", gpu), "dout": to_device(gb, "f16", gpu),
         "out": torch.empty((rows, C), dtype=torch.float16, device=gpu),
         "din": torch.empty((rows, C), dtype=torch.float16, device=gpu),
         ("bias", 0): torch.zeros(C, device=gpu), ("w", 1): torch.ones(C, device=gpu),
         ("w", 2): torch.full((C,), 0.5, device=gpu),
         ("xhat", 1): torch.empty((rows, C), dtype=torch.float16, device=gpu),
         ("istd", 1): torch.empty((rows, 8), device=gpu),
         ("dbias", 0): torch.empty(C, device=gpu), ("dw", 1): torch.empty(C, device=gpu),
         ("dw", 2): torch.empty(C, device=gpu)}
    runs = []
    for _ in range(2):
        P.fwd(t, rows)
        P.bwd(t, rows, 0)
        torch.cuda.synchronize()
        runs.append({k: v.clone() for k, v in t.items()})
    for k in runs[0]:
        assert torch.equal(runs[0][k], runs[1][k]), k
    P.close()


@pytest.mark.parametrize("rng_type", [1, 2, 3, 4])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_plasma_drop_parity(gpu, rng_type, dtype):
    """Drop inside a chain (Bias, Drop, Add): the keep bits the kernel draws from the step seed,
    the node id and the generator equal oracle.drop_keep's bit for bit (a flipped bit moves an
    element by x / (1 - p), far outside the 2-ulp bar); the backward reuses the saved mask."""
    import torch
    from tokamak_amd import plasma
    C, rows, p, node, seed = 192, 333, 0.25, 41, 0x13579BDF
    log(f"[case] plasma Drop rng_type={rng_type} {dtype} C{C} rows={rows}")
    P = plasma.Plasma(C, ["Bias", ("Drop", p, rng_type, node), "Add"], dtype=dtype, group_id=rng_type)
    assert ("mask", 1) in P.fwd_args and ("seed", 1) in P.fwd_args and ("mask", 1) in P.bwd_args
    rng = np.random.default_rng(rng_type)
    x_r, x_b = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
    b_r, b_b = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
    g_r, g_b = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
    bias = (0.2 * rng.standard_normal(C)).astype(np.float32)
    t16 = torch.float16 if dtype == "f16" else torch.bfloat16
    tens = {"in": to_device(x_b, dtype, gpu), "dout": to_device(g_b, dtype, gpu), ("branch", 2): to_device(b_b, dtype, gpu),
            ("bias", 0): torch.from_numpy(bias).to(gpu), ("mask", 1): torch.zeros(rows * C, dtype=torch.uint8, device=gpu),
            ("seed", 1): torch.from_numpy(np.array([seed], np.uint32).view(np.int32)).to(gpu),
            "out": torch.empty((rows, C), dtype=t16, device=gpu), "din": torch.empty((rows, C), dtype=t16, device=gpu),
            ("dbranch", 2): torch.zeros((rows, C), dtype=t16, device=gpu), ("dbias", 0): torch.zeros(C, device=gpu)}
    P.fwd(tens, rows)
    P.bwd(tens, rows, 0)
    torch.cuda.synchronize()
    keep = oracle.drop_keep(rows, C, seed, node, rng_type, p)
    nodes = [(plasma.OPS["Bias"], 0.0), (plasma.OPS["Drop"], p), (plasma.OPS["Add"], 0.0)]
    params = {("bias", 0): bias, ("keep", 1): keep, ("branch", 2): b_r}
    ro, _, _ = oracle.plasma_fwd(x_r, rows, C, nodes, params, dtype=dtype)
    check16("out", from_device(tens["out"]), ro, dtype)
    din, dbr, grads = oracle.plasma_bwd(g_r, x_r, rows, C, nodes, params, {}, {}, dtype=dtype, acc_flags=0)
    check16("din", from_device(tens["din"]), din, dtype)
    check16("dbranch2", from_device(tens[("dbranch", 2)]), dbr[2], dtype)
    got = tens[("dbias", 0)].cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - grads[("dbias", 0)]) <= 1e-4 * np.abs(grads[("dbias", 0)]) + 1e-6 * rows)
    # the dropped elements: din is exactly zero where keep is 0
    assert np.all(from_device(tens["din"])[keep == 0] == 0)
    frac = keep.mean()
    log(f"    kept {frac:.4f} (1 - p = {1 - p})")
    P.close()

"""Plasma epilogues (chains of row-wise ops behind a GEMM) without a GPU.

1. The CPU oracle (oracle/plasma_ref.c) is pinned by
   - central differences of every op's forward against its backward (input and weight);
   - torch's functional forms of the ops that have one (silu, gelu-tanh, mish, hardswish, ...);
   - whole chains (plain, twin, residual Add, F7 group norms) against float64 torch autograd;
   - the F7 rule itself: for C <= 64 the norms equal torch's rms_norm / layer_norm; for
     C > 64 the statistics are per 64-channel group divided by C, which differs from a
     full-row norm;
   - planted mistakes that these checks must catch.
2. The op numbering and parameter flags agree between the product (include/tkm_plasma.h)
   and the oracle; every op, in plain and twin chains, emits HIP that hipRTC compiles for
   gfx950 without spills or scratch.
3. The C ABI rejects bad descriptors.
"""
import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import oracle
from tokamak_amd import plasma, prep

RNG = np.random.default_rng(77)
OPS = plasma.OPS
POINTWISE = [n for n in plasma.OP_NAMES
             if n not in ("RMSNorm", "LN", "BN", "L2Norm", "Add", "Drop") + plasma.FORMULA_OPS]


# ---- op table ----------------------------------------------------------------------------

def test_op_numbering_and_flags_agree():
    assert len(plasma.OP_NAMES) == 33
    want = {"Bias": oracle.PR_BIAS, "RMSNorm": oracle.PR_W | oracle.PR_NORM,
            "LN": oracle.PR_W | oracle.PR_BETA | oracle.PR_NORM, "BN": oracle.PR_W | oracle.PR_BETA | oracle.PR_NORM,
            "L2Norm": oracle.PR_NORM, "LayerScale": oracle.PR_W, "DyT": oracle.PR_W, "PReLU": oracle.PR_W,
            "xATLU": oracle.PR_W, "Add": oracle.PR_BRANCH, "Drop": oracle.PR_MASK}
    for name, code in OPS.items():
        if name not in plasma.FORMULA_OPS:
            assert oracle.plasma_flags(code) == want.get(name, 0), name
    # defaults of the registry (src/tkm_registry.c)
    L = plasma.lib()
    defaults = {"BN": 1e-2, "LN": 1e-5, "RMSNorm": 1e-5, "L2Norm": 1e-5, "LeakyReLU": 0.01, "ELU": 1.0,
                "SwishBeta": 1.5, "Sin": 1.0, "SoftCap": 30.0, "Clamp": 6.0, "Scale": 1.0, "LayerScale": 1e-4,
                "DyT": 0.5, "PReLU": 0.25, "xATLU": 0.5, "Snake": 1.0, "SiLU": 0.0, "Drop": 0.1}
    for name, v in defaults.items():
        assert L.tkm_plasma_default_fval(OPS[name]) == pytest.approx(v, rel=1e-7), name


# ---- per-op pins -------------------------------------------------------------------------

FV = {"LeakyReLU": 0.01, "ELU": 1.0, "SwishBeta": 1.5, "Sin": 1.3, "SoftCap": 4.0, "Clamp": 1.5, "Scale": 0.7,
      "DyT": 0.5, "PReLU": 0.25, "Snake": 1.2}


@pytest.mark.parametrize("name", POINTWISE)
def test_op_derivative_matches_central_difference(name):
    op, fv = OPS[name], FV.get(name, 0.0)
    xs = RNG.uniform(-4, 4, 40)
    w = 0.8
    h = 1e-6
    for x in xs:
        if name in ("ReLU", "ReLU2", "LeakyReLU", "ELU", "PReLU") and abs(x) < 1e-3:
            continue
        if name in ("HardSwish", "HardSigmoid") and min(abs(x - 3), abs(x + 3)) < 1e-3:
            continue
        if name == "Clamp" and abs(abs(x) - fv) < 1e-3:
            continue
        d, dw = oracle.plasma_op_grad(op, fv, x, w)
        fd = (oracle.plasma_op(op, fv, x + h, w, 0.3) - oracle.plasma_op(op, fv, x - h, w, 0.3)) / (2 * h)
        assert abs(d - fd) < 1e-6 * max(1.0, abs(fd)), (name, x, d, fd)
        fdw = (oracle.plasma_op(op, fv, x, w + h, 0.3) - oracle.plasma_op(op, fv, x, w - h, 0.3)) / (2 * h)
        assert abs(dw - fdw) < 1e-6 * max(1.0, abs(fdw)), (name, x, dw, fdw)


def test_ops_match_torch_functional():
    import torch
    import torch.nn.functional as F
    x = torch.linspace(-6, 6, 241, dtype=torch.float64)
    ref = {
        "SiLU": F.silu(x), "ReLU": F.relu(x), "LeakyReLU": F.leaky_relu(x, 0.01), "ELU": F.elu(x, 1.0),
        "GELU": F.gelu(x, approximate="tanh"), "Mish": F.mish(x), "HardSwish": F.hardswish(x),
        "HardSigmoid": F.hardsigmoid(x), "Tanh": torch.tanh(x), "Sigmoid": torch.sigmoid(x),
        "Softplus": F.softplus(x), "Clamp": torch.clamp(x, -1.5, 1.5),
    }
    for name, r in ref.items():
        got = np.array([oracle.plasma_op(OPS[name], FV.get(name, 0.0), float(v)) for v in x])
        # the registry's GELU constant 0.79788456 rounds sqrt(2/pi) at 8 digits
        tol = 1e-8 if name == "GELU" else 1e-12
        np.testing.assert_allclose(got, r.numpy(), rtol=tol, atol=tol, err_msg=name)


# ---- chains against float64 autograd ---------------------------------------------------------

def _torch_op(name, x, fv, w, b):
    import torch
    import torch.nn.functional as F
    return {
        "Bias": lambda: x + b, "SiLU": lambda: F.silu(x), "ReLU": lambda: F.relu(x),
        "ReLU2": lambda: F.relu(x) ** 2, "LeakyReLU": lambda: F.leaky_relu(x, fv),
        "ELU": lambda: torch.where(x > 0, x, fv * torch.expm1(x)),
        "GELU": lambda: 0.5 * x * (1 + torch.tanh(0.79788456 * (x + 0.044715 * x ** 3))),
        "Mish": lambda: x * torch.tanh(torch.where(x > 20, x, F.softplus(x))),
        "HardSwish": lambda: F.hardswish(x), "HardSigmoid": lambda: F.hardsigmoid(x),
        "Tanh": lambda: torch.tanh(x), "Sigmoid": lambda: torch.sigmoid(x),
        "SwishBeta": lambda: x * torch.sigmoid(fv * x), "Sin": lambda: torch.sin(fv * x),
        "CosGate": lambda: x * torch.cos(x), "SoftCap": lambda: fv * torch.tanh(x / fv),
        "Clamp": lambda: torch.clamp(x, -fv, fv), "Scale": lambda: x * fv, "LayerScale": lambda: x * w,
        "DyT": lambda: torch.tanh(fv * x) * w, "PReLU": lambda: torch.where(x > 0, x, x * w * fv),
        "xATLU": lambda: x * (w * torch.sigmoid(x) + 1 - w), "Softplus": lambda: F.softplus(x),
        "Snake": lambda: x + torch.sin(fv * x) ** 2 / fv,
    }[name]()


def _torch_norm(name, x, C, fv, w, beta):
    """F7: statistics over aligned 64-channel groups (whole row if C <= 64), divided by C."""
    import torch
    G = C if C <= 64 else 64
    outs = []
    for g0 in range(0, C, G):
        v = x[:, g0:g0 + G]
        if name in ("LN", "BN"):
            m = v.sum(1, keepdim=True) / C
            var = torch.clamp(v.pow(2).sum(1, keepdim=True) / C - m * m, min=0)
            xh = (v - m) * torch.rsqrt(var + fv)
            outs.append(xh * w[g0:g0 + G] + beta[g0:g0 + G])
        else:
            xh = v * torch.rsqrt(v.pow(2).sum(1, keepdim=True) / C + fv)
            outs.append(xh * w[g0:g0 + G] if name == "RMSNorm" else xh)
    return torch.cat(outs, 1)


def _torch_chain(x, C, names_fv, params, twin, n_left, n_right):
    v = x[:, :C]
    u = x[:, C:] if twin else None
    for k, (name, fv) in enumerate(names_fv):
        if twin and k == n_left + n_right:
            v = v * u
        w, beta, b = params.get(("w", k)), params.get(("beta", k)), params.get(("bias", k))
        br = params.get(("branch", k))
        on_right = twin and n_left <= k < n_left + n_right
        t = u if on_right else v
        if name in ("RMSNorm", "LN", "BN", "L2Norm"):
            t = _torch_norm(name, t, C, fv, w, beta)
        elif name == "Add":
            t = t + br
        else:
            t = _torch_op(name, t, fv, w, b)
        if on_right:
            u = t
        else:
            v = t
    if twin and len(names_fv) == n_left + n_right:
        v = v * u
    return v


def _make_params(names_fv, C, rows, rng):
    params = {}
    for k, (name, _) in enumerate(names_fv):
        fl = oracle.plasma_flags(OPS[name])
        if fl & oracle.PR_W:
            params[("w", k)] = (1.0 + 0.3 * rng.standard_normal(C)).astype(np.float32)
        if fl & oracle.PR_BETA:
            params[("beta", k)] = (0.2 * rng.standard_normal(C)).astype(np.float32)
        if fl & oracle.PR_BIAS:
            params[("bias", k)] = (0.2 * rng.standard_normal(C)).astype(np.float32)
        if fl & oracle.PR_BRANCH:
            params[("branch", k)] = rng.standard_normal((rows, C)).astype(np.float32)
    return params


CHAINS = [
    dict(C=512, chain=["Bias", "Add", "RMSNorm"]),                      # residual + pre-norm, F7 groups
    dict(C=64, chain=["RMSNorm", ("SoftCap", 4.0), "LayerScale"]),
    dict(C=96, chain=["LN", "GELU", "DyT", "PReLU", "xATLU"]),          # partial last group
    dict(C=24, chain=["Bias", "L2Norm", "Mish", ("Snake", 1.2), "Softplus", "BN"]),
    dict(C=128, chain=["SiLU", "ReLU2", ("LeakyReLU", 0.1), "ELU", "HardSwish", "HardSigmoid", "Tanh", "Sigmoid"]),
    dict(C=64, chain=[("SwishBeta", 1.5), ("Sin", 1.3), "CosGate", ("Clamp", 1.5), ("Scale", 0.7), "ReLU", "Add"]),
    dict(C=512, twin=True, left=["SiLU"], right=[], chain=[("Scale", 0.5), "Add"]),
    dict(C=64, twin=True, left=["Bias", "GELU"], right=["Bias", "LayerScale"], chain=["RMSNorm"]),
    dict(C=32, twin=True, left=["Sigmoid"], right=["Tanh"], chain=[]),
]


def _chain_nodes(c):
    def norm(lst):
        return [(x, None) if isinstance(x, str) else x for x in lst]
    if c.get("twin"):
        items = norm(c["left"]) + norm(c["right"]) + norm(c["chain"])
        nl, nr = len(c["left"]), len(c["right"])
    else:
        items = norm(c["chain"])
        nl = nr = 0
    L = plasma.lib()
    names_fv = [(n, float(L.tkm_plasma_default_fval(OPS[n])) if fv is None else float(fv)) for n, fv in items]
    return names_fv, nl, nr


@pytest.mark.parametrize("c", CHAINS, ids=lambda c: f"C{c['C']}{'_twin' if c.get('twin') else ''}_" +
                         "-".join(x if isinstance(x, str) else x[0] for x in c["chain"])[:40])
def test_chain_matches_autograd(c):
    import torch
    C, twin = c["C"], bool(c.get("twin"))
    names_fv, nl, nr = _chain_nodes(c)
    rows = 37
    rng = np.random.default_rng(C + len(names_fv))
    x = rng.standard_normal((rows, 2 * C if twin else C)).astype(np.float32)
    params = _make_params(names_fv, C, rows, rng)
    nodes = [(OPS[n], fv) for n, fv in names_fv]
    out, xhat, istd = oracle.plasma_fwd(x, rows, C, nodes, params, twin, nl, nr, "f32")
    tparams = {k: torch.tensor(v, dtype=torch.float64, requires_grad=(k[0] != "branch")) for k, v in params.items()}
    tbr = {k: v for k, v in tparams.items() if k[0] == "branch"}
    for k in tbr:
        tbr[k].requires_grad_(True)
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    ref = _torch_chain(tx, C, names_fv, tparams, twin, nl, nr)
    np.testing.assert_allclose(out, ref.detach().numpy(), rtol=2e-6, atol=2e-6)
    dout = rng.standard_normal((rows, C)).astype(np.float32)
    (ref * torch.tensor(dout, dtype=torch.float64)).sum().backward()
    din, dbr, grads = oracle.plasma_bwd(dout, x, rows, C, nodes, params, xhat, istd, twin, nl, nr, "f32",
                                        acc_flags=0)
    np.testing.assert_allclose(din, tx.grad.numpy(), rtol=1e-5, atol=1e-5)
    for (kind, k), g in grads.items():
        src = {"dw": "w", "dbeta": "beta", "dbias": "bias"}[kind]
        np.testing.assert_allclose(g, tparams[(src, k)].grad.numpy(), rtol=1e-5, atol=1e-5, err_msg=f"{kind}{k}")
    for k, g in dbr.items():
        np.testing.assert_allclose(g, tparams[("branch", k)].grad.numpy(), rtol=1e-5, atol=1e-5)


def test_f7_group_statistics():
    """C <= 64: the norms are torch's; C > 64: per-64-channel sums over C, unlike a full-row norm."""
    import torch
    import torch.nn.functional as F
    rng = np.random.default_rng(3)
    for C in (16, 64):
        x = rng.standard_normal((9, C)).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(C)).astype(np.float32)
        b = (0.1 * rng.standard_normal(C)).astype(np.float32)
        o, _, _ = oracle.plasma_fwd(x, 9, C, [(OPS["RMSNorm"], 1e-5)], {("w", 0): w}, dtype="f32")
        r = F.rms_norm(torch.tensor(x, dtype=torch.float64), (C,), torch.tensor(w, dtype=torch.float64), eps=1e-5)
        np.testing.assert_allclose(o, r.numpy(), rtol=2e-6, atol=1e-6)
        o, _, _ = oracle.plasma_fwd(x, 9, C, [(OPS["LN"], 1e-5)], {("w", 0): w, ("beta", 0): b}, dtype="f32")
        r = F.layer_norm(torch.tensor(x, dtype=torch.float64), (C,), torch.tensor(w, dtype=torch.float64),
                         torch.tensor(b, dtype=torch.float64), eps=1e-5)
        np.testing.assert_allclose(o, r.numpy(), rtol=2e-6, atol=1e-6)
    C = 512
    x = rng.standard_normal((4, C)).astype(np.float32) * np.repeat(np.arange(1, 9), 64).astype(np.float32)
    o, _, istd = oracle.plasma_fwd(x, 4, C, [(OPS["L2Norm"], 1e-5)], {}, dtype="f32")
    grp = x.reshape(4, 8, 64).astype(np.float64)
    want = grp / np.sqrt((grp ** 2).sum(-1, keepdims=True) / C + 1e-5)
    np.testing.assert_allclose(o, want.reshape(4, C), rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(istd[0], 1 / np.sqrt((grp ** 2).sum(-1) / C + 1e-5), rtol=1e-6)
    full = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-5)
    assert np.abs(o - full).max() > 0.5


def test_planted_mistakes_are_caught():
    """Mistakes planted in the oracle's inputs or its torch counterpart must fail the checks."""
    import torch
    rng = np.random.default_rng(5)
    C, rows = 64, 8
    x = rng.standard_normal((rows, C)).astype(np.float32)
    w = (1 + 0.3 * rng.standard_normal(C)).astype(np.float32)
    # (a) a weight of the wrong node: LayerScale reading RMSNorm's w
    names = [("RMSNorm", 1e-5), ("LayerScale", 1e-4)]
    nodes = [(OPS[n], fv) for n, fv in names]
    good, _, _ = oracle.plasma_fwd(x, rows, C, nodes, {("w", 0): w, ("w", 1): 2 * w}, dtype="f32")
    bad, _, _ = oracle.plasma_fwd(x, rows, C, nodes, {("w", 0): w, ("w", 1): w}, dtype="f32")
    assert np.abs(good - bad).max() > 1e-2
    # (b) full-row statistics instead of F7 groups at C = 128
    x2 = rng.standard_normal((rows, 128)).astype(np.float32) * np.repeat([1.0, 5.0], 64).astype(np.float32)
    o, _, _ = oracle.plasma_fwd(x2, rows, 128, [(OPS["L2Norm"], 1e-5)], {}, dtype="f32")
    full = x2 / np.sqrt((x2.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-5)
    assert np.abs(o - full).max() > 0.1
    # (c) an inverted gate product in a twin group: left * right swapped with left / right
    t = torch.tensor(rng.standard_normal((rows, 2 * C)), dtype=torch.float64)
    ref = _torch_chain(t, C, [("SiLU", 0.0)], {}, True, 1, 0)
    o, _, _ = oracle.plasma_fwd(t.numpy().astype(np.float32), rows, C, [(OPS["SiLU"], 0.0)], {}, True, 1, 0, "f32")
    assert np.abs(o - ref.numpy()).max() < 1e-5
    swapped = torch.nn.functional.silu(t[:, C:]) * t[:, :C]
    assert np.abs(o - swapped.numpy()).max() > 1e-2
    # (d) a derivative with a flipped sign fails its central difference
    d, _ = oracle.plasma_op_grad(OPS["Tanh"], 0.0, 0.5)
    fd = (np.tanh(0.5 + 1e-6) - np.tanh(0.5 - 1e-6)) / 2e-6
    assert abs(d - fd) < 1e-8 and abs(-d - fd) > 0.5


# ---- emitter + hipRTC ---------------------------------------------------------------------

def _objdump():
    for cand in ("/opt/rocm/llvm/bin/llvm-objdump", shutil.which("llvm-objdump")):
        if cand and os.path.exists(cand):
            return cand
    return None


@pytest.mark.parametrize("c", CHAINS, ids=lambda c: f"C{c['C']}{'_twin' if c.get('twin') else ''}")
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_emitted_chain_compiles(c, dtype, tmp_path):
    d = plasma.make_desc(c["C"], c["chain"], bool(c.get("twin")), c.get("left", ()), c.get("right", ()), dtype, 9)
    src = plasma.source(d)
    assert src.startswith(prep.prelude())
    assert "void tkm_plasma_fwd_g9(" in src and "void tkm_plasma_bwd_g9(" in src
    rc, code, log = prep.rtc_compile(src)
    assert rc == 0, log
    od = _objdump()
    if od:
        co = tmp_path / "k.co"
        co.write_bytes(code)
        dis = subprocess.run([od, "-d", "--mcpu=gfx950", str(co)], capture_output=True, text=True).stdout
        assert not re.search(r"v_pk_(add|mul|fma)_f32", dis)
        assert "scratch_" not in dis
        notes = subprocess.run([od.replace("objdump", "readelf"), "--notes", str(co)], capture_output=True,
                               text=True).stdout
        assert max(int(v) for v in re.findall(r"\.vgpr_spill_count:\s+(\d+)", notes)) == 0
        assert max(int(v) for v in re.findall(r"\.private_segment_fixed_size:\s+(\d+)", notes)) == 0


@pytest.mark.parametrize("kw,msg", [
    (dict(channels=21, chain=["SiLU"]), "even"),
    (dict(channels=20, chain=["RMSNorm"]), "multiple of 8"),
    (dict(channels=20, chain=["SiLU", ("Drop", 1.0, 3, 5)]), "Drop needs"),
    (dict(channels=20, chain=["Bias", "SiLU", ("Drop", 0.2, 3, 5), "Add"]), None),
    (dict(channels=64, chain=["SiLU"] * 9), "chain lengths"),
    (dict(channels=64, twin=True, left=["RMSNorm"]), "twin gate"),
    (dict(channels=64, twin=True, right=["Add"]), "twin gate"),
    (dict(channels=64, chain=[("RMSNorm", 0.0)]), "epsilon"),
    (dict(channels=64, chain=[("SoftCap", 0.0)]), "fval"),
    (dict(channels=64, chain=["SiLU"], dtype="bf16"), None),
])
def test_bad_descriptor_rejected(kw, msg):
    chain = kw.pop("chain", ())
    if len(chain) > plasma.MAX_NODES:
        d = plasma.make_desc(kw.pop("channels"), chain[:8], **kw)
        d.n_main = 9
    else:
        d = plasma.make_desc(kw.pop("channels"), chain, **kw)
    L = plasma.lib()
    p = L.tkm_plasma_source(ctypes.byref(d))
    if msg is None:
        assert p
        L.tkm_free(p)
        return
    assert p is None
    assert msg.encode() in L.tkm_attn_last_error()
    h = ctypes.c_void_p()
    assert L.tkm_plasma_create(ctypes.byref(d), ctypes.byref(h)) != 0 and not h.value


def test_null_handles_rejected():
    L = plasma.lib()
    assert L.tkm_plasma_num_args(None, 0) == -1
    k, n = ctypes.c_int(), ctypes.c_int()
    assert L.tkm_plasma_arg(None, 0, 0, ctypes.byref(k), ctypes.byref(n)) == -1
    assert L.tkm_plasma_fwd(None, None, 4, None) == -1
    assert L.tkm_plasma_bwd(None, None, 4, 0, None, 0, None) == -1
    assert L.tkm_plasma_bwd_workspace_bytes(None, 4) == 0
    L.tkm_plasma_destroy(None)


@pytest.mark.parametrize("name", plasma.FORMULA_OPS)
def test_descriptor_api_rejects_registry_only_ops(name):
    """Formula, FormulaW and FormulaB carry no formula of this build: only the whole-graph
    generator, given the registry's code, can emit them."""
    d = plasma.make_desc(64, ["Bias", name])
    with pytest.raises(plasma.AttnError) as e:
        plasma.source(d)
    assert "registry" in str(e.value)


def test_softplus_overflows_as_the_reference_formula():
    """Softplus is the registry's user formula log(1.0 + exp(x)) (tkm_registry.c:446-448), which
    the reference's generated code evaluates in float: finite up to ln(FLT_MAX) ~ 88.72, +inf
    above (expf overflows).  The oracle follows the float evaluation there, not the exact
    function; checked against numpy's float32 evaluation of the same formula."""
    op = OPS["Softplus"]
    with np.errstate(over="ignore"):
        for x in (-30.0, 0.0, 20.0, 80.0, 88.0, 88.72, 88.73, 100.0, 1000.0):
            f32 = float(np.log(np.float32(1.0) + np.exp(np.float32(x))))
            got = oracle.plasma_op(op, 0.0, x)
            if np.isinf(f32):
                assert np.isinf(got) and got > 0, (x, got)
            else:
                assert got == pytest.approx(f32, rel=1e-6, abs=1e-7), (x, got, f32)

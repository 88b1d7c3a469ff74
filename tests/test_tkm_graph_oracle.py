"""Pins of the chained training-step oracle (tests/tkm_graph_oracle.py) on the CPU.

The oracle composes the per-op oracles over the reference front end's graph IR; what it adds is
the wiring (which activation feeds which op, where gradients accumulate, which tensor a group's
parameter gradient lands in) and the optimizer.  A wrong wire or a dropped accumulation shows in
these checks:
  - input and parameter gradients of the whole step against central differences of its own
    loss, in float32 storage (no 16-bit rounding), on llama_small (GQA, twin SwiGLU, three
    residual adds, a final RMSNorm) and exotic_llama (QK-norm with RoPE, SoftCap, LayerScale,
    Drop with the reference's RNG, DyT, CosGate / ReLU2 twin gates);
  - the update against torch.optim.SGD with Nesterov momentum 0.9 and weight decay 1e-4 on the
    GEMM weights only (the reference's update, src/tkm_gpu.cu:684-720, on its first step).
"""
import json
import os

import numpy as np
import pytest

import tkm_graph_oracle as T

HERE = os.path.dirname(os.path.abspath(__file__))
GRAPHS = np.load(os.path.join(HERE, "golden", "tkm_graphs.npz"))
REGISTRY = json.load(open(os.path.join(HERE, "golden", "tkm_registry.json")))


def _setup(name, dtype="f32", seed=0):
    from tokamak_amd import plasma
    js = json.loads(bytes(GRAPHS[name + "/json"]).decode())
    nodes = T._fix_shapes([dict(n) for n in js["nodes"]])
    rng = np.random.default_rng(seed)
    ws = []
    for nid, kind, n in T.tensor_layout(js, REGISTRY):
        if kind == "W":
            ws.append(rng.standard_normal(n) * np.sqrt(1.0 / nodes[nodes[nid]["in0"]]["C"]))
        elif kind == "w":
            ws.append(1 + 0.1 * rng.standard_normal(n))
        else:
            ws.append(0.05 * rng.standard_normal(n))
    gs = T.GraphStep(js, REGISTRY, plasma.OP_NAMES, [w.astype(np.float32) for w in ws], dtype)
    rows = gs.rows(nodes[0])
    x = rng.standard_normal(rows * nodes[0]["C"]).astype(np.float32)
    V = nodes[next(n for n in nodes if n["op"] == T.OP_CE)["in0"]]["C"]
    y = rng.integers(0, V, rows).astype(np.int32)
    return gs, x, y


def _fd_loss(gs, x, y):
    return gs.step(x, y, 0.0, backward=False)["loss"]


@pytest.mark.parametrize("name,eps,n_x", [("llama_small", 1e-2, 8), ("exotic_llama", 1e-3, 3)])
def test_step_gradients_match_finite_differences(name, eps, n_x):
    gs, x, y = _setup(name)
    r = gs.step(x, y, 0.0)
    assert np.isfinite(r["loss"])
    rng = np.random.default_rng(1)
    g0 = r["grad"][0].ravel()
    coords = list(rng.choice(g0.size, n_x, replace=False)) + [int(np.argmax(np.abs(g0)))]
    for i in coords:
        xp, xm = x.copy(), x.copy()
        xp[i] += eps
        xm[i] -= eps
        num = (_fd_loss(gs, xp, y) - _fd_loss(gs, xm, y)) / (2 * eps)
        assert abs(num - g0[i]) <= 1e-4 + 2e-2 * abs(g0[i]), (name, "x", i, g0[i], num)
    # one coordinate of every fourth parameter tensor that has a gradient, of every kind
    keys = [k for k in gs.params if np.any(np.asarray(r["pgrad"].get(k, 0)))]
    assert {"W", "bias", "w"} <= {k[1] for k in keys}
    picked = keys[::4] if name == "llama_small" else keys[::12]
    for key in picked:
        pg = np.asarray(r["pgrad"][key], np.float64).ravel()
        j = int(np.argmax(np.abs(pg)))
        p0 = gs.params[key].copy()
        gs.params[key] = p0.copy()
        gs.params[key].ravel()[j] += eps
        lp = _fd_loss(gs, x, y)
        gs.params[key] = p0.copy()
        gs.params[key].ravel()[j] -= eps
        lm = _fd_loss(gs, x, y)
        gs.params[key] = p0
        num = (lp - lm) / (2 * eps)
        assert abs(num - pg[j]) <= 1e-4 + 2e-2 * abs(pg[j]), (name, key, j, pg[j], num)


def test_untouched_parameters_have_no_gradient():
    """Dead FC weights (the unfused projections the front end replaced) receive no gradient;
    their update is the weight decay alone."""
    gs, x, y = _setup("llama_small")
    r = gs.step(x, y, 0.1)
    dead = [n["id"] for n in gs.nodes if n["dead"] and n["op"] == T.OP_FC]
    assert dead
    for nid in dead:
        assert (nid, "W") not in r["pgrad"]
        p = gs.params[(nid, "W")].astype(np.float64)
        np.testing.assert_allclose(r["new"][(nid, "W")], p - 0.1 * 1.9 * 1e-4 * p, rtol=1e-6)


def test_update_is_torch_nesterov_sgd():
    import torch
    gs, x, y = _setup("llama_small")
    lr = 0.05
    r = gs.step(x, y, lr)
    for key, p in gs.params.items():
        g = np.asarray(r["pgrad"].get(key, np.zeros(p.shape)), np.float64).reshape(p.shape)
        t = torch.tensor(p.astype(np.float64), requires_grad=True)
        opt = torch.optim.SGD([t], lr=lr, momentum=0.9, nesterov=True,
                              weight_decay=1e-4 if key[1] == "W" else 0.0)
        t.grad = torch.tensor(g)
        opt.step()
        np.testing.assert_allclose(r["new"][key], t.detach().numpy(), rtol=1e-6, atol=1e-9, err_msg=str(key))


def test_sixteen_bit_storage_stays_close_to_float32():
    """The f16 walk (every slot rounded as the runtime stores it) stays near the float32 walk."""
    g32, x, y = _setup("llama_small", "f32")
    g16, _, _ = _setup("llama_small", "f16")
    a, b = g32.step(x, y, 0.0), g16.step(x, y, 0.0)
    assert abs(a["loss"] - b["loss"]) < 5e-3 * abs(a["loss"])
    d32, d16 = a["grad"][0], b["grad"][0]
    assert np.abs(d16 - d32).max() <= 3e-2 * np.abs(d32).max()

"""A CPU restatement of one training step of the reference runtime over a graph IR, built from the
per-op oracles (test infrastructure; the GPU runtime tests compare tkm_hip.c against it).

It follows the reference's walks: forward nodes in order (src/tkm_gpu.cu:1176-1289), backward
in reverse with the gradient arena zeroed first (1291-1421), the loss kernel's softmax
cross-entropy (632-682) and the momentum SGD with weight decay on GEMM weights (684-720).  The
groups and attention run through the oracles of this directory's siblings (oracle/plasma_ref.c,
oracle/qkv_prep_ref.c, oracle/attn_ref.c); GEMMs in float64 on the 16-bit rounded operands.
Every arena slot is rounded to the 16-bit storage type where the runtime stores it, so the
comparison measures arithmetic order, not storage precision.
"""
from __future__ import annotations

import numpy as np

import oracle

OP_FC, OP_TWIN, OP_QKV, OP_GQA, OP_QKNORM, OP_ADD, OP_USER, OP_CE = 3, 4, 5, 6, 31, 56, 62, 59
GEMM = (OP_FC, OP_TWIN, OP_QKV)
RES_BIAS, RES_W, RES_BETA = 1, 2, 4
INITIAL_STEP_SEED = 0x13579BDF


def _fix_shapes(nodes):
    for n in nodes:
        if n["C"] == 0 and n["in0"] >= 0:
            p = nodes[n["in0"]]
            n["H"], n["W"] = p["H"], p["W"]
            n["C"] = p["c_out"] if p["c_out"] > 0 else p["C"]
    return nodes


def tensor_layout(js, registry):
    """[(node, kind, size)] in the runtime's TKM1 order; kind: 'W', 'bias', 'w', 'beta'."""
    by_op = {}
    for e in registry:
        by_op.setdefault(e["op"], e)
    nodes = _fix_shapes([dict(n) for n in js["nodes"]])
    out = []
    for n in nodes:
        C = n["C"]
        if C <= 0:
            continue
        if n["op"] in GEMM:
            out.append((n["id"], "W", nodes[n["in0"]]["C"] * C))
        flags = registry[n["spec_id"]]["res_flags"] if n["op"] == OP_USER else by_op[n["op"]]["res_flags"]
        for bit, kind in ((RES_BIAS, "bias"), (RES_W, "w"), (RES_BETA, "beta")):
            if flags & bit:
                out.append((n["id"], kind, C))
    return out


def r16(x, dtype):
    """Storage rounding of an arena slot ("f32": none, for finite-difference checks)."""
    if dtype == "f32":
        return np.asarray(x, np.float32)
    return oracle.round_to(np.asarray(x, np.float32), dtype)[0]


class GraphStep:
    def __init__(self, js, registry, plasma_names, weights, dtype="f16"):
        self.js = js
        self.nodes = _fix_shapes([dict(n) for n in js["nodes"]])
        self.groups = js["groups"]
        self.B = js["batch_size"]
        self.dtype = dtype
        self.registry = registry
        self.pnames = {n: i for i, n in enumerate(plasma_names)}
        self.layout = tensor_layout(js, registry)
        assert len(self.layout) == len(weights)
        self.params = {(nid, kind): w.astype(np.float32).copy() for (nid, kind, _), w in zip(self.layout, weights)}

    def rows(self, n):
        return self.B * n["H"] * n["W"]

    # ---- groups
    def _chain(self, grp):
        nodes = self.nodes
        if grp["is_twin_epilogue"]:
            mul = nodes[grp["nodes"][0]]
            return mul["left"] + mul["right"] + grp["nodes"][1:], True, len(mul["left"]), len(mul["right"])
        return list(grp["nodes"]), False, 0, 0

    def _plasma_setup(self, grp, act, seed):
        chain, twin, nl, nr = self._chain(grp)
        rows, C = self.rows(self.nodes[grp["out_node_id"]]), grp["C"]
        pn, params = [], {}
        for k, nid in enumerate(chain):
            n = self.nodes[nid]
            name = self.registry[n["spec_id"]]["name"]
            op = self.pnames[name]
            pn.append((op, n["fval"]))
            if (nid, "w") in self.params:
                params[("w", k)] = self.params[(nid, "w")]
            if (nid, "beta") in self.params:
                params[("beta", k)] = self.params[(nid, "beta")]
            if (nid, "bias") in self.params:
                params[("bias", k)] = self.params[(nid, "bias")]
            if n["op"] == OP_ADD:
                params[("branch", k)] = act[n["in1"]]
            if name == "Drop":
                params[("keep", k)] = oracle.drop_keep(rows, C, seed, nid, n["rng_type"], n["fval"])
        return chain, twin, nl, nr, rows, C, pn, params

    def _prep_setup(self, grp):
        n = self.nodes[grp["nodes"][0]]
        D, Hq, Hkv = n["head_dim"], n["q_heads"], n["kv_heads"]
        f = oracle.prep_inv_freq(D, n["rope_theta"], n["rope_scale"], n["rope_low_freq_factor"],
                                 n["rope_high_freq_factor"], n["rope_original_context_length"])
        return n, D, Hq, Hkv, f

    def step(self, x, labels, lr, seed=INITIAL_STEP_SEED, backward=True):
        nodes, dt, B = self.nodes, self.dtype, self.B
        act, saved, grad = {}, {}, {}
        act[0] = r16(x.reshape(self.rows(nodes[0]), nodes[0]["C"]), dt)
        done = set()
        loss = 0.0
        for n in nodes[1:]:
            if n["dead"]:
                continue
            i = n["id"]
            if n["plasma_grp"] >= 0:
                gid = n["plasma_grp"]
                if gid in done:
                    continue
                done.add(gid)
                grp = self.groups[gid]
                xin = act[grp["anchor_id"]]
                if grp["is_qkv_prep"]:
                    pn, D, Hq, Hkv, f = self._prep_setup(grp)
                    rows = self.rows(pn)
                    gamma = self.params[(pn["id"], "w")][:(Hq + Hkv) * D]
                    out, xh, ist = oracle.prep_fwd(xin, self.params[(pn["id"], "bias")], gamma, f, rows,
                                                   pn["H"] * pn["W"], Hq, Hkv, D, bool(pn["has_qknorm"]),
                                                   bool(pn["has_rope"]), dt)
                    saved[gid] = (xh, ist, f)
                else:
                    chain, twin, nl, nr, rows, C, pn_, params = self._plasma_setup(grp, act, seed)
                    out, xh, ist = oracle.plasma_fwd(xin, rows, C, pn_, params, twin, nl, nr, dt)
                    saved[gid] = (xh, ist, params, pn_, chain, twin, nl, nr)
                act[grp["out_node_id"]] = out
                continue
            xin = act[n["in0"]]
            if n["op"] in GEMM:
                K = nodes[n["in0"]]["C"]
                W = r16(self.params[(i, "W")].reshape(K, n["C"]), dt).astype(np.float64)
                act[i] = r16(xin.astype(np.float64) @ W, dt)
            elif n["op"] == OP_GQA:
                S = n["H"] * n["W"]
                o, lse = oracle.fwd(xin.reshape(B, S, -1), B, S, n["q_heads"], n["kv_heads"], n["head_dim"],
                                    causal=bool(n["causal"]), f64=True)
                act[i] = r16(o.reshape(B * S, -1), dt)
                saved[("lse", i)] = lse
            elif n["op"] == OP_CE:
                z = xin.astype(np.float64)
                rows = z.shape[0]
                m = z.max(axis=1, keepdims=True)
                e = np.exp(z - m)
                p = e / e.sum(axis=1, keepdims=True)
                y = np.asarray(labels, np.int64)[:rows]
                tp = np.maximum(p[np.arange(rows), y], 1e-7)
                loss += float(np.sum(-np.log(tp)) / rows)
                onehot = np.zeros_like(p)
                onehot[np.arange(rows), y] = 1.0
                grad[n["in0"]] = r16((p - onehot) / rows, dt)
            else:
                raise NotImplementedError(f"op {n['op']}")
        if not backward:
            return {"loss": loss, "act": act}

        def g_of(nid):
            if nid not in grad:
                grad[nid] = np.zeros((self.rows(nodes[nid]), nodes[nid]["C"]), np.float32)
            return grad[nid]
        pgrad = {}
        done = set()
        for n in reversed(nodes[1:]):
            if n["dead"] or n["op"] == OP_CE:
                continue
            i = n["id"]
            if n["plasma_grp"] >= 0:
                gid = n["plasma_grp"]
                if gid in done:
                    continue
                done.add(gid)
                grp = self.groups[gid]
                a, o = grp["anchor_id"], grp["out_node_id"]
                if grp["is_qkv_prep"]:
                    pn, D, Hq, Hkv, f = self._prep_setup(grp)
                    xh, ist, _ = saved[gid]
                    gamma = self.params[(pn["id"], "w")][:(Hq + Hkv) * D]
                    din, dgamma, dbias = oracle.prep_bwd(g_of(o), xh, ist, gamma, f, self.rows(pn), pn["H"] * pn["W"],
                                                         Hq, Hkv, D, bool(pn["has_qknorm"]), bool(pn["has_rope"]), dt,
                                                         din_prev=g_of(a))
                    grad[a] = din
                    pgrad[(pn["id"], "bias")] = pgrad.get((pn["id"], "bias"), 0) + dbias
                    if pn["has_qknorm"]:
                        w = np.zeros(grp["C"])
                        w[:len(dgamma)] = dgamma
                        pgrad[(pn["id"], "w")] = pgrad.get((pn["id"], "w"), 0) + w
                else:
                    xh, ist, params, pn_, chain, twin, nl, nr = saved[gid]
                    rows, C = self.rows(nodes[o]), grp["C"]
                    adds = {k: nodes[nid]["in1"] for k, nid in enumerate(chain) if nodes[nid]["op"] == OP_ADD}
                    acc = (0 if twin else 1) | 2 | 4
                    din, dbr, pg = oracle.plasma_bwd(g_of(o), act[a], rows, C, pn_, params, xh, ist, twin, nl, nr, dt,
                                                     acc_flags=acc, din_prev=None if twin else g_of(a),
                                                     dbranch_prev={k: g_of(src) for k, src in adds.items()})
                    grad[a] = din
                    for k, src in adds.items():
                        grad[src] = dbr[k]
                    for (kind, k), v in pg.items():
                        key = (chain[k], {"dw": "w", "dbeta": "beta", "dbias": "bias"}[kind])
                        pgrad[key] = pgrad.get(key, 0) + v
                continue
            if n["op"] in GEMM:
                K = nodes[n["in0"]]["C"]
                W = r16(self.params[(i, "W")].reshape(K, n["C"]), dt).astype(np.float64)
                dy = g_of(i).astype(np.float64)
                pgrad[(i, "W")] = act[n["in0"]].astype(np.float64).T @ dy
                grad[n["in0"]] = r16(g_of(n["in0"]).astype(np.float64) + dy @ W.T, dt)
            elif n["op"] == OP_GQA:
                S = n["H"] * n["W"]
                d = oracle.bwd(act[n["in0"]].reshape(B, S, -1), act[i].reshape(B, S, -1), g_of(i).reshape(B, S, -1),
                               saved[("lse", i)], B, S, n["q_heads"], n["kv_heads"], n["head_dim"],
                               causal=bool(n["causal"]), f64=True)
                grad[n["in0"]] = r16(d.reshape(B * S, -1), dt)
        # SGD (momentum 0.9, weight decay 1e-4 on GEMM weights, velocities start at zero)
        new = {}
        for (nid, kind), p in self.params.items():
            g = np.asarray(pgrad.get((nid, kind), np.zeros(p.shape)), np.float64).reshape(p.shape)
            p64 = p.astype(np.float64)
            if kind == "W":
                g = g + 1e-4 * p64
            v = g
            new[(nid, kind)] = (p64 - lr * (0.9 * v + g)).astype(np.float32)
        return {"loss": loss, "act": act, "grad": grad, "pgrad": pgrad, "new": new}

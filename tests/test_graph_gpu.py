"""The attention layer's step captured as one graph (tkm_graph_*, include/tkm_prep.h), as the
reference's tkm_runtime_step captures its step (src/tkm_gpu.cu:1498-1508).

Step = qkv-prep forward (generated, hipRTC) -> attention forward -> attention backward (3
kernels) -> qkv-prep backward (2 kernels).  The graph is replayed several times, with eager
work between the replays that overwrites every output; every replay must reproduce the eager
step bit for bit (all kernels are deterministic).  The eager step itself is checked against
the chained CPU oracles.
"""
import numpy as np
import pytest

import oracle
from attn_cases import TOL_BWD, TOL_FWD, compare, from_device, log, to_device

pytestmark = pytest.mark.gpu


def _layer(dev, B, S, Hq, Hkv, D, dtype):
    import torch
    from tokamak_amd import attn, prep
    rows = B * S
    P = prep.Prep(Hq, Hkv, D, S, qknorm=True, rope=True, dtype=dtype, group_id=1)
    C, QK = P.C, P.QK
    rng = np.random.default_rng(11)
    x_r, x_bits = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
    g_r, g_bits = oracle.round_to(rng.standard_normal((rows, Hq * D)).astype(np.float32), dtype)
    host = dict(x=x_r, dout=g_r, bias=(0.1 * rng.standard_normal(C)).astype(np.float32),
                gamma=(1.0 + 0.2 * rng.standard_normal(QK)).astype(np.float32))
    t16 = torch.float16 if dtype == "f16" else torch.bfloat16
    buf = dict(
        x=to_device(x_bits, dtype, dev), dout=to_device(g_bits, dtype, dev),
        bias=torch.from_numpy(host["bias"]).to(dev), gamma=torch.from_numpy(host["gamma"]).to(dev),
        qkv=torch.empty((rows, C), dtype=t16, device=dev),
        xhat=torch.empty((rows, QK), dtype=t16, device=dev),
        istd=torch.empty((rows, P.NH), dtype=torch.float32, device=dev),
        o=torch.empty((rows, Hq * D), dtype=t16, device=dev),
        lse=torch.empty((B, Hq, S), dtype=torch.float32, device=dev),
        dqkv=torch.empty((rows, C), dtype=t16, device=dev),
        din=torch.empty((rows, C), dtype=t16, device=dev),
        dgamma=torch.empty(QK, dtype=torch.float32, device=dev),
        dbias=torch.empty(C, dtype=torch.float32, device=dev),
        ws_attn=torch.empty(attn.bwd_workspace_bytes(B, S, Hq), dtype=torch.uint8, device=dev),
        ws_prep=torch.empty(P.bwd_workspace_bytes(rows), dtype=torch.uint8, device=dev),
    )

    def step(stream):
        b = buf
        P.fwd(b["x"], b["bias"], b["gamma"], out=b["qkv"], xhat=b["xhat"], istd=b["istd"], stream=stream)
        attn.gqa_fwd(b["qkv"], B, S, Hq, Hkv, D, causal=True, out=b["o"], lse=b["lse"], stream=stream)
        attn.gqa_bwd(b["qkv"], b["o"], b["dout"], b["lse"], B, S, Hq, Hkv, D, causal=True,
                     dqkv=b["dqkv"], workspace=b["ws_attn"], stream=stream)
        P.bwd(b["dqkv"], b["xhat"], b["istd"], b["gamma"], din=b["din"], dgamma=b["dgamma"],
              dbias=b["dbias"], accumulate=False, workspace=b["ws_prep"], stream=stream)

    return P, host, buf, step


OUTPUTS = ("qkv", "xhat", "istd", "o", "lse", "dqkv", "din", "dgamma", "dbias")


@pytest.mark.parametrize("shape,dtype", [((2, 384, 4, 2, 64), "f16"), ((2, 384, 4, 2, 64), "bf16"),
                                         ((8, 512, 8, 8, 64), "bf16"), ((2, 512, 4, 2, 128), "f16"),
                                         ((2, 512, 4, 2, 128), "bf16")],
                         ids=["gqa-f16", "gqa-bf16", "config4-bf16", "gqa-f16-d128-asm", "gqa-bf16-d128-asm"])
def test_layer_step_graph_replays_match_eager(gpu, shape, dtype):
    """The layer step (qkv-prep forward, attention forward and backward, qkv-prep backward)
    captured once and replayed: every replay bit-equal to the eager step, both within the
    oracles' tolerances.  The third case is BASELINE config 4's attention layer: batch 8,
    sequence 512, 8 heads of 64, bf16; the last two capture the gfx950 assembly kernels
    (D = 128, fp16 and bf16, launched through hipModuleLaunchKernel)."""
    import torch
    from tokamak_amd import prep
    B, S, Hq, Hkv, D = shape
    log(f"[case] graph step B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} {dtype}")
    P, host, buf, step = _layer(gpu, B, S, Hq, Hkv, D, dtype)
    stream = torch.cuda.Stream(device=gpu)
    with torch.cuda.stream(stream):
        step(stream)
    torch.cuda.synchronize()
    eager = {k: buf[k].clone() for k in OUTPUTS}
    if D == 128:
        from tokamak_amd import attn
        assert attn.last_kernels() == ["dq_asm", "dkdv_asm"], attn.last_kernels()

    prep.Graph.begin(stream)
    try:
        step(stream)
    finally:
        g = prep.Graph.end(stream)
    for rep in range(4):
        with torch.cuda.stream(stream):
            for k in OUTPUTS:                        # eager work between replays
                buf[k].fill_(float("nan"))
        g.launch(stream)
        stream.synchronize()
        torch.cuda.synchronize()
        for k in OUTPUTS:
            assert torch.equal(buf[k], eager[k]), (rep, k)
        log(f"    replay {rep}: all {len(OUTPUTS)} outputs bitwise equal to the eager step")
    g.close()

    # the eager step against the chained oracles
    rows, C = B * S, P.C
    f = oracle.prep_inv_freq(D)
    qkv_r, xh_r, is_r = oracle.prep_fwd(host["x"], host["bias"], host["gamma"], f, rows, S, Hq, Hkv, D,
                                        True, True, dtype)
    o_r, lse_r = oracle.fwd(qkv_r, B, S, Hq, Hkv, D, causal=True, f64=True)
    res = [compare("O", from_device(eager["o"]), o_r.reshape(rows, -1), TOL_FWD),
           compare("LSE", from_device(eager["lse"]), lse_r, TOL_FWD)]
    o_st, _ = oracle.round_to(o_r, dtype)
    dqkv_r = oracle.bwd(qkv_r, o_st, host["dout"], lse_r, B, S, Hq, Hkv, D, causal=True, f64=True)
    res.append(compare("dqkv", from_device(eager["dqkv"]), dqkv_r.reshape(rows, C), TOL_BWD))
    dq_st, _ = oracle.round_to(dqkv_r, dtype)
    din_r, dg_r, db_r = oracle.prep_bwd(dq_st.reshape(rows, C), xh_r, is_r, host["gamma"], f, rows, S, Hq, Hkv,
                                        D, True, True, dtype)
    res.append(compare("din", from_device(eager["din"]), din_r, TOL_BWD))
    # sums over all rows of din, each within the dqkv bar: a plausibility bound whose absolute
    # part grows like the square root of the row count (0.1 at 768 rows)
    sum_tol = (1e-1 * np.sqrt(rows / 768), 2e-2)
    res.append(compare("dbias", eager["dbias"].cpu().numpy(), db_r, sum_tol))
    res.append(compare("dgamma", eager["dgamma"].cpu().numpy(), dg_r, sum_tol))
    for st in res:
        log(f"    {st['name']}: max_abs={st['max_abs']:.3e} bad={st['n_bad']}/{st['n']}")
    assert not [r for r in res if r["n_bad"]], res
    P.close()


def test_first_attention_call_inside_capture():
    """A fresh process whose very first attention call is inside a global-mode capture (the
    reference captures its first step): the code objects load without being recorded, the
    assembly kernels are the ones captured, and three replays equal the eager run bit for
    bit.  Runs tests/graph_first_call_child.py as a child process (a fresh HIP context)."""
    import os
    import subprocess
    import sys
    child = os.path.join(os.path.dirname(os.path.abspath(__file__)), "graph_first_call_child.py")
    log("[case] first attention call inside a capture (child process)")
    r = subprocess.run([sys.executable, "-u", child], capture_output=True, text=True, timeout=300)
    for line in (r.stdout + r.stderr).splitlines()[-12:]:
        log("    " + line)
    assert r.returncode == 0 and r.stdout.strip().endswith("OK"), r.stdout + r.stderr

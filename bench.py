#!/usr/bin/env python3
"""Benchmark of the MI355X attention hot path (BASELINE.json metric).

One step = one causal GQA attention forward + backward (tkm_attn_fwd, then the three
backward kernels) over one batch of synthetic fp16 inputs already resident in HBM, at
B=4, Hq=Hkv=16, S=2048, D=128, scale 1/sqrt(128).

Prints one JSON line.  value = algorithmic fwd+bwd TFLOP/s (FlashAttention convention:
F_fwd = 4*B*H*S^2*D/2 for causal, F_fwd+bwd = 3.5*F_fwd; recompute not credited).
roofline = the dominant kernel (longest average duration inside the timed region, from
HIP events recorded on the launch stream between the kernels), its algorithmic FLOPs per
launch / its average duration, against MI355X dense fp16 MFMA peak 2516.6 TFLOP/s.
cpu_baseline = the CPU oracle (oracle/attn_ref.c, fp32, OpenMP) timed on a bounded sample
of the same workload on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg3|cfg3-bf16|cfg2|cfg4|cfg4-attn|cfg5]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

PEAK_FP16_TFLOPS = 2516.6   # 256 CU x 4096 FLOP/clk x 2.4 GHz, dense
PEAK_HBM_GBPS = 8000.0

CONFIGS = {
    # name: (B, S, Hq, Hkv, D, causal, kv_len, backward, qkv scale, dtype)
    "cfg3": (4, 2048, 16, 16, 128, True, None, True, 1.0, "f16"),
    "cfg3-bf16": (4, 2048, 16, 16, 128, True, None, True, 1.0, "bf16"),
    "cfg2": (4, 1024, 8, 8, 64, True, None, False, 0.5, "f16"),
    # config 4's attention layer alone (the full step: --config cfg4)
    "cfg4-attn": (8, 512, 8, 8, 64, True, None, True, 1.0, "bf16"),
    "cfg5": (2, 8192, 32, 32, 128, False, [8192, 5000], True, 1.0, "f16"),
}
METRIC = "FlashAttn fwd+bwd TFLOP/s & % fp16 MFMA peak, B4 H16 S2048 D128 causal"

# qkv-prep epilogue (generated, hipRTC): name -> (B, S, Hq, Hkv, D, qknorm, rope, rope args).
# prep4 = config 4's group (QKNorm + RoPE, D64); prep3 = config 3's shape with llama3 RoPE
# (the reference accepts QKNorm only with D = 64).
PREP_CONFIGS = {
    "prep4": (8, 512, 8, 8, 64, True, True, {}),
    "prep3": (4, 2048, 16, 16, 128, False, True,
              dict(theta=500000.0, scale=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                   original_context_length=8192.0)),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # Defaults measure steady state: the GPU's clocks settle over the first ~50-80 steps of a
    # run (steps there measured up to 40% slower than later ones); explicit values are honoured.
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="cfg3",
                    choices=sorted(CONFIGS) + sorted(PREP_CONFIGS) + sorted(PLASMA_CONFIGS) + ["cfg4"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="time the K steps as one replay of a captured hipGraph (at cfg2 and cfg4-attn "
                         "this measured the same as eager launches)")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="threads for the CPU baseline (default: min(16, online CPUs); the GPU "
                         "boxes allot 16 host CPUs to each GPU)")
    ap.add_argument("--cpu-runs", type=int, default=3,
                    help="CPU baseline runs; the median is reported")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="also run one plain device copy of this many MiB (calibrates the "
                         "FETCH_SIZE / WRITE_SIZE counters of a profiling run)")
    ap.add_argument("--flush-mib", type=int, default=512,
                    help="cold-cache figure after the timed region: each step preceded by a write "
                         "of this many MiB (more than the 256 MB Infinity Cache); 0 skips it")
    return ap.parse_args()


def cpu_baseline(cfg, threads, max_heads, runs=3):
    """Time the CPU oracle (fp32, OpenMP) on a bounded sample of the same workload: all
    batches and S x S positions of the first max_heads heads (the whole workload when Hq
    <= max_heads), forward + backward; the median of `runs` runs."""
    import numpy as np

    import oracle
    B, S, Hq, Hkv, D, causal, kv_len, backward, mul, _ = cfg
    hs = min(Hq, max_heads)
    oracle.set_threads(threads)
    inp = oracle.make_inputs(B, S, hs, hs, D, "f16", mul=mul, with_dout=backward)
    times = []
    for _ in range(max(1, runs)):
        t0 = time.perf_counter()
        o, lse = oracle.fwd(inp["qkv"], B, S, hs, hs, D, causal=causal, kv_len=kv_len)
        if backward:
            oracle.bwd(inp["qkv"], o, inp["dout"], lse, B, S, hs, hs, D, causal=causal, kv_len=kv_len)
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    skv = S if kv_len is None else float(np.mean(kv_len))
    f = 4.0 * B * hs * S * skv * D * (0.5 if causal else 1.0) * (3.5 if backward else 1.0)
    return {"value": round(f / dt / 1e12, 6), "unit": "TFLOP/s", "cores": oracle.threads(),
            "host_online_cpus": oracle.online_cpus(), "kind": "port",
            "sample": f"oracle/attn_ref.c fp32 {'fwd+bwd' if backward else 'fwd'} on B={B} "
                      f"H={hs} of {Hq} S={S} D={D} causal={int(causal)}, {f / 1e9:.1f} GFLOP; "
                      f"median of {len(times)} runs {dt:.3f} s wall "
                      f"(runs: {', '.join(f'{t:.3f}' for t in times)}); OpenMP threads = cores, "
                      f"capped at 16, the host CPUs the GPU box allots to one GPU"}


def prep_bytes(rows, C, QK, NH, qknorm, accumulate, part_bytes):
    """Algorithmic HBM bytes of one qkv-prep forward and one backward (16-bit rows); part_bytes
    is the backward's partial-sum buffer, written once and read once."""
    fwd = 2 * rows * C * 2 + C * 4
    bwd = rows * C * 2 + rows * C * 2 * (2 if accumulate else 1) + C * 4 * (2 if accumulate else 1)
    if qknorm:
        fwd += rows * QK * 2 + rows * NH * 4 + QK * 4
        bwd += rows * QK * 2 + rows * NH * 4 + QK * 4 * (3 if accumulate else 2)
    bwd += 2 * part_bytes
    return fwd, bwd


def cpu_baseline_prep(cfg, max_rows):
    """The qkv-prep oracle (oracle/qkv_prep_ref.c, double, one thread) on the first max_rows rows."""
    import numpy as np

    import oracle
    B, S, Hq, Hkv, D, qknorm, rope, rargs = cfg
    rows = min(B * S, max_rows)
    C, QK, NH = (Hq + 2 * Hkv) * D, (Hq + Hkv) * D, Hq + Hkv
    rng = np.random.default_rng(0)
    x, _ = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), "f16")
    g, _ = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), "f16")
    bias = np.zeros(C, np.float32)
    gamma = np.ones(QK, np.float32)
    f = oracle.prep_inv_freq(D, theta=rargs.get("theta", 10000.0), scale=rargs.get("scale", 1.0))
    t0 = time.perf_counter()
    out, xh, ist = oracle.prep_fwd(x, bias, gamma, f, rows, S, Hq, Hkv, D, qknorm, rope, "f16")
    oracle.prep_bwd(g, xh, ist, gamma, f, rows, S, Hq, Hkv, D, qknorm, rope, "f16", din_prev=x)
    dt = time.perf_counter() - t0
    fb, bb = prep_bytes(rows, C, QK, NH, qknorm, True, 0)
    return {"value": round((fb + bb) / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle/qkv_prep_ref.c fwd+bwd on {rows} of {B * S} rows, "
                      f"{(fb + bb) / 1e6:.1f} MB in {dt:.2f} s"}


def run_prep(args):
    """qkv-prep forward + backward (accumulating, as the reference's step) at a prep config."""
    import numpy as np
    import torch

    from tokamak_amd import prep
    cfg = PREP_CONFIGS[args.config]
    B, S, Hq, Hkv, D, qknorm, rope, rargs = cfg
    rows = B * S
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    P = prep.Prep(Hq, Hkv, D, S, qknorm=qknorm, rope=rope, **rargs)
    C, QK, NH = P.C, P.QK, P.NH
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    x = torch.randn((rows, C), generator=g, device=dev).half()
    dout = torch.randn((rows, C), generator=g, device=dev).half()
    bias = torch.zeros(C, device=dev)
    gamma = torch.ones(QK, device=dev)
    out = torch.empty_like(x)
    din = torch.zeros_like(x)
    xhat = torch.empty((rows, QK), dtype=torch.float16, device=dev) if qknorm else None
    istd = torch.empty((rows, NH), dtype=torch.float32, device=dev) if qknorm else None
    dbias = torch.zeros(C, device=dev)
    dgamma = torch.zeros(QK, device=dev) if qknorm else None
    ws = torch.empty(P.bwd_workspace_bytes(rows), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()

    def fwd():
        P.fwd(x, bias, gamma, out=out, xhat=xhat, istd=istd)

    def bwd():
        P.bwd(dout, xhat, istd, gamma, din=din, dgamma=dgamma, dbias=dbias, accumulate=True, workspace=ws)

    for _ in range(args.warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(K)]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for k in range(K):
        ev[k][0].record(stream)
        fwd()
        ev[k][1].record(stream)
        bwd()
        ev[k][2].record(stream)
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / K
    tf = np.array([ev[k][0].elapsed_time(ev[k][1]) for k in range(K)])
    tb = np.array([ev[k][1].elapsed_time(ev[k][2]) for k in range(K)])
    fb, bb = prep_bytes(rows, C, QK, NH, qknorm, True, P.bwd_workspace_bytes(rows))
    gbs = {"qkv_prep_fwd": fb / (tf.mean() * 1e-3) / 1e9, "qkv_prep_bwd": bb / (tb.mean() * 1e-3) / 1e9}
    dom = "qkv_prep_fwd" if tf.mean() >= tb.mean() else "qkv_prep_bwd"
    res = {
        "metric": f"qkv-prep fwd+bwd GB/s ({args.config})", "value": round((fb + bb) / (ms_step * 1e-3) / 1e9, 1),
        "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f16",
        "data": "synthetic: x, dO ~ N(0,1) (torch.randn on device, seed 0), fp16",
        "config": {"workload": f"{args.config}: qkv-prep fwd + bwd (accumulate)", "B": B, "S": S, "Hq": Hq,
                   "Hkv": Hkv, "D": D, "qknorm": qknorm, "rope": rope, "rope_args": rargs},
        "kernels": {"qkv_prep_fwd": {"avg_ms": round(float(tf.mean()), 5), "bytes": fb,
                                     "gbps": round(gbs["qkv_prep_fwd"], 1)},
                    "qkv_prep_bwd": {"avg_ms": round(float(tb.mean()), 5), "bytes": bb,
                                     "gbps": round(gbs["qkv_prep_bwd"], 1)}},
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": round(gbs[dom], 1), "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(gbs[dom] / PEAK_HBM_GBPS, 4), "traffic": None},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_prep(cfg, 2048)
    print(json.dumps(res))


# plasma epilogues: name -> list of (label, C, rows, plasma kwargs, acc flags); config 4's groups
PLASMA_CONFIGS = {
    "plasma4": [("residual_rmsnorm", 512, 4096, dict(chain=["Add", "RMSNorm"]), 7),
                ("swiglu", 1536, 4096, dict(twin=True, left=["SiLU"]), 2)],
}


def plasma_bytes(P, rows, acc):
    """Algorithmic HBM bytes of one forward and one backward of a plasma group, from its
    argument lists (16-bit rows, fp32 parameters and istd, partial sums written and read)."""
    C, W, NG = P.C, (2 * P.C if P.twin else P.C), P.norm_groups()
    size = {"in": rows * W * 2, "out": rows * C * 2, "dout": rows * C * 2, "xhat": rows * C * 2,
            "istd": rows * NG * 4, "branch": rows * C * 2, "w": C * 4, "beta": C * 4, "bias": C * 4,
            "dw": C * 4, "dbeta": C * 4, "dbias": C * 4}
    fwd = sum(size[k] for k, _ in P.fwd_args)
    bwd = 0
    for k, _ in P.bwd_args:
        if k == "din":
            bwd += rows * W * 2 * (2 if acc & 1 else 1)
        elif k == "dbranch":
            bwd += rows * C * 2 * (2 if acc & 4 else 1)
        elif k in ("dw", "dbeta", "dbias"):
            bwd += C * 4 * (2 if acc & 2 else 1)
        else:
            bwd += size[k]
    bwd += 2 * P.bwd_workspace_bytes(rows)
    return fwd, bwd


def run_plasma(args):
    """Forward + backward of config 4's plasma groups (generated, hipRTC)."""
    import numpy as np
    import torch

    from tokamak_amd import plasma
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    groups = []
    for label, C, rows, kw, acc in PLASMA_CONFIGS[args.config]:
        P = plasma.Plasma(C, group_id=len(groups), **kw)
        W = 2 * C if P.twin else C
        t = {"in": torch.randn((rows, W), generator=g, device=dev).half(),
             "dout": torch.randn((rows, C), generator=g, device=dev).half(),
             "out": torch.empty((rows, C), dtype=torch.float16, device=dev),
             "din": torch.zeros((rows, W), dtype=torch.float16, device=dev)}
        for kind, node in P.fwd_args + P.bwd_args:
            if node < 0 or (kind, node) in t:
                continue
            if kind in ("w", "dw"):
                t[(kind, node)] = torch.ones(C, device=dev) if kind == "w" else torch.zeros(C, device=dev)
            elif kind in ("beta", "bias", "dbeta", "dbias"):
                t[(kind, node)] = torch.zeros(C, device=dev)
            elif kind in ("branch", "dbranch"):
                t[(kind, node)] = torch.randn((rows, C), generator=g, device=dev).half()
            elif kind == "xhat":
                t[(kind, node)] = torch.empty((rows, C), dtype=torch.float16, device=dev)
            elif kind == "istd":
                t[(kind, node)] = torch.empty((rows, P.norm_groups()), device=dev)
        ws = torch.empty(max(P.bwd_workspace_bytes(rows), 1), dtype=torch.uint8, device=dev)
        groups.append((label, P, t, rows, acc, ws))
    stream = torch.cuda.current_stream()

    def step(evs=None):
        for i, (label, P, t, rows, acc, ws) in enumerate(groups):
            P.fwd(t, rows)
            if evs is not None:
                evs[2 * i].record(stream)
            P.bwd(t, rows, acc, workspace=ws)
            if evs is not None:
                evs[2 * i + 1].record(stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2 * len(groups) + 1)] for _ in range(K)]
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    for k in range(K):
        ev[k][0].record(stream)
        step(ev[k][1:])
    t1.record(stream)
    torch.cuda.synchronize()
    ms_step = t0.elapsed_time(t1) / K
    kernels, total = {}, 0
    for i, (label, P, t, rows, acc, ws) in enumerate(groups):
        fb, bb = plasma_bytes(P, rows, acc)
        total += fb + bb
        tf = np.array([ev[k][2 * i].elapsed_time(ev[k][2 * i + 1]) for k in range(K)])
        tb = np.array([ev[k][2 * i + 1].elapsed_time(ev[k][2 * i + 2]) for k in range(K)])
        kernels[label + "_fwd"] = {"avg_ms": round(float(tf.mean()), 5), "bytes": fb,
                                   "gbps": round(fb / (tf.mean() * 1e-3) / 1e9, 1)}
        kernels[label + "_bwd"] = {"avg_ms": round(float(tb.mean()), 5), "bytes": bb,
                                   "gbps": round(bb / (tb.mean() * 1e-3) / 1e9, 1)}
    dom = max(kernels, key=lambda n: kernels[n]["avg_ms"])
    res = {
        "metric": f"plasma epilogues fwd+bwd GB/s ({args.config})",
        "value": round(total / (ms_step * 1e-3) / 1e9, 1), "unit": "GB/s", "n_gpus": 1, "steps": K,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f16", "data": "synthetic: torch.randn on device (seed 0), fp16",
        "config": {"workload": f"{args.config}: config 4's residual+RMSNorm (C512) and SwiGLU (2x1536) groups, "
                               "4096 rows, fwd + bwd"},
        "kernels": kernels,
        "roofline": {"kernel": dom, "bound": "hbm", "achieved": kernels[dom]["gbps"], "peak": PEAK_HBM_GBPS,
                     "unit": "GB/s", "frac": round(kernels[dom]["gbps"] / PEAK_HBM_GBPS, 4), "traffic": None},
    }
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline_plasma(args.config, 1024)
    print(json.dumps(res))


def cpu_baseline_plasma(name, max_rows):
    """The plasma oracle (oracle/plasma_ref.c, double, one thread) on the first max_rows rows."""
    import numpy as np

    import oracle
    from tokamak_amd import plasma
    total, t = 0, 0.0
    for label, C, rows, kw, acc in PLASMA_CONFIGS[name]:
        r = min(rows, max_rows)
        twin = kw.get("twin", False)
        items = kw.get("left", []) + kw.get("right", []) + kw.get("chain", [])
        nodes = [(plasma.OPS[n], float(plasma.lib().tkm_plasma_default_fval(plasma.OPS[n]))) for n in items]
        rng = np.random.default_rng(0)
        x = rng.standard_normal((r, 2 * C if twin else C)).astype(np.float32)
        params = {}
        for k, (op, _) in enumerate(nodes):
            fl = oracle.plasma_flags(op)
            if fl & oracle.PR_W:
                params[("w", k)] = np.ones(C, np.float32)
            if fl & oracle.PR_BRANCH:
                params[("branch", k)] = rng.standard_normal((r, C)).astype(np.float32)
        t0 = time.perf_counter()
        out, xh, ist = oracle.plasma_fwd(x, r, C, nodes, params, twin, len(kw.get("left", [])), 0, "f16")
        oracle.plasma_bwd(out, x, r, C, nodes, params, xh, ist, twin, len(kw.get("left", [])), 0, "f16", acc)
        t += time.perf_counter() - t0
        W = 2 * C if twin else C
        total += r * (W + C) * 2 * 3
    return {"value": round(total / t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle/plasma_ref.c fwd+bwd of both groups on {max_rows} of 4096 rows "
                      f"(bytes counted as 3 x (in + out) rows), {t:.2f} s"}


def step_flops(js):
    """Algorithmic FLOPs of one training step of a graph fixture: every live GEMM three times
    (forward, dW, dX: 2*rows*K*N each) and every attention node 3.5 F_fwd (causal S^2/2)."""
    nodes = js["nodes"]
    B = js["batch_size"]
    gemm = attn_f = 0.0
    for n in nodes:
        if n["dead"]:
            continue
        rows = B * n["H"] * n["W"]
        if n["op"] in (3, 4, 5):
            gemm += 3 * 2.0 * rows * nodes[n["in0"]]["C"] * n["C"]
        elif n["op"] == 6:
            S = n["H"] * n["W"]
            attn_f += 3.5 * 4.0 * B * n["q_heads"] * S * S * n["head_dim"] * (0.5 if n["causal"] else 1.0)
    return gemm, attn_f


def run_step(args):
    """one full training step (forward, backward, SGD) of the 8-layer
    Llama-style decoder (d_model 512, 8 heads x 64, SwiGLU 1376, vocabulary 8192, S 512, B 8),
    bf16 storage with fp32 master weights and int32 next-token labels, through libtkm_hip.so
    (the tkm.h runtime on HIP): one hipGraph replay per step on inputs already in HBM.  The
    graph is the reference front end's IR of tests/golden/models/cfg4_llama.tkm (fixture
    tests/golden/tkm_graphs.npz).  value = tokens/s; the attention share is config 4's attention
    layer (tkm_attn_fwd + tkm_attn_bwd at B8 S512 H8 D64 bf16) timed alone, times 8 layers,
    over the step time."""
    import numpy as np
    import torch

    from tokamak_amd import attn
    from tokamak_amd import runtime as R

    here = os.path.dirname(os.path.abspath(__file__))
    fx = np.load(os.path.join(here, "tests", "golden", "tkm_graphs.npz"))
    js = json.loads(bytes(fx["cfg4/json"]).decode())
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rt = R.Runtime(R.graph_buffer(fx["cfg4/graph"].tobytes()), dtype=attn.BF16, token_labels=True)
    B, S, C, V = js["batch_size"], 512, 512, 8192
    rng = np.random.default_rng(0)
    x = rng.standard_normal(B * S * C).astype(np.float32)
    y = rng.integers(0, V, B * S).astype(np.int32)
    rt.upload(x, y)
    lr = 1e-4
    stream = torch.cuda.ExternalStream(rt.stream())
    for _ in range(args.warmup):
        rt.step_device(lr)
    torch.cuda.synchronize()
    K = args.steps
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(K + 1)]
    wall0 = time.perf_counter()
    ev[0].record(stream)
    for k in range(K):
        rt.step_device(lr)
        ev[k + 1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    step_ms = np.array([ev[k].elapsed_time(ev[k + 1]) for k in range(K)])
    ms = float(step_ms.mean())
    loss = rt.last_loss()

    # config 4's attention layer alone, same shape and type, eager
    Hq = D = None
    for n in js["nodes"]:
        if n["op"] == 6 and not n["dead"]:
            Hq, Hkv, D = n["q_heads"], n["kv_heads"], n["head_dim"]
    n_attn = sum(1 for n in js["nodes"] if n["op"] == 6 and not n["dead"])
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    qkv = torch.randn((B, S, (Hq + 2 * Hkv) * D), generator=g, device=dev).to(torch.bfloat16)
    dout = torch.randn((B, S, Hq * D), generator=g, device=dev).to(torch.bfloat16)
    o = torch.empty((B, S, Hq * D), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=dev)
    dqkv = torch.empty_like(qkv)
    ws = torch.empty(attn.bwd_workspace_bytes(B, S, Hq), dtype=torch.uint8, device=dev)
    cur = torch.cuda.current_stream()

    def layer():
        attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, True, None, out=o, lse=lse)
        attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, True, None, dqkv=dqkv, workspace=ws)
    for _ in range(50):
        layer()
    torch.cuda.synchronize()
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a0.record(cur)
    for _ in range(100):
        layer()
    a1.record(cur)
    torch.cuda.synchronize()
    attn_ms = a0.elapsed_time(a1) / 100
    kpath = {"fwd": None, "bwd": None}
    attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, True, None, out=o, lse=lse)
    kpath["fwd"] = attn.last_kernels()
    attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, True, None, dqkv=dqkv, workspace=ws)
    kpath["bwd"] = attn.last_kernels()
    torch.cuda.synchronize()

    gemm_f, attn_f = step_flops(js)
    total_f = gemm_f + attn_f
    ach = total_f / (ms * 1e-3) / 1e12
    res = {
        "metric": "config 4 training step tokens/s (8-layer Llama-style decoder, bf16, one hipGraph)",
        "value": round(B * S / (ms * 1e-3), 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: input rows ~ N(0,1), token labels uniform in [0, 8192) (numpy seed 0); "
                "random-init weights (the runtime's seeded PCG32)",
        "config": {"workload": "cfg4: full training step (forward, backward, SGD), 8 layers",
                   "B": B, "S": S, "d_model": C, "heads": Hq, "head_dim": D, "ffn": 1376, "vocab": V,
                   "launches_per_step": rt.kernel_count()},
        "step_ms_p10_p50_p90": [round(float(np.percentile(step_ms, p)), 5) for p in (10, 50, 90)],
        "attention": {"layer_fwd_bwd_ms": round(attn_ms, 5), "layers": n_attn,
                      "share_of_step": round(n_attn * attn_ms / ms, 4),
                      "layer_tflops": round(attn_f / n_attn / (attn_ms * 1e-3) / 1e12, 2),
                      "kernel_path": kpath},
        "roofline": {"kernel": "whole step (GEMMs + attention, algorithmic FLOPs)", "bound": "mfma",
                     "achieved": round(ach, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(ach / PEAK_FP16_TFLOPS, 4), "traffic": None,
                     "flops_per_step": total_f, "gemm_flops": gemm_f, "attention_flops": attn_f},
        "last_loss": round(float(loss), 5),
        "wall_s": round(wall, 3),
    }
    rt.close()
    print(json.dumps(res))


# roofline.traffic is not measured by this run: hardware counters need a profiler run of their
# own (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE).  It is read from the committed summary of
# those runs, and the line says so.
TRAFFIC_SOURCE = ("profiles/attn_cfg3_traffic.md: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE runs of "
                  "this kernel at config 3, not this run")


def measured_traffic(name):
    """HBM bytes per launch of a kernel at config 3, from the FETCH_SIZE / WRITE_SIZE counter
    runs summarized in profiles/attn_cfg3_traffic.md (None if absent)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "attn_cfg3_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    for kv in line.split(":", 1)[1].split():
                        k, v = kv.split("=")
                        if k == name:
                            return float(v)
    except OSError:
        pass
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build targets one GPU: the attention kernels run on one "
                          "MI355X; multi-GPU sharding is design-only (run with --gpus 1)"}))
        sys.exit(2)
    if args.config in PREP_CONFIGS:
        run_prep(args)
        return
    if args.config in PLASMA_CONFIGS:
        run_plasma(args)
        return
    if args.config == "cfg4":
        run_step(args)
        return
    import numpy as np
    import torch

    from tokamak_amd import attn

    cfg = CONFIGS[args.config]
    B, S, Hq, Hkv, D, causal, kv_len, backward, mul, dtype = cfg
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    qkv = (torch.randn((B, S, (Hq + 2 * Hkv) * D), generator=g, device=dev) * mul).to(tdt)
    g.manual_seed(1)
    dout = torch.randn((B, S, Hq * D), generator=g, device=dev).to(tdt)
    o = torch.empty((B, S, Hq * D), dtype=tdt, device=dev)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=dev)
    dqkv = torch.empty_like(qkv)
    ws = torch.empty(attn.bwd_workspace_bytes(B, S, Hq), dtype=torch.uint8, device=dev)
    kvl = None if kv_len is None else torch.tensor(kv_len, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream()

    stages = [("attn_fwd", lambda: attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal, kvl, out=o, lse=lse))]
    if backward:
        # tkm_attn_bwd's schedule: dQ (computing D on the way), then dK/dV.
        for name, st in (("bwd_dq", attn.BWD_DQ_DELTA), ("bwd_dkdv", attn.BWD_DKDV)):
            stages.append((name, (lambda st=st: attn.gqa_bwd(
                qkv, o, dout, lse, B, S, Hq, Hkv, D, causal, kvl, dqkv=dqkv, workspace=ws,
                stage=st))))

    attn.init()  # load the gfx950 code objects now, not inside the first timed call

    if args.copy_mib:
        src = torch.empty(args.copy_mib << 20, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    for _ in range(args.warmup):
        for _, fn in stages:
            fn()
    torch.cuda.synchronize()

    # The timed region holds the K steps and two events, nothing between the kernels: an
    # event recorded between two kernels leaves the GPU idle for 6-10 us (kernel trace).
    # With --graph the K steps are captured first (nothing runs during a capture) and the
    # timed region is one replay of that graph.
    K = args.steps
    use_graph = args.graph

    def timed(fns, reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        graph = None
        if use_graph:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for _ in range(reps):
                    for fn in fns:
                        fn()
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        e0.record(stream)
        if graph is not None:
            graph.replay()
        else:
            for _ in range(reps):
                for fn in fns:
                    fn()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1), time.perf_counter() - w0

    total_ms, wall = timed([fn for _, fn in stages], K)
    ms_step = total_ms / K
    # Per kernel, right after: K launches of each kernel back to back between two events
    # (each launch recomputes the same outputs from the same inputs).
    kernel_path = {}
    per = {}
    for name, fn in stages:
        per[name] = timed([fn], K)[0] / K
        fn()
        torch.cuda.synchronize()
        kernel_path[name] = attn.last_kernels()

    # Cold cache: the inputs (config 3: qkv, O, dO, LSE, about 168 MB) fit in the 256 MB
    # Infinity Cache, so the figure above runs on whatever it holds.  Here every step follows a
    # write of flush_mib MiB.  No event sits between the flush and the step (an event between
    # two kernels idles the GPU for several us): K (flush + step) and K flushes alone are each
    # timed as one region, and the step's cold time is their difference over K.
    cold = None
    if args.flush_mib and not use_graph:
        junk = torch.empty(args.flush_mib << 20, dtype=torch.uint8, device=dev)

        def flush():
            junk.fill_(7)
        all_fns = [fn for _, fn in stages]
        timed([flush] + all_fns, 2)
        with_ms = timed([flush] + all_fns, K)[0]
        flush_ms = timed([flush], K)[0]
        cold_ms = (with_ms - flush_ms) / K
        cold = {"flush_mib": args.flush_mib, "ms_per_step": round(cold_ms, 5),
                "tflops": None, "flush_ms": round(flush_ms / K, 5),
                "method": "(K x (flush + step) - K x flush) / K, each one timed region"}
        del junk

    f_fwd = attn.attention_flops(B, S, Hq, D, causal, kv_len, "fwd")
    f_total = f_fwd * (3.5 if backward else 1.0)
    # Algorithmic FLOPs credited to each kernel (sums to F_fwd + 2.5 F_fwd):
    # dK/dV kernel: S, dP, dV, dK GEMMs = 2.0 F_fwd; dQ kernel: the dQ GEMM = 0.5 F_fwd
    # (its S and dP recompute, and the D = <O, dO> it computes on the way, are not credited).
    credit = {"attn_fwd": f_fwd, "bwd_dkdv": 2.0 * f_fwd, "bwd_dq": 0.5 * f_fwd}
    delta_bytes = 2.0 * B * S * Hq * D * 2 + 4.0 * B * Hq * S
    kernels = {}
    for name, avg in per.items():
        k = {"avg_ms": round(avg, 5)}
        if name in credit:
            k["tflops"] = round(credit[name] / (avg * 1e-3) / 1e12, 2)
            k["frac_peak"] = round(k["tflops"] / PEAK_FP16_TFLOPS, 4)
        else:
            k["gbps"] = round(delta_bytes / (avg * 1e-3) / 1e9, 1)
        kernels[name] = k
    dom = max(per, key=lambda n: per[n])
    dom_avg = per[dom]
    if dom in credit:
        ach = credit[dom] / (dom_avg * 1e-3) / 1e12
        roof = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_FP16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_FP16_TFLOPS, 4),
                "traffic": measured_traffic(dom) if args.config == "cfg3" else None,
                "traffic_source": TRAFFIC_SOURCE if args.config == "cfg3" else None,
                "avg_ms": round(dom_avg, 5), "flops_per_launch": credit[dom]}
    else:
        ach = delta_bytes / (dom_avg * 1e-3) / 1e9
        roof = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBPS,
                "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBPS, 4),
                "traffic": measured_traffic(dom) if args.config == "cfg3" else None,
                "traffic_source": TRAFFIC_SOURCE if args.config == "cfg3" else None,
                "avg_ms": round(dom_avg, 5)}

    value = f_total / (ms_step * 1e-3) / 1e12
    if cold is not None:
        cold["tflops"] = round(f_total / (cold["ms_per_step"] * 1e-3) / 1e12, 2)
    fwd_ms = per["attn_fwd"]
    res = {
        "metric": METRIC if args.config == "cfg3" else f"FlashAttn TFLOP/s ({args.config})",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": f"synthetic: Q/K/V, dO ~ N(0,1) (torch.randn on device, seeds 0/1), {dtype}",
        "config": {"workload": f"{args.config}: GQA attention {'fwd+bwd' if backward else 'fwd'}",
                   "B": B, "S": S, "Hq": Hq, "Hkv": Hkv, "D": D, "causal": causal,
                   "kv_len": kv_len, "scale": "1/sqrt(D)"},
        "frac_peak": round(value / PEAK_FP16_TFLOPS, 4),
        "fwd": {"ms": round(fwd_ms, 5), "tflops": kernels["attn_fwd"]["tflops"],
                "frac_peak": kernels["attn_fwd"]["frac_peak"]},
        "kernels": kernels,
        "kernel_timing": "after the timed region: K launches of each kernel back to back between two events",
        "timed_as": "one replay of a captured hipGraph of the K steps" if use_graph else "eager launches",
        "kernel_path": kernel_path,
        "roofline": roof,
        "cold_cache": cold,
        "wall_s": round(wall, 3),
    }
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or min(16, os.cpu_count() or 1)
        res["cpu_baseline"] = cpu_baseline(cfg, threads, 16 if args.config != "cfg5" else 1,
                                           args.cpu_runs)
    print(json.dumps(res))


if __name__ == "__main__":
    main()

"""The attention kernels on trained weights (GPU).

The forwards start each row's softmax offset m at the row maximum of the first 64-key tile and
move it only when they must: the D = 128 assembly forwards (fp16, bf16) when a later tile has a
score more than RESCALE_LOG2 = 15 log2 units above m (tokamak_amd/asmgen/attn_fwd.py), the HIP
forward (D = 64) when a tile's packed P overflows its 16-bit type or, in bf16, its packed P sum
reaches 65504 (tokamak_amd/csrc/attn_fwd.hip); both then rescale O and the row sums.  Random N(0,1) inputs
never do; trained attention that singles out a far key does.  This test trains, with the
runtime, tests/golden/models/induction.tkm (two layers, GQA 4:2, head dim 128, causal, in fp16
and in bf16)
and BASELINE config 4's decoder (tests/golden/models/cfg4_llama.tkm: 8 heads of 64, causal,
in fp16 and in bf16) on an induction task -- the second half of every sequence repeats the
first, so the loss of the second half can only fall through attention to the key half a
sequence back -- and then, on the actual input rows of its attention layers (all of the
induction model's, the first and last of config 4's):

- counts the (wave, tile) steps whose test moves m, by evaluating the kernel's own test on the
  CPU (scores (q . k) * scale * log2 e in fp32, m from the first tile, raised per wave), and
  reports the largest growth of a row's score over its first-tile maximum;
- checks the forward against the CPU oracle with the plain bar;
- checks the backward on the oracle's state (its O rounded to 16 bits and its LSE, the inputs
  tkm_attn_bwd receives) against the oracle's backward, and the backward on the GPU forward's
  own O and LSE against the oracle's backward on that same state.  Both use the plain bar
  widened by 16-bit rounding in a cancelling sum, atol + rtol |r| + 4 u sqrt(sum of the
  element's squared terms), u = 2^-11 (fp16) or 2^-8 (bf16): a trained head that puts nearly all of a row's weight
  on one key makes dS_ij = P_ij (dP_ij - O_i . dO_i) cancel, and the fp16 rounding of dS
  before its GEMM (tkm_gpu.cu:552 rounds it too) is then of the order of the bar.  The chain
  is not compared with the oracle's backward on the oracle's O: there the fp16 store of O
  (and the fp16 P of the forward's PV product, tkm_gpu.cu:402) moves O . dO by more than the
  cancelled difference, and even an exact backward on such an O misses the plain bar;
- times the forward against random inputs of the same shape (reported, not asserted: timing
  belongs to the bench).
"""
import ctypes
import json
import os
import time

import numpy as np
import pytest

import oracle
from attn_cases import (TOL_BWD, TOL_FWD, compare, fp16_forward_rescales, from_device, gradient_term_rms, log,
                        split_dqkv, to_device)

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
OP_GQA = 6


def _fixture(name):
    from tokamak_amd import runtime as R
    g = np.load(os.path.join(HERE, "golden", "tkm_graphs.npz"))
    return R.graph_buffer(g[name + "/graph"].tobytes()), json.loads(bytes(g[name + "/json"]).decode())


def _read16(ptr, n):
    """n 16-bit values from device memory (after the device is idle)."""
    import torch
    buf = np.empty(n, np.uint16)
    torch.cuda.synchronize()
    rc = ctypes.CDLL("libamdhip64.so").hipMemcpy(ctypes.c_void_p(buf.ctypes.data), ctypes.c_void_p(ptr),
                                                  ctypes.c_size_t(2 * n), 2)
    assert rc == 0
    return buf


def _time_fwd(qkv, B, S, Hq, Hkv, D, n=20):
    import torch
    from tokamak_amd import attn
    o, lse = attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=True)
    for _ in range(5):
        attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=True, out=o, lse=lse)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n):
        attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=True, out=o, lse=lse)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / n * 1e6


MODELS = [
    # name, storage type, vocabulary, steps, learning rate, forward kernel, attention layers checked
    ("induction", "f16", 256, 600, 0.05, "fwd_asm", None),
    ("induction", "bf16", 256, 600, 0.05, "fwd_asm", None),
    ("cfg4", "f16", 8192, 300, 0.01, "fwd_hip", (0, -1)),
    ("cfg4", "bf16", 8192, 300, 0.01, "fwd_hip", (0, -1)),
]


@pytest.mark.parametrize("name,dtype,V,steps,lr,kernel,pick", MODELS, ids=[f"{m[0]}-{m[1]}" for m in MODELS])
def test_trained_attention(gpu, name, dtype, V, steps, lr, kernel, pick):
    import torch
    from tokamak_amd.asmgen.attn_fwd import RESCALE_LOG2
    from tokamak_amd import attn
    from tokamak_amd import runtime as R
    buf, js = _fixture(name)
    B, S = js["batch_size"], js["nodes"][0]["W"]
    C0 = js["nodes"][0]["C"]
    rt = R.Runtime(buf, dtype=attn.F16 if dtype == "f16" else attn.BF16, token_labels=True, init_seed=3)
    rng = np.random.default_rng(5)
    emb = rng.standard_normal((V, C0)).astype(np.float32)
    half = S // 2

    def batch():
        first = rng.integers(0, V, (B, half))
        tok = np.concatenate([first, first], axis=1)
        y = np.concatenate([tok[:, 1:], np.zeros((B, 1), np.int64)], axis=1).astype(np.int32)
        return emb[tok].reshape(-1), y.reshape(-1), tok

    log(f"[case] {name}.tkm {dtype}: {steps} training steps, B{B} S{S}")
    losses = []
    for k in range(steps):
        x, y, _ = batch()
        losses.append(rt.step(x, y, lr if k < 2 * steps // 3 else 0.4 * lr))
    log(f"    loss: first {np.mean(losses[:10]):.3f}, last {np.mean(losses[-10:]):.3f} "
        f"(uniform guess {np.log(V):.3f}; the repeated half alone bounds it near {np.log(V) / 2:.3f})")
    assert np.all(np.isfinite(losses)) and np.mean(losses[-10:]) < np.mean(losses[:10]) - 0.5

    x, y, _ = batch()
    rt.step(x, y, 0.0)                       # the activations of one more batch, weights unchanged
    layers = [(i, n) for i, n in enumerate(js["nodes"]) if n["op"] == OP_GQA and not n["dead"]]
    if pick is not None:
        layers = [layers[i] for i in pick]
    dev = torch.device("cuda:0")
    u = 2.0 ** -11 if dtype == "f16" else 2.0 ** -8
    for li, (nid, n) in enumerate(layers):
        Hq, Hkv, D = n["q_heads"], n["kv_heads"], n["head_dim"]
        C = (Hq + 2 * Hkv) * D
        bits = _read16(rt.node_device(n["in0"]), B * S * C)
        xq = oracle.widen(bits, dtype).reshape(B, S, C)
        tested, rescaled, growth = fp16_forward_rescales(xq, B, S, Hq, Hkv, D, bool(n["causal"]))
        log(f"    layer {li}: largest score growth over the first tile's maximum {growth:.2f} log2 units; "
            f"the assembly forward's test would move m on {rescaled} of {tested} (wave, tile) steps "
            f"(threshold {RESCALE_LOG2})")
        qkv = to_device(bits, dtype, dev)
        o, lse = attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=True)
        assert attn.last_kernels() == [kernel]
        dout_f = rng.standard_normal((B, S, Hq * D)).astype(np.float32)
        dout_r, dout_bits = oracle.round_to(dout_f, dtype)
        o_ref, l_ref = oracle.fwd(xq, B, S, Hq, Hkv, D, causal=True, f64=True)
        res = [compare("O", from_device(o), o_ref, TOL_FWD), compare("LSE", from_device(lse), l_ref, TOL_FWD)]
        for st in res:
            log(f"      {st['name']:>3}: max_abs={st['max_abs']:.3e} bad={st['n_bad']}/{st['n']}")
        assert not any(st["n_bad"] for st in res)
        o_st, o_bits = oracle.round_to(o_ref, dtype)
        dout = to_device(dout_bits, dtype, dev)
        states = (("oracle state", o_st, l_ref, to_device(o_bits, dtype, dev), torch.from_numpy(np.ascontiguousarray(l_ref, np.float32)).to(dev)),
                  ("forward's state", from_device(o), from_device(lse), o, lse))
        for tag, o_np, l_np, o_dev, l_dev in states:
            dqkv = attn.gqa_bwd(qkv, o_dev, dout, l_dev, B, S, Hq, Hkv, D, causal=True)
            torch.cuda.synchronize()
            d_ref = oracle.bwd(xq, o_np, dout_r, l_np, B, S, Hq, Hkv, D, causal=True, f64=True)
            rms = gradient_term_rms(xq, o_np, dout_r, l_np, B, S, Hq, Hkv, D, causal=True)
            for nm, g_, r_, m_ in zip(("dQ", "dK", "dV"), split_dqkv(from_device(dqkv), B, S, Hq, Hkv, D),
                                      split_dqkv(d_ref, B, S, Hq, Hkv, D), rms):
                st = compare(nm, g_, r_, TOL_BWD)
                err = np.abs(g_ - r_)
                worst = float((err / (TOL_BWD[0] + TOL_BWD[1] * np.abs(r_) + 4 * u * m_)).max())
                log(f"      {nm} on the {tag}: max_abs={err.max():.3e} plain-bar misses={st['n_bad']} "
                    f"worst |g-r|/bound={worst:.3f}")
                assert worst <= 1.0, (tag, nm, worst)
        t_trained = _time_fwd(qkv, B, S, Hq, Hkv, D)
        rand = torch.randn((B, S, C), device=dev).to(qkv.dtype)
        t_rand = _time_fwd(rand, B, S, Hq, Hkv, D)
        log(f"      forward on these rows {t_trained:.1f} us, on random rows of the same shape {t_rand:.1f} us")
    rt.close()

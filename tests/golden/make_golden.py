"""Writes the golden attention fixtures (tests/golden/attn_golden.npz) with torch on the CPU.

Independent of the oracle's arithmetic: O via torch.nn.functional.scaled_dot_product_attention
in float64, LSE = logsumexp of the masked scaled scores, gradients by torch autograd in
float64.  Inputs come from the oracle's seeded generator (PCG32 + Box-Muller, rounded to the
case's dtype) so the test can regenerate them; an input checksum is stored with each case.
Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

# name: (B, S, Hq, Hkv, D, dtype, causal, kv_len, qkv seed, dO seed, subsample)
CASES = {
    # fp32 B2 H4 S128 D64 causal, Q/K/V seed 0, dO seed 1
    "cfg1": (2, 128, 4, 4, 64, "f32", True, None, 0, 1, 4096),
    "tiny_gqa_causal": (1, 17, 2, 1, 64, "f16", True, None, 5, 6, 0),
    "gqa_kvlen": (2, 40, 4, 2, 128, "f16", False, [40, 23], 7, 8, 2048),
    "bf16_causal_kvlen": (2, 33, 3, 3, 64, "bf16", True, [33, 9], 9, 10, 0),
    "s1": (2, 1, 2, 2, 128, "f16", False, None, 11, 12, 0),
}


def torch_reference(qkv, dout, B, S, Hq, Hkv, D, causal, kv_len):
    g = Hq // Hkv
    x = torch.tensor(qkv, dtype=torch.float64).view(B, S, Hq + 2 * Hkv, D)
    q = x[:, :, :Hq].permute(0, 2, 1, 3).clone().requires_grad_(True)
    k = x[:, :, Hq:Hq + Hkv].permute(0, 2, 1, 3).clone().requires_grad_(True)
    v = x[:, :, Hq + Hkv:].permute(0, 2, 1, 3).clone().requires_grad_(True)
    kr = k.repeat_interleave(g, dim=1)
    vr = v.repeat_interleave(g, dim=1)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    i = torch.arange(S).view(S, 1)
    j = torch.arange(S).view(1, S)
    vis = torch.ones(B, 1, S, S, dtype=torch.bool)
    if causal:
        vis = vis & (j <= i)
    if kv_len is not None:
        kl = torch.tensor(kv_len).view(B, 1, 1, 1)
        vis = vis & (j.view(1, 1, 1, S) < kl)
    o = torch.nn.functional.scaled_dot_product_attention(q, kr, vr, attn_mask=vis, scale=scale)
    scores = (q @ kr.transpose(-1, -2)) * scale
    lse = torch.logsumexp(scores.masked_fill(~vis, float("-inf")), dim=-1)
    do = torch.tensor(dout, dtype=torch.float64).view(B, S, Hq, D).permute(0, 2, 1, 3)
    (o * do).sum().backward()
    o_out = o.detach().permute(0, 2, 1, 3).reshape(B, S, Hq * D).numpy()
    dqkv = torch.cat([q.grad.permute(0, 2, 1, 3), k.grad.permute(0, 2, 1, 3),
                      v.grad.permute(0, 2, 1, 3)], dim=2).reshape(B, S, -1).numpy()
    return o_out, lse.detach().numpy(), dqkv


def main():
    out = {}
    for name, (B, S, Hq, Hkv, D, dt, causal, kv_len, s1, s2, sub) in CASES.items():
        inp = oracle.make_inputs(B, S, Hq, Hkv, D, dt, seed_qkv=s1, seed_do=s2)
        o, lse, dqkv = torch_reference(inp["qkv"], inp["dout"], B, S, Hq, Hkv, D, causal, kv_len)
        out[f"{name}/qkv_sum"] = np.array([inp["qkv"].astype(np.float64).sum(),
                                           np.abs(inp["qkv"]).astype(np.float64).sum()])
        out[f"{name}/lse"] = lse.astype(np.float32)
        for key, arr in (("o", o), ("dqkv", dqkv)):
            flat = arr.reshape(-1)
            if sub:
                rng = np.random.default_rng(1234)
                idx = np.sort(rng.choice(flat.size, size=sub, replace=False))
                out[f"{name}/{key}_idx"] = idx.astype(np.int32)
                out[f"{name}/{key}_val"] = flat[idx].astype(np.float32)
                out[f"{name}/{key}_headsum"] = arr.reshape(B, S, -1, D).sum(axis=(1, 3))
            else:
                out[f"{name}/{key}"] = arr.astype(np.float32)
    path = os.path.join(HERE, "attn_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()

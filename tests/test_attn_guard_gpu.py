"""Memory discipline of the attention kernels on the GPU: every tensor of a call lives inside a
larger buffer whose guard regions, before and after it, hold all-ones bytes (NaN for fp16,
bf16 and fp32); the outputs and the backward workspace start as all-ones too.

After the forward and the backward:
  - the guard regions are unchanged (nothing writes outside its tensor);
  - the results match the oracle, which fails on any NaN (an out-of-bounds read whose value
    reaches a result, or an output element or workspace byte some kernel should have written
    and did not, would show as NaN).
Shapes cover both kernel families (the assembly kernels for D=128, fp16 and bf16, the HIP
kernels for D=64), GQA, ragged S, per-batch key lengths with 0, and the causal diagonal."""
import pytest

import oracle
from attn_cases import TOL_BWD, TOL_FWD, compare, from_device, log, split_dqkv
from guarded import GUARD, Guarded, from_numpy16

CASES = [  # B, S, Hq, Hkv, D, dtype, causal, kv_len
    (2, 300, 4, 2, 128, "f16", True, None),
    (2, 333, 8, 2, 128, "f16", False, [333, 0]),
    (1, 6, 4, 2, 128, "f16", True, [2]),
    (3, 131, 4, 2, 128, "f16", True, None),
    (2, 200, 4, 4, 64, "f16", True, [77, 200]),
    (2, 129, 6, 2, 128, "bf16", True, None),
    (2, 333, 8, 2, 128, "bf16", False, [333, 0]),
    (1, 6, 4, 2, 128, "bf16", True, [2]),
    (1, 517, 2, 1, 64, "bf16", False, [300]),
]


def test_guard_helper_on_cpu():
    """The helper itself (on the CPU): the tensor starts as NaN, the guards report a single
    changed byte on either side, and writes inside the tensor leave them intact."""
    import torch
    g = Guarded(10, torch.float16, torch.device("cpu"))
    assert torch.isnan(g.t).all() and g.intact()
    g.t.fill_(1.0)
    assert g.intact()
    g.raw[GUARD - 1] = 0
    assert not g.intact()
    g.raw[GUARD - 1] = 255
    g.raw[GUARD + g.nbytes] = 7
    assert not g.intact()


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,Hq,Hkv,D,dtype,causal,kv_len", CASES)
def test_guarded_buffers(gpu, B, S, Hq, Hkv, D, dtype, causal, kv_len):
    import torch
    from tokamak_amd import attn
    log(f"[case] guarded B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} {dtype} causal={int(causal)} kv_len={kv_len}")
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, dtype, seed_qkv=3, seed_do=4, with_dout=True)
    C = (Hq + 2 * Hkv) * D
    qkv = Guarded(B * S * C, tdt, gpu)
    dout = Guarded(B * S * Hq * D, tdt, gpu)
    o = Guarded(B * S * Hq * D, tdt, gpu)
    lse = Guarded(B * Hq * S, torch.float32, gpu)
    dqkv = Guarded(B * S * C, tdt, gpu)
    ws = Guarded(attn.bwd_workspace_bytes(B, S, Hq), torch.uint8, gpu)
    bufs = [qkv, dout, o, lse, dqkv, ws]
    kvl = None
    if kv_len is not None:
        kvl = Guarded(B, torch.int32, gpu)
        kvl.t.copy_(torch.tensor(kv_len, dtype=torch.int32))
        bufs.append(kvl)
    qkv.t.copy_(from_numpy16(inp["qkv_bits"], dtype))
    dout.t.copy_(from_numpy16(inp["dout_bits"], dtype))
    attn.gqa_fwd(qkv.t, B, S, Hq, Hkv, D, causal=causal, kv_len=None if kvl is None else kvl.t,
                 out=o.t, lse=lse.t)
    attn.gqa_bwd(qkv.t, o.t, dout.t, lse.t, B, S, Hq, Hkv, D, causal=causal,
                 kv_len=None if kvl is None else kvl.t, dqkv=dqkv.t, workspace=ws.t)
    torch.cuda.synchronize()
    assert all(b.intact() for b in bufs), [i for i, b in enumerate(bufs) if not b.intact()]
    o_ref, lse_ref = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=causal, kv_len=kv_len, f64=True)
    res = [compare("O", from_device(o.t).reshape(o_ref.shape), o_ref, TOL_FWD),
           compare("LSE", from_device(lse.t).reshape(lse_ref.shape), lse_ref, TOL_FWD)]
    o_stored, _ = oracle.round_to(o_ref, dtype)
    d_ref = oracle.bwd(inp["qkv"], o_stored, inp["dout"], lse_ref, B, S, Hq, Hkv, D,
                       causal=causal, kv_len=kv_len, f64=True)
    got = split_dqkv(from_device(dqkv.t), B, S, Hq, Hkv, D)
    ref = split_dqkv(d_ref, B, S, Hq, Hkv, D)
    res += [compare(n, g, r, TOL_BWD) for n, g, r in zip(("dQ", "dK", "dV"), got, ref)]
    for st in res:
        log(f"    {st['name']:>3}: max_abs={st['max_abs']:.3e} bad={st['n_bad']}/{st['n']} "
            f"nonfinite={st['n_nonfinite_got']}")
    assert not [r for r in res if r["n_bad"]], res

"""tkm_attn_bwd_noalloc (static device scratch, no allocation) against tkm_attn_bwd (caller
workspace): bit-equal dQ, dK, dV on two calls in a row, the second with a smaller input, both
through the C ABI.  Also: a size beyond the static scratch is rejected before anything runs."""
import ctypes

import pytest

from attn_cases import log

pytestmark = pytest.mark.gpu


def _noalloc(L, qkv, o, dout, lse, dqkv, kv, B, S, Hq, Hkv, D, causal, dtype, stream):
    from tokamak_amd import attn
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    return L.tkm_attn_bwd_noalloc(p(qkv), p(o), p(dout), p(lse), p(dqkv), p(kv), B, S, Hq, Hkv,
                                  D, ctypes.c_float(attn.default_scale(D)), int(causal), dtype,
                                  ctypes.c_void_p(stream.cuda_stream))


def test_noalloc_matches_workspace_backward_twice(gpu):
    import torch
    from tokamak_amd import attn
    L = attn.lib()
    L.tkm_attn_bwd_noalloc.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 5 + \
        [ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    L.tkm_attn_bwd_noalloc.restype = ctypes.c_int
    stream = torch.cuda.current_stream()
    # config 3 (fp16, D 128: assembly kernels), then a smaller GQA bf16 D 64 case with kv_len
    # (HIP kernels): the second call finds the first call's values in the shared scratch.
    cases = [(4, 2048, 16, 16, 128, torch.float16, True, None),
             (2, 300, 4, 2, 64, torch.bfloat16, True, [300, 123])]
    for B, S, Hq, Hkv, D, dt, causal, kvl in cases:
        log(f"[case] noalloc backward B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} {dt} kv_len={kvl}")
        g = torch.Generator(device=gpu)
        g.manual_seed(B * 1000 + S)
        qkv = torch.randn((B, S, (Hq + 2 * Hkv) * D), generator=g, device=gpu).to(dt)
        dout = torch.randn((B, S, Hq * D), generator=g, device=gpu).to(dt)
        kv = None if kvl is None else torch.tensor(kvl, dtype=torch.int32, device=gpu)
        o, lse = attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=causal, kv_len=kv)
        ref = attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, causal=causal, kv_len=kv)
        ref_kernels = attn.last_kernels()
        got = torch.full_like(qkv, float("nan"))
        rc = _noalloc(L, qkv, o, dout, lse, got, kv, B, S, Hq, Hkv, D, causal,
                      attn.F16 if dt == torch.float16 else attn.BF16, stream)
        assert rc == 0, L.tkm_attn_last_error()
        assert attn.last_kernels() == ref_kernels, (attn.last_kernels(), ref_kernels)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), float((got.float() - ref.float()).abs().max())
        log(f"    dqkv bitwise equal to tkm_attn_bwd ({ref_kernels})")


def test_noalloc_rejects_beyond_scratch(gpu):
    """A problem whose workspace exceeds the static scratch is rejected before anything runs;
    every tensor is a real allocation of the size the call names, so the call could not touch
    memory outside them even if the check were gone (the rejection itself is also checked on
    the CPU, tests/test_abi.py)."""
    import torch
    from tokamak_amd import attn
    L = attn.lib()
    L.tkm_attn_bwd_noalloc.argtypes = [ctypes.c_void_p] * 6 + [ctypes.c_int] * 5 + \
        [ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    L.tkm_attn_bwd_noalloc.restype = ctypes.c_int
    B, S, Hq, Hkv, D = 1, 1 << 20, 4, 1, 64  # 4M (row, head) pairs: 48 MiB of workspace > 16 MiB
    assert L.tkm_attn_bwd_workspace_bytes(B, S, Hq) > 16 << 20
    qkv = torch.zeros((B, S, (Hq + 2 * Hkv) * D), dtype=torch.float16, device=gpu)
    o = torch.zeros((B, S, Hq * D), dtype=torch.float16, device=gpu)
    dout = torch.zeros_like(o)
    lse = torch.zeros((B, Hq, S), dtype=torch.float32, device=gpu)
    dqkv = torch.full_like(qkv, 1.0)
    rc = _noalloc(L, qkv, o, dout, lse, dqkv, None, B, S, Hq, Hkv, D, True, attn.F16,
                  torch.cuda.current_stream())
    torch.cuda.synchronize()
    assert rc == -4 and b"scratch" in L.tkm_attn_last_error()
    assert bool((dqkv == 1.0).all())   # nothing ran

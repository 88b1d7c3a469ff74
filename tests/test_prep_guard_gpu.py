"""Memory discipline of the generated qkv-prep kernels on the GPU, as for attention
(tests/test_attn_guard_gpu.py): every tensor of a forward and a backward lives inside an
all-ones (NaN) guarded buffer, outputs and the workspace start as NaN; afterwards the guards
are intact and every output matches the oracle at the bars of tests/test_prep_gpu.py."""
import numpy as np
import pytest

import oracle
from attn_cases import from_device, log
from guarded import Guarded, from_numpy16
from test_prep_gpu import check16, check_sum, make_case


@pytest.mark.gpu
@pytest.mark.parametrize("B,S,Hq,Hkv,D,qknorm,rope,dtype", [
    (2, 77, 4, 2, 64, True, True, "f16"),
    (1, 300, 2, 1, 128, False, True, "bf16"),
    (3, 33, 6, 3, 64, True, False, "bf16"),
    (1, 5, 8, 8, 64, False, False, "f16"),
])
def test_prep_guarded_buffers(gpu, B, S, Hq, Hkv, D, qknorm, rope, dtype):
    import torch
    from tokamak_amd import prep
    log(f"[case] guarded qkv-prep B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} qknorm={int(qknorm)} rope={int(rope)} {dtype}")
    rows = B * S
    c = make_case(rows, Hq, Hkv, D, dtype, 5)
    P = prep.Prep(Hq, Hkv, D, S, qknorm=qknorm, rope=rope, dtype=dtype, group_id=7)
    tdt = torch.float16 if dtype == "f16" else torch.bfloat16
    C, QK, NH = P.C, P.QK, P.NH
    x, out = Guarded(rows * C, tdt, gpu), Guarded(rows * C, tdt, gpu)
    bias = Guarded(C, torch.float32, gpu)
    dout, din = Guarded(rows * C, tdt, gpu), Guarded(rows * C, tdt, gpu)
    dbias = Guarded(C, torch.float32, gpu)
    ws = Guarded(max(P.bwd_workspace_bytes(rows), 1), torch.uint8, gpu)
    bufs = [x, out, bias, dout, din, dbias, ws]
    gamma = xhat = istd = dgamma = None
    if qknorm:
        gamma, dgamma = Guarded(QK, torch.float32, gpu), Guarded(QK, torch.float32, gpu)
        xhat, istd = Guarded(rows * QK, tdt, gpu), Guarded(rows * NH, torch.float32, gpu)
        bufs += [gamma, dgamma, xhat, istd]
        gamma.t.copy_(torch.from_numpy(c["gamma"]))
    x.t.copy_(from_numpy16(c["x_bits"], dtype))
    dout.t.copy_(from_numpy16(c["dout_bits"], dtype))
    bias.t.copy_(torch.from_numpy(c["bias"]))
    g = lambda b: None if b is None else b.t
    P.fwd(x.t, bias.t, g(gamma), out=out.t, xhat=g(xhat), istd=g(istd))
    P.bwd(dout.t, g(xhat), g(istd), g(gamma), din=din.t, dgamma=g(dgamma), dbias=dbias.t,
          workspace=ws.t)
    torch.cuda.synchronize()
    assert all(b.intact() for b in bufs), [i for i, b in enumerate(bufs) if not b.intact()]
    f = oracle.prep_inv_freq(D, theta=10000.0, scale=1.0, low=1.0, high=4.0, ocl=8192.0)
    ro, rxh, ris = oracle.prep_fwd(c["x"], c["bias"], c["gamma"], f, rows, S, Hq, Hkv, D, qknorm, rope, dtype)
    check16("out", from_device(out.t).reshape(ro.shape), ro, dtype)
    sx = si = None
    if qknorm:
        sx = from_device(xhat.t).reshape(rxh.shape)
        si = from_device(istd.t).reshape(ris.shape)
        check16("xhat", sx, rxh, dtype)
        np.testing.assert_allclose(si, ris, rtol=4e-6)
    rdin, rdg, rdb = oracle.prep_bwd(c["dout"], sx, si, c["gamma"], f, rows, S, Hq, Hkv, D, qknorm, rope, dtype)
    check16("din", from_device(din.t).reshape(rdin.shape), rdin, dtype)
    check_sum("dbias", dbias.t.cpu().numpy(), rdb, rows, 1.0)
    if qknorm:
        check_sum("dgamma", dgamma.t.cpu().numpy(), rdg, rows, 2.0)
    P.close()

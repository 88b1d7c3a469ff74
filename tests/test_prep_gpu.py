"""GPU parity of the generated qkv-prep kernels (hipRTC-compiled, launched through the C ABI
include/tkm_prep.h) against the CPU oracle oracle/qkv_prep_ref.c.

Bars, element-wise against the oracle on the same rounded inputs:
  out, xhat, din (16-bit)   |gpu - ref| <= 1 ulp of the storage type at |ref| + 1e-5 * max(1, |ref|max)
  istd (fp32)               relative 4e-6
  dbias, dgamma (fp32 sums) |gpu - ref| <= 1e-5 * |ref| + 2e-7 * rows * max(1, rms of the summands)
The oracle computes in double and rounds once; the kernels compute in fp32, so a result may
land on the other side of a rounding boundary (1 ulp).  The backward is checked on the state
the GPU forward saved (xhat, istd), so each kernel is tested on its own.
"""
import numpy as np
import pytest

import oracle
from attn_cases import from_device, log, to_device
from parity_checks import check16_mask

pytestmark = pytest.mark.gpu


def check16(name, got, ref, dtype):
    bad = check16_mask(got, ref, dtype, n_ulp=1, rel_floor=1e-5)
    diff = np.abs(np.asarray(got, np.float64) - np.asarray(ref, np.float64))
    log(f"    {name}: max_abs={np.nanmax(diff, initial=0.0):.3e} n_bad={int(bad.sum())}/{bad.size}")
    if bad.any():
        i = tuple(np.argwhere(bad)[0])
        pytest.fail(f"{name}: {int(bad.sum())} elements off, e.g. {i}: gpu {got[i]} ref {ref[i]}")


def check_sum(name, got, ref, rows, scale):
    got = np.asarray(got, np.float64)
    bound = 1e-5 * np.abs(ref) + 2e-7 * max(rows, 1) * max(1.0, scale)
    diff = np.abs(got - ref)
    log(f"    {name}: max_abs={diff.max(initial=0.0):.3e}")
    assert np.all(diff <= bound), (name, float(diff.max()), float(bound.min()))


def make_case(rows, Hq, Hkv, D, dtype, seed):
    C, QK = (Hq + 2 * Hkv) * D, (Hq + Hkv) * D
    rng = np.random.default_rng(seed)
    x_r, x_bits = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32) * 1.5, dtype)
    d_r, d_bits = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
    p_r, p_bits = oracle.round_to(rng.standard_normal((rows, C)).astype(np.float32), dtype)
    bias = (0.1 * rng.standard_normal(C)).astype(np.float32)
    gamma = (1.0 + 0.2 * rng.standard_normal(QK)).astype(np.float32)
    return dict(x=x_r, x_bits=x_bits, dout=d_r, dout_bits=d_bits, prev=p_r, prev_bits=p_bits,
                bias=bias, gamma=gamma)


def run_case(dev, B, S, Hq, Hkv, D, qknorm, rope, dtype, accumulate=False, seed=0, rope_args=None):
    import torch
    from tokamak_amd import prep
    rope_args = rope_args or {}
    rows = B * S
    tag = (f"B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} qknorm={int(qknorm)} rope={int(rope)} {dtype} "
           f"acc={int(accumulate)} rope_args={rope_args} seed={seed}")
    log(f"[case] qkv-prep {tag}")
    c = make_case(rows, Hq, Hkv, D, dtype, seed)
    P = prep.Prep(Hq, Hkv, D, S, qknorm=qknorm, rope=rope, dtype=dtype, group_id=seed, **rope_args)
    f = oracle.prep_inv_freq(D, theta=rope_args.get("theta", 10000.0), scale=rope_args.get("scale", 1.0),
                             low=rope_args.get("low_freq_factor", 1.0), high=rope_args.get("high_freq_factor", 4.0),
                             ocl=rope_args.get("original_context_length", 8192.0))
    x = to_device(c["x_bits"], dtype, dev)
    bias = torch.from_numpy(c["bias"]).to(dev)
    gamma = torch.from_numpy(c["gamma"]).to(dev)
    out, xhat, istd = P.fwd(x, bias, gamma if qknorm else None)
    torch.cuda.synchronize()
    ro, rxh, ris = oracle.prep_fwd(c["x"], c["bias"], c["gamma"], f, rows, S, Hq, Hkv, D, qknorm, rope, dtype)
    check16("out", from_device(out), ro, dtype)
    if qknorm:
        check16("xhat", from_device(xhat), rxh, dtype)
        gi = from_device(istd)
        np.testing.assert_allclose(gi, ris, rtol=4e-6)
    dout = to_device(c["dout_bits"], dtype, dev)
    din = to_device(c["prev_bits"], dtype, dev) if accumulate else None
    dbias0 = (0.5 * np.arange(P.C) / P.C).astype(np.float32)
    dgamma0 = (-0.25 * np.arange(P.QK) / P.QK).astype(np.float32)
    dbias = torch.from_numpy(dbias0).to(dev) if accumulate else None
    dgamma = (torch.from_numpy(dgamma0).to(dev) if accumulate else None) if qknorm else None
    din, dgamma, dbias = P.bwd(dout, xhat, istd, gamma if qknorm else None, din=din, dgamma=dgamma,
                               dbias=dbias, accumulate=accumulate)
    torch.cuda.synchronize()
    sx = from_device(xhat) if qknorm else None
    si = from_device(istd) if qknorm else None
    rdin, rdg, rdb = oracle.prep_bwd(c["dout"], sx, si, c["gamma"], f, rows, S, Hq, Hkv, D, qknorm, rope, dtype,
                                     din_prev=c["prev"] if accumulate else None)
    if accumulate:
        rdb = rdb + dbias0
        if qknorm:
            rdg = rdg + dgamma0
    check16("din", from_device(din), rdin, dtype)
    check_sum("dbias", dbias.cpu().numpy(), rdb, rows, 1.0)
    if qknorm:
        check_sum("dgamma", dgamma.cpu().numpy(), rdg, rows, 2.0)
    P.close()
    return P


@pytest.mark.parametrize("qknorm,rope", [(1, 1), (1, 0), (0, 1), (0, 0)], ids=["qkn+rope", "qkn", "rope", "bias"])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(2, 77, 4, 2, 64), (1, 300, 2, 1, 128), (3, 33, 6, 3, 64)],
                         ids=lambda s: "B{}S{}Hq{}Hkv{}D{}".format(*s))
def test_prep_parity(gpu, shape, dtype, qknorm, rope):
    B, S, Hq, Hkv, D = shape
    rope_args = {} if D == 64 else dict(theta=500000.0, scale=8.0, original_context_length=1024.0)
    run_case(gpu, B, S, Hq, Hkv, D, bool(qknorm), bool(rope), dtype, accumulate=(S == 33), seed=S,
             rope_args=rope_args)


def test_prep_config4(gpu):
    """Config 4's prep group: B8 S512 Hq=Hkv=8 D64, QKNorm + RoPE, fp16, gradients accumulated
    as the reference's step does."""
    run_case(gpu, 8, 512, 8, 8, 64, True, True, "f16", accumulate=True, seed=4)


def test_prep_llama3_rope(gpu):
    """llama3_style.tkm's RoPE (theta 5e5, scale 8, factors 1 / 4, context 8192), GQA 32/8, D128."""
    run_case(gpu, 1, 1024, 32, 8, 128, False, True, "bf16", seed=5,
             rope_args=dict(theta=500000.0, scale=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                            original_context_length=8192.0))


def test_prep_long_positions(gpu):
    """Angles up to 8191 rad: the fp32 angle, then an accurate sine / cosine."""
    run_case(gpu, 1, 8192, 1, 1, 128, True, True, "f16", seed=6)


def test_prep_deterministic_and_inplace(gpu):
    import torch
    from tokamak_amd import prep
    B, S, Hq, Hkv, D = 4, 200, 4, 2, 128
    rows = B * S
    c = make_case(rows, Hq, Hkv, D, "f16", 9)
    P = prep.Prep(Hq, Hkv, D, S, qknorm=True, rope=True)
    x = to_device(c["x_bits"], "f16", gpu)
    bias = torch.from_numpy(c["bias"]).to(gpu)
    gamma = torch.from_numpy(c["gamma"]).to(gpu)
    dout = to_device(c["dout_bits"], "f16", gpu)
    runs = []
    for _ in range(2):
        out, xhat, istd = P.fwd(x, bias, gamma)
        din, dg, db = P.bwd(dout, xhat, istd, gamma)
        torch.cuda.synchronize()
        runs.append([t.clone() for t in (out, xhat, istd, din, dg, db)])
    for a, b in zip(*runs):
        assert torch.equal(a, b)
    y = x.clone()
    P.fwd(y, bias, gamma, out=y)          # in place
    torch.cuda.synchronize()
    assert torch.equal(y, runs[0][0].view_as(y))
    P.close()


def test_prep_zero_rows(gpu):
    import torch
    from tokamak_amd import prep
    P = prep.Prep(2, 1, 64, 16, qknorm=True, rope=True)
    e16 = torch.empty((0, P.C), dtype=torch.float16, device=gpu)
    bias = torch.zeros(P.C, device=gpu)
    gamma = torch.ones(P.QK, device=gpu)
    out, xhat, istd = P.fwd(e16, bias, gamma, rows=0)
    db = torch.full((P.C,), 7.0, device=gpu)
    dg = torch.full((P.QK,), 7.0, device=gpu)
    P.bwd(e16, xhat, istd, gamma, rows=0, dgamma=dg, dbias=db, accumulate=True)
    torch.cuda.synchronize()
    assert torch.all(db == 7.0) and torch.all(dg == 7.0)
    P.bwd(e16, xhat, istd, gamma, rows=0, dgamma=dg, dbias=db, accumulate=False)
    torch.cuda.synchronize()
    assert torch.all(db == 0.0) and torch.all(dg == 0.0)
    P.close()

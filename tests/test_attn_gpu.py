"""GPU parity of the attention kernels (the gfx950 assembly kernels for D=128, the HIP kernels
for D=64; through the C ABI) against the CPU oracle.

Every case generates seeded inputs (oracle.make_inputs), runs tkm_attn_fwd / tkm_attn_bwd
on cuda:0 and the oracle on the identical rounded values, and checks
|gpu - ref| <= atol + rtol*|ref| with (2e-3, 1e-2) for O/LSE and (5e-3, 2e-2) for
dQ/dK/dV.
"""
import numpy as np
import pytest

import oracle
from attn_cases import TOL_BWD, TOL_FWD, compare, from_device, log, run_gpu_case, split_dqkv, to_device

pytestmark = pytest.mark.gpu


def _assert_ok(res):
    bad = [r for r in res if r["n_bad"]]
    assert not bad, bad


# (B, S, Hq, Hkv, D): ragged S (not multiples of any tile), S=1, GQA ratios 2/4/8.
SMALL = [
    (1, 1, 1, 1, 64),
    (1, 17, 2, 1, 64),
    (2, 100, 4, 2, 128),
    (1, 129, 3, 3, 128),
    (2, 333, 8, 2, 64),
    (1, 515, 8, 1, 128),
    (1, 1000, 2, 2, 128),
]


@pytest.mark.parametrize("shape", SMALL, ids=lambda s: "B{}S{}Hq{}Hkv{}D{}".format(*s))
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_small_shapes(gpu, shape, causal, dtype):
    B, S, Hq, Hkv, D = shape
    _assert_ok(run_gpu_case(gpu, B, S, Hq, Hkv, D, dtype=dtype, causal=causal))


@pytest.mark.parametrize("kv_len,causal,S,D", [
    ([300, 177], False, 300, 128),
    ([300, 177], True, 300, 64),
    ([1, 64], False, 200, 128),
    ([0, 129], False, 160, 64),     # a batch with no visible key: O = 0, LSE = -inf, grads 0
    ([0, 5], True, 96, 128),
    ([1000, 1], True, 1000, 64),
], ids=lambda v: str(v))
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_kv_len(gpu, kv_len, causal, S, D, dtype):
    _assert_ok(run_gpu_case(gpu, 2, S, 4, 2, D, dtype=dtype, causal=causal, kv_len=kv_len))


def _negative_scores(D):
    """Every visible score near -20 (q = a*u + noise, k = -a*u + noise, |u| = 1): each row's
    LSE is about -20 + log(visible keys), so exp(s - LSE) for a zero key past kv_len (s = 0)
    is ~1e7, above the fp16 range.  Keys past kv_len must get P = dS = 0 exactly."""
    a = np.sqrt(20.0 * np.sqrt(D))
    def fn(q, k, v):
        B, S = q.shape[:2]
        u = np.full(D, 1.0 / np.sqrt(D), np.float32)
        q = (q.reshape(B, S, -1, D) * 0.3 + a * u).reshape(B, S, -1)
        k = (k.reshape(B, S, -1, D) * 0.3 - a * u).reshape(B, S, -1)
        return q, k, v
    return fn


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_kv_len_negative_scores(gpu, causal, D, dtype):
    res = run_gpu_case(gpu, 2, 200, 4, 2, D, dtype=dtype, causal=causal, kv_len=[61, 137],
                       transform=_negative_scores(D))
    _assert_ok(res)


def test_config2_fwd(gpu):
    """fp16 causal B4 H8 S1024 D64, Q/K/V scaled by 0.5, forward."""
    _assert_ok(run_gpu_case(gpu, 4, 1024, 8, 8, 64, dtype="f16", causal=True, mul=0.5, bwd=False))


def test_config3_fwdbwd(gpu):
    """BASELINE config 3 (headline): fp16 causal B4 H16 S2048 D128, forward + backward."""
    _assert_ok(run_gpu_case(gpu, 4, 2048, 16, 16, 128, dtype="f16", causal=True, f64=False))


def test_config3_bf16(gpu):
    _assert_ok(run_gpu_case(gpu, 4, 2048, 16, 16, 128, dtype="bf16", causal=True, f64=False))


def test_gqa_equals_repeated_heads_full_size(gpu):
    """Config 3's size with GQA (Hq 16, Hkv 4): O, LSE and dQ are bit-equal to those of the MHA
    problem whose K and V heads repeat each kv head over its group of 4 (every q-head sees
    the same keys in the same order), and dK, dV equal that problem's per-head gradients
    summed over each group (fp32 sums on the host, so within rounding)."""
    import torch
    from tokamak_amd import attn
    B, S, Hq, Hkv, D = 4, 2048, 16, 4, 128
    g = Hq // Hkv
    log(f"[case] GQA vs repeated heads B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} f16 causal")
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f16", seed_qkv=21, seed_do=22)
    bits = inp["qkv_bits"].reshape(B, S, Hq + 2 * Hkv, D)
    rep = np.repeat(np.arange(Hkv), g)
    mha = np.concatenate([bits[:, :, :Hq], bits[:, :, Hq + rep], bits[:, :, Hq + Hkv + rep]], axis=2)
    dout = to_device(inp["dout_bits"], "f16", gpu)
    outs = {}
    for name, x, hkv in (("gqa", inp["qkv_bits"], Hkv), ("mha", mha.reshape(B, S, -1), Hq)):
        qkv = to_device(x, "f16", gpu)
        o, lse = attn.gqa_fwd(qkv, B, S, Hq, hkv, D, causal=True)
        dqkv = attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, hkv, D, causal=True)
        torch.cuda.synchronize()
        outs[name] = (from_device(o), from_device(lse), split_dqkv(from_device(dqkv), B, S, Hq, hkv, D))
    (o1, l1, (dq1, dk1, dv1)), (o2, l2, (dq2, dk2, dv2)) = outs["gqa"], outs["mha"]
    assert np.array_equal(o1, o2) and np.array_equal(l1, l2) and np.array_equal(dq1, dq2)
    for nm, got, per_head in (("dK", dk1, dk2), ("dV", dv1, dv2)):
        summed = per_head.reshape(B, S, Hkv, g, D).sum(axis=3)
        st = compare(nm, got, summed, TOL_BWD)
        log(f"    {nm}: max_abs={st['max_abs']:.3e} bad={st['n_bad']}/{st['n']}")
        assert not st["n_bad"], st


CFG5 = dict(B=2, S=8192, H=32, D=128, kvl=[8192, 5000])


@pytest.fixture(scope="module")
def cfg5_run(gpu):
    """BASELINE config 5 run once on the GPU: fp16 non-causal B2 H32 S8192 D128 with per-batch
    kv_len {8192, 5000} (3192 padded keys, a partial last tile), forward + backward at full
    size; the inputs and the outputs (host copies) for the per-head-group checks."""
    import torch
    from tokamak_amd import attn
    B, S, H, D, kvl = (CFG5[k] for k in ("B", "S", "H", "D", "kvl"))
    log(f"[case] config 5 B{B} S{S} Hq{H} Hkv{H} D{D} f16 causal=0 kv_len={kvl}")
    inp = oracle.make_inputs(B, S, H, H, D, "f16", seed_qkv=5, seed_do=6)
    qkv = to_device(inp["qkv_bits"], "f16", gpu)
    dout = to_device(inp["dout_bits"], "f16", gpu)
    kv = torch.tensor(kvl, dtype=torch.int32, device=gpu)
    o, lse = attn.gqa_fwd(qkv, B, S, H, H, D, causal=False, kv_len=kv)
    dqkv = attn.gqa_bwd(qkv, o, dout, lse, B, S, H, H, D, causal=False, kv_len=kv)
    torch.cuda.synchronize()
    out = dict(inp=inp, o=from_device(o), lse=from_device(lse), d=from_device(dqkv))
    del qkv, dout, o, lse, dqkv
    return out


@pytest.mark.parametrize("h0", [0, 8, 16, 24], ids=lambda h: f"heads{h}-{h + 7}")
def test_config5_fwdbwd_all_heads(cfg5_run, h0):
    """Config 5, every head over the four cases: heads are independent (Hq = Hkv), so the
    oracle runs on heads h0 .. h0+7 as the 8-head problem made of their Q, K, V and dO
    columns, covering O, LSE, dQ, dK and dV of every row of both batches."""
    B, S, H, D, kvl = (CFG5[k] for k in ("B", "S", "H", "D", "kvl"))
    inp, o_g, lse_g, d_g = cfg5_run["inp"], cfg5_run["o"], cfg5_run["lse"], cfg5_run["d"]
    heads = list(range(h0, h0 + 8))

    def cols(first):
        return np.concatenate([np.arange((first + h) * D, (first + h + 1) * D) for h in heads])
    n, qkv_cols = len(heads), np.concatenate([cols(0), cols(H), cols(2 * H)])
    log(f"[case] config 5 oracle on heads {h0}..{h0 + 7}")
    o_ref, lse_ref = oracle.fwd(inp["qkv"][:, :, qkv_cols], B, S, n, n, D, causal=False, kv_len=kvl)
    res = [compare(f"O[h{h0}+]", o_g[:, :, cols(0)], o_ref, TOL_FWD),
           compare(f"LSE[h{h0}+]", lse_g[:, heads, :], lse_ref, TOL_FWD)]
    d_ref = oracle.bwd(inp["qkv"][:, :, qkv_cols], oracle.round_to(o_ref, "f16")[0],
                       inp["dout"][:, :, cols(0)], lse_ref, B, S, n, n, D, causal=False, kv_len=kvl)
    for nm, g, r in zip(("dQ", "dK", "dV"), split_dqkv(d_g[:, :, qkv_cols], B, S, n, n, D),
                        split_dqkv(d_ref, B, S, n, n, D)):
        res.append(compare(f"{nm}[h{h0}+]", g, r, TOL_BWD))
    for st in res:
        log(f"    {st['name']:>9}: max_abs={st['max_abs']:.3e} max_rel={st['max_rel']:.3e} "
            f"bad={st['n_bad']}/{st['n']}")
    _assert_ok(res)


@pytest.mark.parametrize("causal", [True, False], ids=["causal", "full"])
@pytest.mark.parametrize("B,S", [(4, 2048), (8, 1000)], ids=["B4S2048", "B8S1000"])
def test_workspace_row_values(gpu, causal, B, S):
    """After the dQ stage that computes D (config 3: two items per workgroup, so item
    boundaries are exercised; S=1000 adds padding rows), the workspace holds D = <O, dO> per row
    and, per (batch, head)
    in tiles of 32 rows, -LSE*log2(e) then -D, padding rows zero.  D is checked against fp64
    sums of the same fp16 O and dO (fp32 accumulation order differs: rtol 1e-5)."""
    import torch
    from tokamak_amd import attn
    H, D = 16, 128
    log(f"[case] workspace row values B{B} S{S} H{H} D{D} causal={int(causal)}")
    g = torch.Generator(device=gpu)
    g.manual_seed(3)
    qkv = torch.randn(B, S, 3 * H * D, device=gpu, generator=g).half()
    dout = torch.randn(B, S, H * D, device=gpu, generator=g).half()
    o, lse = attn.gqa_fwd(qkv, B, S, H, H, D, causal=causal)
    nbytes = attn.bwd_workspace_bytes(B, S, H)
    ws = torch.full((nbytes,), 0x7F, dtype=torch.uint8, device=gpu)
    dqkv = torch.empty_like(qkv)
    attn.gqa_bwd(qkv, o, dout, lse, B, S, H, H, D, causal, None, dqkv=dqkv, workspace=ws,
                 stage=attn.BWD_DQ_DELTA)
    torch.cuda.synchronize()
    wsf = ws.view(torch.float32).cpu().numpy()
    o64 = o.float().cpu().numpy().astype(np.float64).reshape(B, S, H, D)
    do64 = dout.float().cpu().numpy().astype(np.float64).reshape(B, S, H, D)
    d_ref = np.einsum("bshd,bshd->bhs", o64, do64)                 # [B][H][S]
    d_gpu = wsf[:B * H * S].reshape(B, H, S)
    assert np.allclose(d_gpu, d_ref, rtol=1e-5, atol=1e-5), float(np.abs(d_gpu - d_ref).max())
    sp = (S + 31) // 32 * 32
    off = ((B * H * S * 4 + 255) // 256 * 256) // 4
    rows = wsf[off:off + B * H * sp * 2].reshape(B, H, sp // 32, 2, 32)
    nl2 = -lse.cpu().numpy().astype(np.float64) * 1.4426950408889634
    got_l = rows[:, :, :, 0, :].reshape(B, H, sp)
    got_d = rows[:, :, :, 1, :].reshape(B, H, sp)
    assert np.allclose(got_l[:, :, :S], nl2, rtol=1e-6, atol=1e-6)
    assert np.allclose(got_d[:, :, :S], -d_ref, rtol=1e-5, atol=1e-5)
    assert not got_l[:, :, S:].any() and not got_d[:, :, S:].any()


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_stage_schedules(gpu, D, dtype):
    """Both backward schedules: DELTA -> DKDV -> DQ and DQ_DELTA -> DKDV (tkm_attn_bwd's).
    Each matches the oracle; their D vectors agree to fp32 rounding (the two kernels sum the
    same products in different orders)."""
    import torch
    from tokamak_amd import attn
    B, S, Hq, Hkv = 2, 300, 4, 2
    log(f"[case] stage schedules B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} {dtype}")
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, dtype, seed_qkv=11, seed_do=12)
    qkv = to_device(inp["qkv_bits"], dtype, gpu)
    dout = to_device(inp["dout_bits"], dtype, gpu)
    kvl = torch.tensor([300, 211], dtype=torch.int32, device=gpu)
    o, lse = attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=True, kv_len=kvl)
    o_ref, lse_ref = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=True, kv_len=[300, 211], f64=True)
    d_ref = oracle.bwd(inp["qkv"], oracle.round_to(o_ref, dtype)[0], inp["dout"], lse_ref, B, S, Hq, Hkv, D,
                       causal=True, kv_len=[300, 211], f64=True)
    res, ds = {}, {}
    for name, stages in (("split", (attn.BWD_DELTA, attn.BWD_DKDV, attn.BWD_DQ)),
                         ("fused", (attn.BWD_DQ_DELTA, attn.BWD_DKDV))):
        ws = torch.zeros(attn.bwd_workspace_bytes(B, S, Hq), dtype=torch.uint8, device=gpu)
        dqkv = torch.empty_like(qkv)
        for st in stages:
            attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, causal=True, kv_len=kvl, dqkv=dqkv,
                         workspace=ws, stage=st)
        torch.cuda.synchronize()
        res[name] = from_device(dqkv)
        ds[name] = ws[:B * Hq * S * 4].view(torch.float32).cpu().numpy()
        for nm, g, r in zip(("dQ", "dK", "dV"), split_dqkv(res[name], B, S, Hq, Hkv, D),
                            split_dqkv(d_ref, B, S, Hq, Hkv, D)):
            st = compare(nm, g, r, TOL_BWD)
            log(f"    {name} {nm}: max_abs={st['max_abs']:.3e} bad={st['n_bad']}")
            assert not st["n_bad"], st
    np.testing.assert_allclose(ds["fused"], ds["split"], rtol=1e-5, atol=1e-6)
    d_whole = attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, causal=True, kv_len=kvl)
    torch.cuda.synchronize()
    assert np.array_equal(from_device(d_whole), res["fused"])


def test_deterministic(gpu):
    """The backward has no atomics: two runs are bitwise identical."""
    import torch
    from tokamak_amd import attn
    B, S, H, D = 2, 777, 4, 128
    inp = oracle.make_inputs(B, S, H, H, D, "f16", seed_qkv=3, seed_do=4)
    qkv = to_device(inp["qkv_bits"], "f16", gpu)
    dout = to_device(inp["dout_bits"], "f16", gpu)
    outs = []
    for _ in range(2):
        o, lse = attn.gqa_fwd(qkv, B, S, H, H, D, causal=True)
        d = attn.gqa_bwd(qkv, o, dout, lse, B, S, H, H, D, causal=True)
        torch.cuda.synchronize()
        outs.append((o.clone(), lse.clone(), d.clone()))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("causal,kv_len", [(True, None), (False, None), (False, 450), (True, 450)],
                         ids=["causal", "full", "full-kv450", "causal-kv450"])
@pytest.mark.parametrize("dtype,D,ramp", [("f16", 128, 40), ("bf16", 128, 40), ("f16", 64, 40),
                                          ("f16", 128, 90), ("bf16", 128, 90), ("bf16", 64, 90)],
                         ids=["f16", "bf16", "f16-d64", "f16-steep", "bf16-steep", "bf16-d64-steep"])
def test_growing_scores_move_m(gpu, causal, kv_len, dtype, D, ramp):
    """Scores that grow by ~40 or ~90 nats along the keys: the max from the first tile is stale
    by far more than the fp16 range.  The D = 128 assembly forwards (fp16 and bf16) raise m
    and rescale O and the row sums as the scores grow, before a P can pass 2^15; the HIP
    forward (D = 64) sees a tile's packed P overflow (fp16), or a tile's packed P sum reach
    65504 (bf16, where a growth of 40 nats stays inside the type's range and 90 nats, 2^130
    over the first tile, does not), rescales and repeats that tile's exp2.  With kv_len = 450 the largest
    scores lie past the visible
    keys, in the masked part of the last tile and beyond: m must follow the visible keys only
    (a rescale from unmasked scores would push every visible P below the fp16 range).  Must
    still match the oracle, and the rescale model (tests/attn_cases.py) must see m move."""
    import torch
    from tokamak_amd import attn
    from attn_cases import fp16_forward_rescales
    B, S, H = 1, 700, 2
    rng = np.random.default_rng(7)
    u = rng.standard_normal(D)
    u /= np.linalg.norm(u)
    x = np.zeros((B, S, 3 * H, D), dtype=np.float32)
    lin = np.linspace(0.0, 1.0, S)
    for h in range(H):
        x[0, :, h] = 8.0 * u + 0.3 * rng.standard_normal((S, D))                      # Q
        x[0, :, H + h] = (lin[:, None] * ramp * np.sqrt(D) / 8.0) * u \
            + 0.3 * rng.standard_normal((S, D))                                        # K
        x[0, :, 2 * H + h] = rng.standard_normal((S, D))                               # V
    qkv_r, bits = oracle.round_to(x.reshape(B, S, -1), dtype)
    log(f"[case] growing scores S{S} D{D} {dtype} ramp {ramp} causal={int(causal)} kv_len={kv_len}")
    qkv = to_device(bits, dtype, gpu)
    kvl = None if kv_len is None else torch.tensor([kv_len], dtype=torch.int32, device=gpu)
    o, lse = attn.gqa_fwd(qkv, B, S, H, H, D, causal=causal, kv_len=kvl)
    torch.cuda.synchronize()
    kvs = None if kv_len is None else [kv_len]
    o_ref, lse_ref = oracle.fwd(qkv_r, B, S, H, H, D, causal=causal, kv_len=kvs, f64=True)
    # the growth is real: some row's max score exceeds its max over keys 0..63 by > 20 nats
    xs = qkv_r.reshape(B, S, 3 * H, D).astype(np.float64)
    sc = np.einsum("sd,td->st", xs[0, :, 0], xs[0, :, H]) / np.sqrt(D)
    if causal:
        sc = np.where(np.tril(np.ones((S, S), dtype=bool)), sc, -np.inf)
    if kv_len is not None:
        sc[:, kv_len:] = -np.inf
    assert float((sc.max(axis=1) - sc[:, :64].max(axis=1)).max()) > 20.0
    if kv_len is None and D == 128:
        tested, rescaled, _ = fp16_forward_rescales(qkv_r, B, S, H, H, D, causal)
        log(f"    rescale model: {rescaled} of {tested} (wave, tile) steps move m")
        assert rescaled > 0
    res = [compare("O", from_device(o), o_ref, TOL_FWD), compare("LSE", from_device(lse), lse_ref, TOL_FWD)]
    for st in res:
        log(f"    {st['name']}: max_abs={st['max_abs']:.3e} bad={st['n_bad']}")
    _assert_ok(res)


def test_growing_scores_many_items(gpu):
    """Growing scores at config 3's size with GQA (B4 Hq16 Hkv4 S2048 D128, fp16, causal):
    512 work items over the persistent workgroups, so each walks several items in which m
    moves, through the DMA stream that runs across items.  Forward and backward against the
    oracle."""
    B, S, Hq, Hkv, D = 4, 2048, 16, 4, 128
    u = np.random.default_rng(11).standard_normal(D).astype(np.float32)
    u /= np.linalg.norm(u)
    lin = np.linspace(0.0, 1.0, S, dtype=np.float32)

    def grow(q, k, v):
        q = (0.3 * q.reshape(B, S, Hq, D) + 8.0 * u).reshape(B, S, Hq * D)
        k = (0.3 * k.reshape(B, S, Hkv, D) + (lin[None, :, None, None] * 40.0 * np.sqrt(D) / 8.0) * u)
        return q, k.reshape(B, S, Hkv * D).astype(np.float32), v

    from attn_cases import fp16_forward_rescales
    x = oracle.make_inputs(B, S, Hq, Hkv, D, "f16", seed_qkv=21, with_dout=False, transform=grow)["qkv"]
    x = x.reshape(B, S, Hq + 2 * Hkv, D)[:1, :, [0, Hq, Hq + Hkv]]       # batch 0, q-head 0 and its K, V
    tested, rescaled, growth = fp16_forward_rescales(x, 1, S, 1, 1, D, True)
    log(f"    head 0: m moves on {rescaled} of {tested} (wave, tile) steps; growth {growth:.1f} log2 units")
    assert rescaled > 0
    _assert_ok(run_gpu_case(gpu, B, S, Hq, Hkv, D, dtype="f16", causal=True, seed=21, transform=grow))


@pytest.mark.parametrize("dtype,D", [("bf16", 64), ("bf16", 128), ("f16", 64), ("f16", 128)])
def test_single_key_jump_keeps_o_finite(gpu, dtype, D):
    """One key whose score is 2^126 above every earlier score (87.3 nats) and whose V row is
    8: P V reaches 2^129, past fp32, while a bf16 P of 2^126 and a lane's row sum stay finite.
    The HIP forward must move m before that tile's PV product (it does when a lane's packed P
    sum reaches 65504; an earlier bound at infinity left O infinite, which a bf16 training
    run of BASELINE config 4's decoder hit), and the assembly forwards (D = 128, fp16 and
    bf16) when the score exceeds m by 15 log2 units.  Rows from the key on then take O = V of
    that key."""
    import torch
    from tokamak_amd import attn
    B, S, H, j = 1, 256, 2, 100
    rng = np.random.default_rng(3)
    u = rng.standard_normal(D)
    u /= np.linalg.norm(u)
    x = np.zeros((B, S, 3 * H, D), dtype=np.float32)
    for h in range(H):
        x[0, :, h] = 8.0 * u                                                            # Q
        x[0, :, H + h] = 0.05 * rng.standard_normal((S, D))                             # K
        x[0, j, H + h] = (87.3 * np.sqrt(D) / 8.0) * u
        x[0, :, 2 * H + h] = rng.standard_normal((S, D))                                # V
        x[0, j, 2 * H + h] = 8.0
    qkv_r, bits = oracle.round_to(x.reshape(B, S, -1), dtype)
    log(f"[case] single key jump S{S} D{D} {dtype}")
    qkv = to_device(bits, dtype, gpu)
    o, lse = attn.gqa_fwd(qkv, B, S, H, H, D, causal=True)
    torch.cuda.synchronize()
    o_ref, lse_ref = oracle.fwd(qkv_r, B, S, H, H, D, causal=True, f64=True)
    got = from_device(o)
    assert np.all(np.isfinite(got)) and np.all(np.isfinite(from_device(lse)))
    res = [compare("O", got, o_ref, TOL_FWD), compare("LSE", from_device(lse), lse_ref, TOL_FWD)]
    for st in res:
        log(f"    {st['name']}: max_abs={st['max_abs']:.3e} bad={st['n_bad']}")
    _assert_ok(res)


def _random_cases(seed, n):
    """Seeded shapes beyond the fixed cases: GQA ratios up to 8, ragged S, per-batch key
    lengths (0 and S included), both head dims and element types, causal or not."""
    import random
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        B, Hkv = rng.randint(1, 3), rng.randint(1, 2)
        Hq = Hkv * rng.choice((1, 2, 3, 4, 8))
        if B * Hq > 12:
            continue
        S = rng.choice((rng.randint(1, 128), rng.randint(129, 600)))
        kv_len = None
        if rng.random() < 0.4:
            kv_len = [rng.choice((0, S, rng.randint(0, S))) for _ in range(B)]
        D, dtype = rng.choice(((128, "f16"), (128, "f16"), (128, "bf16"), (64, "f16"), (64, "bf16")))
        out.append((B, S, Hq, Hkv, D, dtype, rng.random() < 0.6, kv_len, rng.randint(0, 1000)))
    return out


@pytest.mark.parametrize("B,S,Hq,Hkv,D,dtype,causal,kv_len,seed", _random_cases(11, 20))
def test_random_shapes(gpu, B, S, Hq, Hkv, D, dtype, causal, kv_len, seed):
    """Forward and backward of seeded random shapes against the oracle (the assembly kernels
    for D=128, the HIP kernels for D=64)."""
    _assert_ok(run_gpu_case(gpu, B, S, Hq, Hkv, D, dtype=dtype, causal=causal, kv_len=kv_len, seed=seed))


FEW_KEY_SHAPES = [
    (2, 168, 2, 1, 128, "f16", True, [4, 62], 407),
    (1, 327, 2, 1, 128, "f16", True, [2], 739),
    (1, 98, 8, 1, 128, "f16", True, [6], 448),
    (2, 300, 4, 2, 128, "f16", False, [3, 300], 8),
    (1, 200, 2, 2, 64, "bf16", True, [5], 9),
    (3, 1265, 32, 8, 64, "f16", True, [0, 464, 6], 7),
    (4, 1187, 32, 8, 128, "f16", True, [1187, 1187, 14, 1187], 93),
]


def _few_key_shapes(seed, n):
    """Seeded shapes whose rows see 1 to 16 keys (kv_len), the regime where every P is of
    order 1 and the dK / dV sums cancel."""
    import random
    rng = random.Random(seed)
    out = []
    while len(out) < n:
        B, Hkv = rng.randint(1, 2), rng.randint(1, 2)
        Hq = Hkv * rng.choice((1, 2, 4, 8))
        D, dt = rng.choice(((128, "f16"), (128, "f16"), (64, "f16"), (64, "bf16"), (128, "bf16")))
        out.append((B, rng.randint(8, 400), Hq, Hkv, D, dt, rng.random() < 0.6,
                    [rng.randint(1, 16) for _ in range(B)], rng.randint(0, 9999)))
    return out


@pytest.mark.parametrize("B,S,Hq,Hkv,D,dtype,causal,kv_len,seed", FEW_KEY_SHAPES + _few_key_shapes(5, 8))
def test_few_key_chain_within_rounding_bound(gpu, B, S, Hq, Hkv, D, dtype, causal, kv_len, seed):
    """Few visible keys, forward then backward from the GPU's own state, against the chained
    oracle.  O and LSE meet the bar against the exact oracle and against the one that follows
    the reference kernel's order of work with P rounded to fp16 (tkm_gpu.cu:359-435).  The
    gradients meet the bar widened by the size of 16-bit rounding in a cancelling sum:
    |g - r| <= atol + rtol |r| + 4 u sqrt(sum of the element's squared terms), u = 2^-11 (fp16)
    or 2^-8 (bf16).  With kv_len small, each dK / dV element sums hundreds of order-1 terms
    P dO (dS q) over the rows and heads of its group, and their sum can be 1000x smaller than
    their magnitudes; the fp16 rounding of P and dS before their GEMMs (which the reference
    also does, tkm_gpu.cu:402, 552) then leaves an error of order u sqrt(sum of squares),
    above the bar's 5e-3 absolute part.  A wrong or missing term
    (a whole P dO of order 1) stays far outside the widened bound."""
    import torch
    from tokamak_amd import attn
    from attn_cases import gradient_term_rms
    log(f"[case] few keys, chained: B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} {dtype} causal={int(causal)} "
        f"kv_len={kv_len} seed={seed}")
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, dtype, seed_qkv=seed, seed_do=seed + 1)
    qkv = to_device(inp["qkv_bits"], dtype, gpu)
    kvl = torch.tensor(kv_len, dtype=torch.int32, device=gpu)
    o, lse = attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=causal, kv_len=kvl)
    dqkv = attn.gqa_bwd(qkv, o, to_device(inp["dout_bits"], dtype, gpu), lse, B, S, Hq, Hkv, D,
                        causal=causal, kv_len=kvl)
    torch.cuda.synchronize()
    res = []
    for p16 in (False, True):
        o_r, l_r = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=causal, kv_len=kv_len, f64=True, p_f16=p16)
        res += [compare(n + ("/fp16 P" if p16 else ""), g, r, TOL_FWD)
                for n, g, r in (("O", from_device(o), o_r), ("LSE", from_device(lse), l_r))]
    o_ref, lse_ref = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=causal, kv_len=kv_len, f64=True)
    o_st, _ = oracle.round_to(o_ref, dtype)
    d_ref = oracle.bwd(inp["qkv"], o_st, inp["dout"], lse_ref, B, S, Hq, Hkv, D, causal=causal,
                       kv_len=kv_len, f64=True)
    rms = gradient_term_rms(inp["qkv"], o_st, inp["dout"], lse_ref, B, S, Hq, Hkv, D, causal=causal,
                            kv_len=kv_len)
    u = 2.0 ** -11 if dtype == "f16" else 2.0 ** -8
    for n, g, r, m in zip(("dQ", "dK", "dV"), split_dqkv(from_device(dqkv), B, S, Hq, Hkv, D),
                          split_dqkv(d_ref, B, S, Hq, Hkv, D), rms):
        bound = TOL_BWD[0] + TOL_BWD[1] * np.abs(r) + 4 * u * m
        err = np.abs(g - r)
        worst = float((err / bound).max())
        log(f"    {n}: max_abs={err.max():.3e} worst |g-r|/bound={worst:.3f}")
        assert np.all(err <= bound), (n, worst)
    for st in res:
        log(f"    {st['name']}: max_abs={st['max_abs']:.3e} bad={st['n_bad']}")
    _assert_ok(res)


@pytest.mark.parametrize("B,S,Hq,Hkv,D,dtype,causal,kv_len,seed", FEW_KEY_SHAPES)
def test_backward_on_forward_state(gpu, B, S, Hq, Hkv, D, dtype, causal, kv_len, seed):
    """The backward kernels on their own inputs: the oracle's backward takes the O and LSE that
    the GPU forward produced (what tkm_attn_bwd receives), so the forward's rounding drops out
    and what is left is the backward's own: its rounding of P and dS to the 16-bit type
    before their GEMMs (tkm_gpu.cu:402, 552 round them too), of order u sqrt(sum of the
    element's squared terms) in a sum that cancels.  The bar is the one of the chained test
    above, atol + rtol |r| + 4 u sqrt(sum of squares); most shapes meet the plain bar, and the
    log says how many elements do not.  The last two walk several rounds of work items (a
    batch with 6 or 14 visible keys per row, 4 q-heads per kv head), one for each kernel
    family."""
    import torch
    from tokamak_amd import attn
    from attn_cases import gradient_term_rms
    log(f"[case] backward on the forward's state B{B} S{S} Hq{Hq} Hkv{Hkv} D{D} {dtype} "
        f"causal={int(causal)} kv_len={kv_len} seed={seed}")
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, dtype, seed_qkv=seed, seed_do=seed + 1)
    qkv = to_device(inp["qkv_bits"], dtype, gpu)
    kvl = torch.tensor(kv_len, dtype=torch.int32, device=gpu)
    o, lse = attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=causal, kv_len=kvl)
    dqkv = attn.gqa_bwd(qkv, o, to_device(inp["dout_bits"], dtype, gpu), lse, B, S, Hq, Hkv, D,
                        causal=causal, kv_len=kvl)
    torch.cuda.synchronize()
    o_np, l_np = from_device(o), from_device(lse)
    d_ref = oracle.bwd(inp["qkv"], o_np, inp["dout"], l_np, B, S, Hq, Hkv, D,
                       causal=causal, kv_len=kv_len, f64=True)
    rms = gradient_term_rms(inp["qkv"], o_np, inp["dout"], l_np, B, S, Hq, Hkv, D, causal=causal,
                            kv_len=kv_len)
    u = 2.0 ** -11 if dtype == "f16" else 2.0 ** -8
    for n, g, r, m in zip(("dQ", "dK", "dV"), split_dqkv(from_device(dqkv), B, S, Hq, Hkv, D),
                          split_dqkv(d_ref, B, S, Hq, Hkv, D), rms):
        st = compare(n, g, r, TOL_BWD)
        bound = TOL_BWD[0] + TOL_BWD[1] * np.abs(r) + 4 * u * m
        err = np.abs(g - r)
        worst = float((err / bound).max())
        log(f"    {n}: max_abs={err.max():.3e} plain-bar misses={st['n_bad']}/{st['n']} "
            f"worst |g-r|/bound={worst:.3f}")
        assert np.all(err <= bound), (n, worst)


def test_kernel_paths(gpu):
    """Which kernels each configuration runs (tkm_attn_last_kernels): D=128 -- in fp16 the
    config-3 hot path -- and bf16 D=128 take the three gfx950 assembly kernels; D=64 the HIP
    kernels.  tkm_attn_init loads the code objects
    (the runtime calls it before capturing a step)."""
    import torch
    from tokamak_amd import attn
    attn.init()
    assert attn.asm_available()
    B, S, Hq, Hkv = 1, 300, 4, 2
    cases = [(128, torch.float16, ["fwd_asm"], ["dq_asm", "dkdv_asm"]),
             (128, torch.bfloat16, ["fwd_asm"], ["dq_asm", "dkdv_asm"]),
             (64, torch.float16, ["fwd_hip"], ["dq_hip", "dkdv_hip"]),
             (64, torch.bfloat16, ["fwd_hip"], ["dq_hip", "dkdv_hip"])]
    for D, dt, k_fwd, k_bwd in cases:
        log(f"[case] kernel path D{D} {dt}")
        qkv = torch.randn((B, S, (Hq + 2 * Hkv) * D), device=gpu).to(dt)
        dout = torch.randn((B, S, Hq * D), device=gpu).to(dt)
        o, lse = attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=True)
        assert attn.last_kernels() == k_fwd, (D, dt, attn.last_kernels())
        attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, causal=True)
        assert attn.last_kernels() == k_bwd, (D, dt, attn.last_kernels())
        ws = torch.empty(attn.bwd_workspace_bytes(B, S, Hq), dtype=torch.uint8, device=gpu)
        attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, causal=True, workspace=ws,
                     stage=attn.BWD_DELTA)
        assert attn.last_kernels() == ["delta_hip"]
    torch.cuda.synchronize()

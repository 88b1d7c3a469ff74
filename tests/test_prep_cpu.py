"""qkv-prep epilogue, HIP prelude and run-time compilation without a GPU.

1. The CPU oracle (oracle/qkv_prep_ref.c) is pinned by
   - the RoPE inverse frequency in closed form, exp(-ln(theta) * i / D) (the reference's
     exponent i/D, tkm_codegen.c:45-46), and the rescaled bands of tkm_codegen.c:47-62;
   - invariants: position 0 is the identity, rotation keeps each pair's norm, the inverse
     rotation undoes it, QKNorm output has unit RMS per head;
   - an independent float64 torch formulation (complex rotation, autograd backward) for the
     forward and the hand-written backward, and central finite differences;
   - planted mistakes that the checks above must catch.
2. The emitter produces sources that hipRTC compiles for gfx950, with the RoPE frequencies
   baked bit-exactly, no packed-fp32 instructions and no register spills.
3. The C ABI rejects bad descriptors and arguments before touching a device.
"""
import ctypes
import math
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

import oracle
from tokamak_amd import attn, prep

RNG = np.random.default_rng(1234)


def _rand_case(rows, Hq, Hkv, D, scale=1.0):
    C, QK = (Hq + 2 * Hkv) * D, (Hq + Hkv) * D
    x = (RNG.standard_normal((rows, C)) * scale).astype(np.float32)
    bias = (RNG.standard_normal(C) * 0.1).astype(np.float32)
    gamma = (1.0 + 0.2 * RNG.standard_normal(QK)).astype(np.float32)
    return x, bias, gamma


# ---- RoPE frequency -----------------------------------------------------------------------

@pytest.mark.parametrize("theta,D", [(10000.0, 64), (500000.0, 128), (1e6, 64)])
def test_inv_freq_closed_form(theta, D):
    f = oracle.prep_inv_freq(D, theta=theta)
    i = np.arange(D // 2)
    exact = np.exp(-np.log(theta) * i / D)                   # theta^(-i/D)
    # fp32 evaluation: ln(theta)*i rounded, divided, exp rounded: a few ulp of |ln(theta) i / D|
    tol = 4 * 2.0 ** -24 * (1.0 + np.log(theta) * i / D) + 2.0 ** -23
    assert np.all(np.abs(f / exact - 1.0) <= tol)
    # not the textbook theta^(-2i/D): pair 1 differs by a factor theta^(1/D)
    assert f[1] > 1.05 * theta ** (-2.0 / D)


@pytest.mark.parametrize("ocl", [8192.0, 1024.0])
def test_inv_freq_rescaled_bands(ocl):
    """scale > 1.  With llama3_style.tkm's values (theta 5e5, scale 8, factors 1 / 4, context
    8192) and the reference's exponent i/D, every wavelength is below 8192 (the longest is
    2 pi theta^(63/128) ~ 4.0e3), so only the short and middle bands occur; context 1024
    exercises all three."""
    D, theta, scale, low, high = 128, 500000.0, 8.0, 1.0, 4.0
    f = oracle.prep_inv_freq(D, theta, scale, low, high, ocl).astype(np.float64)
    base = oracle.prep_inv_freq(D, theta).astype(np.float64)
    wl = 2 * np.pi / base
    lo_wl, hi_wl = ocl / low, ocl / high
    far = np.abs(wl - lo_wl) > 1e-3 * lo_wl
    far &= np.abs(wl - hi_wl) > 1e-3 * hi_wl
    short = far & (wl < hi_wl)
    long_ = far & (wl > lo_wl)
    mid = far & (wl > hi_wl) & (wl < lo_wl)
    assert short.sum() and mid.sum()
    if ocl == 8192.0:
        assert long_.sum() == 0
    else:
        assert long_.sum() > 0
    np.testing.assert_allclose(f[short], base[short], rtol=0)
    np.testing.assert_allclose(f[long_], base[long_] / scale, rtol=1e-6)
    smooth = (ocl / wl[mid] - low) / (high - low)
    np.testing.assert_allclose(f[mid], base[mid] * (1 - smooth * (1 - 1 / scale)), rtol=2e-6)
    # the reference's middle band is not the published Llama-3 blend
    # ((1 - smooth) / scale + smooth): the two differ wherever 0 < smooth < 1
    published = base[mid] * ((1 - smooth) / scale + smooth)
    assert np.all(np.abs(f[mid] - published) > 1e-3 * published)


# ---- forward invariants -------------------------------------------------------------------

def test_rope_position0_identity_and_norm():
    Hq, Hkv, D, S = 4, 2, 64, 7
    rows = 3 * S
    QK = (Hq + Hkv) * D
    x, bias, _ = _rand_case(rows, Hq, Hkv, D)
    f = oracle.prep_inv_freq(D, theta=10000.0)
    out, _, _ = oracle.prep_fwd(x, bias, None, f, rows, S, Hq, Hkv, D, False, True, "f32")
    v = x.astype(np.float64) + bias
    for r in range(rows):
        if r % S == 0:
            np.testing.assert_allclose(out[r], v[r], rtol=1e-7, atol=1e-7)
    pn_out = np.hypot(out[:, 0:QK:2], out[:, 1:QK:2])
    pn_in = np.hypot(v[:, 0:QK:2], v[:, 1:QK:2])
    np.testing.assert_allclose(pn_out, pn_in, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(out[:, QK:], v[:, QK:], rtol=1e-7, atol=1e-7)   # V untouched


def test_rope_inverse_undoes_forward():
    Hq, Hkv, D, S = 2, 1, 128, 50
    rows = S
    x, bias, _ = _rand_case(rows, Hq, Hkv, D)
    f = oracle.prep_inv_freq(D, theta=500000.0, scale=8.0)
    out, _, _ = oracle.prep_fwd(x, np.zeros_like(bias), None, f, rows, S, Hq, Hkv, D, False, True, "f32")
    back, _, _ = oracle.prep_bwd(out, None, None, None, f, rows, S, Hq, Hkv, D, False, True, "f32")
    np.testing.assert_allclose(back, x, rtol=1e-6, atol=1e-6)


def test_qknorm_unit_rms_and_saved_state():
    Hq, Hkv, D, S = 4, 4, 64, 9
    rows = 2 * S
    QK, NH = (Hq + Hkv) * D, Hq + Hkv
    x, bias, gamma = _rand_case(rows, Hq, Hkv, D, scale=3.0)
    out, xhat, istd = oracle.prep_fwd(x, bias, np.ones_like(gamma), None, rows, S, Hq, Hkv, D, True, False, "f32")
    h = xhat.reshape(rows, NH, D).astype(np.float64)
    rms = np.sqrt((h ** 2).mean(-1))
    v = (x.astype(np.float64) + bias)[:, :QK].reshape(rows, NH, D)
    expect_rms = np.sqrt((v ** 2).mean(-1) / ((v ** 2).mean(-1) + 1e-5))
    np.testing.assert_allclose(rms, expect_rms, rtol=1e-6)
    np.testing.assert_allclose(istd, 1 / np.sqrt((v ** 2).mean(-1) + 1e-5), rtol=1e-6)
    np.testing.assert_allclose(out[:, :QK], xhat, rtol=1e-6, atol=1e-7)   # gamma = 1, no RoPE


# ---- independent float64 formulation (torch, autograd) --------------------------------------

def _torch_prep(x, bias, gamma, f32_freq, S, Hq, Hkv, D, qknorm, rope):
    """Forward in float64: complex rotation by exp(i * fp32(pos * inv_freq))."""
    import torch
    rows = x.shape[0]
    QK, NH = (Hq + Hkv) * D, Hq + Hkv
    v = x + bias
    qk = v[:, :QK].reshape(rows, NH, D)
    if qknorm:
        qk = qk * torch.rsqrt(qk.pow(2).mean(-1, keepdim=True) + 1e-5) * gamma.reshape(NH, D)
    if rope:
        pos = torch.arange(rows, dtype=torch.float32) % S
        ang = (pos[:, None] * torch.from_numpy(f32_freq)[None, :]).double()     # fp32 product
        z = torch.view_as_complex(qk.reshape(rows, NH, D // 2, 2).contiguous())
        z = z * torch.polar(torch.ones_like(ang), ang)[:, None, :]
        qk = torch.view_as_real(z).reshape(rows, NH, D)
    return torch.cat([qk.reshape(rows, QK), v[:, QK:]], dim=1)


@pytest.mark.parametrize("qknorm,rope", [(True, True), (True, False), (False, True), (False, False)])
@pytest.mark.parametrize("D", [64, 128])
def test_oracle_matches_autograd(qknorm, rope, D):
    import torch
    Hq, Hkv, S = 4, 2, 13
    rows = 3 * S - 2
    x, bias, gamma = _rand_case(rows, Hq, Hkv, D, scale=2.0)
    f = oracle.prep_inv_freq(D, theta=10000.0, scale=4.0, low=1.0, high=4.0, ocl=64.0)
    out, xhat, istd = oracle.prep_fwd(x, bias, gamma, f, rows, S, Hq, Hkv, D, qknorm, rope, "f32")
    tx = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    tb = torch.tensor(bias, dtype=torch.float64, requires_grad=True)
    tg = torch.tensor(gamma, dtype=torch.float64, requires_grad=True)
    ref = _torch_prep(tx, tb, tg, f, S, Hq, Hkv, D, qknorm, rope)
    np.testing.assert_allclose(out, ref.detach().numpy(), rtol=2e-6, atol=2e-6)
    dout = RNG.standard_normal(out.shape).astype(np.float32)
    (ref * torch.tensor(dout, dtype=torch.float64)).sum().backward()
    din, dgamma, dbias = oracle.prep_bwd(dout, xhat, istd, gamma, f, rows, S, Hq, Hkv, D, qknorm, rope, "f32")
    np.testing.assert_allclose(din, tx.grad.numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(dbias, tb.grad.numpy(), rtol=1e-5, atol=1e-5)
    if qknorm:
        np.testing.assert_allclose(dgamma, tg.grad.numpy(), rtol=1e-5, atol=1e-5)


def test_oracle_finite_differences():
    """Central differences of sum(out * w) against the oracle's backward (QKNorm + RoPE)."""
    Hq, Hkv, D, S = 2, 1, 64, 5
    rows = 6
    x, bias, gamma = _rand_case(rows, Hq, Hkv, D)
    f = oracle.prep_inv_freq(D)
    w = RNG.standard_normal((rows, (Hq + 2 * Hkv) * D)).astype(np.float32)

    def loss(xx, bb, gg):
        o, _, _ = oracle.prep_fwd(xx, bb, gg, f, rows, S, Hq, Hkv, D, True, True, "f32")
        return float((o.astype(np.float64) * w).sum())

    _, xhat, istd = oracle.prep_fwd(x, bias, gamma, f, rows, S, Hq, Hkv, D, True, True, "f32")
    din, dgamma, dbias = oracle.prep_bwd(w, xhat, istd, gamma, f, rows, S, Hq, Hkv, D, True, True, "f32")
    h = 1e-2
    for idx in [(0, 3), (2, 70), (5, 130), (4, 200)]:
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        fd = (loss(xp, bias, gamma) - loss(xm, bias, gamma)) / (2 * h)
        assert abs(fd - din[idx]) < 2e-3 * max(1.0, abs(fd)), (idx, fd, din[idx])
    for c in [1, 65, 150]:
        gp, gm = gamma.copy(), gamma.copy()
        gp[c] += h
        gm[c] -= h
        fd = (loss(x, bias, gp) - loss(x, bias, gm)) / (2 * h)
        assert abs(fd - dgamma[c]) < 2e-3 * max(1.0, abs(fd)), (c, fd, dgamma[c])
    for c in [0, 100, 250]:
        bp, bm = bias.copy(), bias.copy()
        bp[c] += h
        bm[c] -= h
        fd = (loss(x, bp, gamma) - loss(x, bm, gamma)) / (2 * h)
        assert abs(fd - dbias[c]) < 2e-3 * max(1.0, abs(fd)), (c, fd, dbias[c])


def test_accumulate_and_rounding():
    Hq, Hkv, D, S = 2, 2, 64, 4
    rows = 8
    x, bias, gamma = _rand_case(rows, Hq, Hkv, D)
    dout, _, _ = _rand_case(rows, Hq, Hkv, D)
    prev = RNG.standard_normal(dout.shape).astype(np.float32)
    prev16, _ = oracle.round_to(prev, "f16")
    d0, _, b0 = oracle.prep_bwd(dout, None, None, None, None, rows, S, Hq, Hkv, D, False, False, "f32")
    d1, _, b1 = oracle.prep_bwd(dout, None, None, None, None, rows, S, Hq, Hkv, D, False, False, "f16",
                                din_prev=prev16)
    np.testing.assert_array_equal(b0, b1)
    np.testing.assert_allclose(b0, dout.astype(np.float64).sum(0), rtol=1e-12)
    expect, _ = oracle.round_to(prev16.astype(np.float64) + d0.astype(np.float64), "f16")
    np.testing.assert_array_equal(d1, expect)
    # rounding helper: ties to even, overflow, subnormals
    assert oracle.prep_round(1 + 2 ** -11, "f16") == 1.0
    assert oracle.prep_round(1 + 3 * 2 ** -11, "f16") == 1 + 2 ** -9
    assert oracle.prep_round(65520.0, "f16") == math.inf
    assert oracle.prep_round(2 ** -25, "f16") == 0.0
    assert oracle.prep_round(3 * 2 ** -26, "f16") == 2 ** -24
    assert oracle.prep_round(1 + 2 ** -8, "bf16") == 1.0
    assert oracle.prep_round(1 + 3 * 2 ** -8, "bf16") == 1 + 2 ** -6


def test_planted_mistakes_are_caught():
    """Mistakes planted in the oracle's inputs must fail the checks above."""
    import torch
    Hq, Hkv, D, S = 2, 1, 64, 11
    rows = S
    x, bias, gamma = _rand_case(rows, Hq, Hkv, D)
    f = oracle.prep_inv_freq(D)
    tx = torch.tensor(x, dtype=torch.float64)
    ref = _torch_prep(tx, torch.tensor(bias, dtype=torch.float64), torch.tensor(gamma, dtype=torch.float64),
                      f, S, Hq, Hkv, D, True, True).numpy()
    # (a) rotation by the opposite angle (sign of sin flipped)
    bad, _, _ = oracle.prep_fwd(x, bias, gamma, -f, rows, S, Hq, Hkv, D, True, True, "f32")
    assert np.abs(bad - ref).max() > 1e-2
    # (b) textbook frequencies theta^(-2i/D) instead of the reference's theta^(-i/D)
    tb = np.exp(-np.log(10000.0) * 2 * np.arange(D // 2) / D).astype(np.float32)
    bad, _, _ = oracle.prep_fwd(x, bias, gamma, tb, rows, S, Hq, Hkv, D, True, True, "f32")
    assert np.abs(bad - ref).max() > 1e-2
    # (c) a bias dropped from the V part
    good, _, _ = oracle.prep_fwd(x, bias, gamma, f, rows, S, Hq, Hkv, D, True, True, "f32")
    b2 = bias.copy()
    b2[(Hq + Hkv) * D:] = 0
    bad, _, _ = oracle.prep_fwd(x, b2, gamma, f, rows, S, Hq, Hkv, D, True, True, "f32")
    assert np.abs(bad - good).max() > 1e-3
    # (d) QKNorm backward without the projection term m2 disagrees with autograd
    out, xhat, istd = oracle.prep_fwd(x, bias, np.ones_like(gamma), None, rows, S, Hq, Hkv, D, True, False, "f32")
    din, _, _ = oracle.prep_bwd(out, xhat, istd, np.ones_like(gamma), None, rows, S, Hq, Hkv, D, True, False, "f32")
    naive = out[:, :(Hq + Hkv) * D] * np.repeat(istd, D, axis=1)
    assert np.abs(din[:, :(Hq + Hkv) * D] - naive).max() > 1e-2


# ---- emitter + hipRTC ---------------------------------------------------------------------

VARIANTS = [
    dict(q_heads=8, kv_heads=8, head_dim=64, seq_len=512, qknorm=True, rope=True, dtype="f16"),
    dict(q_heads=32, kv_heads=8, head_dim=128, seq_len=2048, qknorm=False, rope=True, dtype="bf16",
         theta=500000.0, scale=8.0),
    dict(q_heads=4, kv_heads=2, head_dim=128, seq_len=100, qknorm=True, rope=False, dtype="f16"),
    dict(q_heads=2, kv_heads=1, head_dim=64, seq_len=1, qknorm=False, rope=False, dtype="bf16"),
]


def _objdump():
    for cand in ("/opt/rocm/llvm/bin/llvm-objdump", shutil.which("llvm-objdump")):
        if cand and os.path.exists(cand):
            return cand
    return None


@pytest.mark.parametrize("v", VARIANTS, ids=lambda v: "D{head_dim}_qkn{qknorm:d}_rope{rope:d}_{dtype}".format(**v))
def test_emitted_source_compiles(v, tmp_path):
    d = prep.make_desc(group_id=7, **v)
    src = prep.source(d)
    assert src.startswith(prep.prelude())
    for name in ("tkm_plasma_fwd_g7", "tkm_plasma_bwd_g7", "tkm_plasma_bwd_g7_reduce"):
        assert f"void {name}(" in src
    if v["rope"]:
        lits = re.search(r"tkm_inv_freq_g7\[(\d+)\] = \{([^}]*)\}", src)
        assert int(lits.group(1)) == v["head_dim"] // 2
        vals = np.array([float.fromhex(t.strip().rstrip("f")) for t in lits.group(2).split(",")], np.float32)
        want = oracle.prep_inv_freq(v["head_dim"], theta=v.get("theta", 10000.0), scale=v.get("scale", 1.0))
        np.testing.assert_array_equal(vals, want)       # bit-exact, baked in hex
    else:
        assert "tkm_inv_freq" not in src
    rc, code, log = prep.rtc_compile(src)
    assert rc == 0, log
    assert code[:4] == b"\x7fELF"
    co = tmp_path / "k.co"
    co.write_bytes(code)
    od = _objdump()
    if od:
        dis = subprocess.run([od, "-d", "--mcpu=gfx950", str(co)], capture_output=True, text=True).stdout
        assert "tkm_plasma_fwd_g7" in dis
        assert not re.search(r"v_pk_(add|mul|fma)_f32", dis)
        notes = subprocess.run([od.replace("objdump", "readelf"), "--notes", str(co)],
                               capture_output=True, text=True).stdout
        spills = [int(x) for x in re.findall(r"\.vgpr_spill_count:\s+(\d+)", notes)]
        assert spills and max(spills) == 0


def test_prelude_identifiers_compile():
    """Every identifier the reference's generated code takes from its prelude is defined."""
    body = r'''
extern "C" __global__ void probe(const __half2 *in, __half2 *out, const __half *img, float *f, uint32_t *u) {
    const int t = threadIdx.x;
    float2 v = __half22float2(__ldg(&in[t]));
    float s = subwarp_reduce_sum(v.x, 16) + tkm_sum_lanes8(v.y) + tkm_sum_lanes16(v.x);
    float sn, cs; __sincosf(s, &sn, &cs);
    s += __expf(sn) + __logf(cs + 2.f) + __sinf(s) + __cosf(s) + rsqrtf(2.f + s * s) + tanhf(s);
    out[t] = __float22half2_rn(make_float2(s, v.y));
    out[t + 64] = __floats2half2_rn(__half2float(__float2half(s)), 1.f);
    RngXorshift32 a; rng_init(&a, 1u, t); RngWangXorshift32 b; rng_init(&b, 2u, t);
    RngPcg32 c; rng_init(&c, 3u, t); RngPhilox d; rng_init(&d, 4u, t);
    u[t] = rng_u32(&a) ^ rng_u32(&b) ^ rng_u32(&c) ^ rng_u32(&d);
    float2 n = rng_normal2(&c);
    f[t] = n.x + rng_uniform(&d) + bilinear_sample_nhwc_h(img, 1.5f, 2.5f, 0, 8, 8, 3)
         + bilinear_sample_nhwc_reflect_h(img, -0.5f, 7.5f, 1, 8, 8, 3) + (float)tkm_reflect_idx(-3, 8);
    float w[8]; tkm_unpack_f16(make_uint4(u[0], u[1], u[2], u[3]), w);
    tkm_unpack_bf16(tkm_pack_bf16(w), w);
    uint4 p = tkm_pack_f16(w); u[t + 128] = p.x ^ p.w;
}
'''
    rc, code, log = prep.rtc_compile(prep.prelude() + body)
    assert rc == 0, log


def test_compile_error_is_reported():
    rc, code, log = prep.rtc_compile("extern \"C\" __global__ void k(float *x) { x[0] = undefined_name; }\n")
    assert rc == -6 and code == b"" and "undefined_name" in log
    assert b"undefined_name" in attn.lib().tkm_attn_last_error()


# ---- ABI ----------------------------------------------------------------------------------

@pytest.mark.parametrize("field,value,msg", [
    ("head_dim", 96, "head_dim"),
    ("q_heads", 3, "Hq"),
    ("kv_heads", 0, "Hq"),
    ("seq_len", 0, "seq_len"),
    ("has_rope", 2, "has_qknorm"),
    ("dtype", 5, "dtype"),
    ("rope_theta", 0.0, "RoPE"),
    ("rope_scale", 0.5, "RoPE"),
    ("rope_high_freq_factor", 0.5, "RoPE"),
    ("rope_original_context_length", float("nan"), "RoPE"),
])
def test_bad_descriptor_rejected(field, value, msg):
    d = prep.make_desc(4, 2, 64, 16, qknorm=True, rope=True)
    setattr(d, field, value)
    L = prep.lib()
    assert L.tkm_prep_source(ctypes.byref(d)) is None
    assert msg.encode() in L.tkm_attn_last_error()
    h = ctypes.c_void_p()
    assert L.tkm_prep_create(ctypes.byref(d), ctypes.byref(h)) != 0 and not h.value


def test_null_handles_rejected():
    L = prep.lib()
    P = ctypes.c_void_p(0x10000)
    assert L.tkm_prep_fwd(None, P, P, P, P, P, P, 4, None) == -1
    assert L.tkm_prep_bwd(None, P, P, P, P, P, P, P, 4, 0, P, 1 << 20, None) == -1
    assert L.tkm_prep_bwd_workspace_bytes(None, 4) == 0
    assert L.tkm_graph_begin(None) == -1
    assert L.tkm_graph_launch(None, None) == -1
    out = ctypes.c_void_p()
    assert L.tkm_graph_end(None, ctypes.byref(out)) == -1
    L.tkm_prep_destroy(None)
    L.tkm_graph_destroy(None)
    code, n = ctypes.c_void_p(), ctypes.c_size_t()
    assert L.tkm_rtc_compile(None, None, ctypes.byref(code), ctypes.byref(n), None) == -1


def test_prep_header_compiles_as_c99(tmp_path):
    c = tmp_path / "h.c"
    c.write_text('#include "tkm_prep.h"\nint main(void) { tkm_prep_desc d; tkm_prep_desc_init(&d); return d.head_dim != 64; }\n')
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror", "-pedantic", f"-I{attn.ROOT}/include",
                        str(c), "-o", str(tmp_path / "h"), f"-L{attn.PKG}", "-ltkm_attn",
                        f"-Wl,-rpath,{attn.PKG}"], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    assert subprocess.run([str(tmp_path / "h")]).returncode == 0

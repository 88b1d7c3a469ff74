"""The parity comparators must fail on planted NaN and inf outputs (CPU only)."""
import numpy as np
import pytest

from attn_cases import TOL_BWD, TOL_FWD, compare
from parity_checks import check16_mask


def _ref(seed=0, n=1000):
    return np.random.default_rng(seed).standard_normal(n)


@pytest.mark.parametrize("tol", [TOL_FWD, TOL_BWD])
def test_compare_passes_equal_and_close(tol):
    r = _ref()
    assert compare("x", r, r, tol)["n_bad"] == 0
    assert compare("x", r + 0.5 * tol[0], r, tol)["n_bad"] == 0
    assert compare("x", r + 3 * tol[0] + 2 * tol[1] * np.abs(r), r, tol)["n_bad"] == r.size


@pytest.mark.parametrize("planted", [np.nan, np.inf, -np.inf])
def test_compare_fails_on_nonfinite_output(planted):
    r = _ref()
    g = r.copy()
    g[17] = planted
    st = compare("x", g, r, TOL_FWD)
    assert st["n_bad"] == 1 and st["examples"][0][0] == (17,)
    st = compare("x", np.full_like(r, np.nan), r, TOL_FWD)
    assert st["n_bad"] == r.size


def test_compare_nonfinite_reference_needs_equal_value():
    r = _ref()
    r[:3] = [-np.inf, np.inf, -np.inf]   # rows with no visible key: LSE = -inf
    g = r.copy()
    assert compare("lse", g, r, TOL_FWD)["n_bad"] == 0
    for planted in (np.nan, 0.0, np.inf, -1e30):
        g2 = g.copy()
        g2[0] = planted
        assert compare("lse", g2, r, TOL_FWD)["n_bad"] == 1, planted


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("planted", [np.nan, np.inf, -np.inf])
def test_check16_fails_on_nonfinite_output(dtype, planted):
    r = _ref(1)
    assert not check16_mask(r, r, dtype, 1, 1e-5).any()
    g = r.copy()
    g[5] = planted
    bad = check16_mask(g, r, dtype, 1, 1e-5)
    assert bad.sum() == 1 and bad[5]
    assert check16_mask(np.full_like(r, np.nan), r, dtype, 2, 1e-4).all()


def test_check16_ulp_bound():
    r = np.array([1.0, 1.0, 1.0])
    g = np.array([1.0 + 2.0 ** -10, 1.0 + 2.0 ** -9, 1.0 - 2.0 ** -12])
    # fp16 ulp at 1.0 is 2^-10; bound = 1 ulp + 1e-6 * 1
    assert check16_mask(g, r, "f16", 1, 1e-6).tolist() == [False, True, False]


# ----------------------------------------------------- the rounding-aware gradient bound
def test_gradient_term_rms_closed_forms():
    """gradient_term_rms on cases with closed forms: one visible key gives P = 1, dS = 0, so
    dV_0's terms are the dO rows themselves (rms = sqrt(sum_i dO_i^2)) and dQ, dK have none;
    two visible keys give P_i0 = 1 / (1 + exp(s_1 - s_0))."""
    import oracle
    from attn_cases import gradient_term_rms
    B, S, Hq, Hkv, D = 1, 40, 2, 1, 64
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f16", seed_qkv=3, seed_do=4)
    do = inp["dout"].reshape(B, S, Hq, D).astype(np.float64)
    x = inp["qkv"].reshape(B, S, Hq + 2 * Hkv, D).astype(np.float64)
    sc = 1.0 / np.sqrt(np.float32(D))
    for kvl in (1, 2):
        o, lse = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=False, kv_len=[kvl], f64=True)
        rq, rk, rv = gradient_term_rms(inp["qkv"], o, inp["dout"], lse, B, S, Hq, Hkv, D, causal=False,
                                       kv_len=[kvl])
        if kvl == 1:
            np.testing.assert_allclose(rv[0, 0, 0], np.sqrt((do[0] ** 2).sum(axis=(0, 1))), rtol=1e-6)
            assert np.abs(rq).max() < 1e-6 and np.abs(rk).max() < 1e-6
        else:
            s0 = sc * np.einsum("ihd,d->ih", x[0, :, :Hq], x[0, 0, Hq])
            s1 = sc * np.einsum("ihd,d->ih", x[0, :, :Hq], x[0, 1, Hq])
            p0 = 1.0 / (1.0 + np.exp(s1 - s0))
            want = np.sqrt(np.einsum("ih,ihd->d", p0 ** 2, do[0] ** 2))
            np.testing.assert_allclose(rv[0, 0, 0], want, rtol=1e-6)
        assert np.all(rv[0, kvl:] == 0.0)       # keys past kv_len have no terms


def test_rounding_bound_catches_a_missing_term():
    """The widened gradient bound (atol + rtol |r| + 4 u rms, u = 2^-11) still fails a
    gradient that lacks one row's term P_i0 dO_i, in the most cancelling few-key case of the
    GPU suite, and passes the exact result perturbed by independent fp16 roundings of P."""
    import oracle
    from attn_cases import gradient_term_rms, split_dqkv
    B, S, Hq, Hkv, D = 1, 327, 2, 1, 128
    inp = oracle.make_inputs(B, S, Hq, Hkv, D, "f16", seed_qkv=739, seed_do=740)
    o, lse = oracle.fwd(inp["qkv"], B, S, Hq, Hkv, D, causal=True, kv_len=[2], f64=True)
    o_st, _ = oracle.round_to(o, "f16")
    d = oracle.bwd(inp["qkv"], o_st, inp["dout"], lse, B, S, Hq, Hkv, D, causal=True, kv_len=[2], f64=True)
    _, _, dv = split_dqkv(d, B, S, Hq, Hkv, D)
    _, _, rv = gradient_term_rms(inp["qkv"], o_st, inp["dout"], lse, B, S, Hq, Hkv, D, causal=True, kv_len=[2])
    bound = 5e-3 + 2e-2 * np.abs(dv) + 4 * 2.0 ** -11 * rv
    x = inp["qkv"].reshape(B, S, Hq + 2 * Hkv, D).astype(np.float64)
    do = inp["dout"].reshape(B, S, Hq, D).astype(np.float64)
    sc = 1.0 / np.sqrt(np.float32(D))
    s = sc * np.einsum("hd,jd->hj", x[0, 200, :Hq], x[0, :2, Hq])
    p = np.exp(s - lse[0, :, 200][:, None])                 # row 200's P over keys 0, 1
    missing = dv.copy()
    missing[0, 0, 0] -= p[0, 0] * do[0, 200, 0]
    assert np.any(np.abs(missing - dv) > bound)
    # fp16 rounding of every P before the dV product: within the bound
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    dv16 = np.zeros_like(dv[0, :, 0])
    for h in range(Hq):
        sc_all = sc * x[0, :, h] @ x[0, :, Hq].T
        P = np.where((j <= i) & (j < 2), np.exp(sc_all - lse[0, h][:, None]), 0.0)
        P16 = P.astype(np.float32).astype(np.float16).astype(np.float64)
        dv16 += P16.T @ do[0, :, h]
    err = np.abs(dv16 - dv[0, :, 0])
    assert np.all(err <= bound[0, :, 0]) and err.max() > 5e-3 * 0.2


def test_fp16_forward_rescales_flags_growth():
    """The CPU evaluation of the fp16 forward's lazy rescale: random N(0,1) rows never move m
    (their scores stay within a few log2 units of the first tile's maximum); keys whose
    scores grow along the sequence make the waves rescale, about once per growth of the
    threshold, and the reported growth says by how much."""
    import oracle
    from attn_cases import fp16_forward_rescales
    from tokamak_amd.asmgen.attn_fwd import RESCALE_LOG2
    B, S, Hq, Hkv, D = 1, 512, 2, 1, 128
    x = oracle.make_inputs(B, S, Hq, Hkv, D, "f16", seed_qkv=1)["qkv"].reshape(B, S, Hq + 2 * Hkv, D)
    tested, rescaled, growth = fp16_forward_rescales(x, B, S, Hq, Hkv, D, True)
    assert tested == Hq * sum(range(8)) and rescaled == 0 and growth < 8
    u = x[0, :, :Hq].mean(axis=(0, 1))
    u /= np.linalg.norm(u)
    for gr in (0.05, 0.4):
        y = x.copy()
        y[0, :, Hq:Hq + Hkv] += gr * np.arange(S)[:, None, None] * u
        y = y.astype(np.float16).astype(np.float32)
        tested, rescaled, growth = fp16_forward_rescales(y, B, S, Hq, Hkv, D, True)
        assert (rescaled > 0) == (growth > RESCALE_LOG2), (gr, rescaled, growth)
        assert gr < 0.1 or (growth > 40 and rescaled >= growth // RESCALE_LOG2), (gr, rescaled, growth)
        # a threshold above every growth never rescales; a tiny one rescales at every rise
        assert fp16_forward_rescales(y, B, S, Hq, Hkv, D, True, threshold=growth + 1)[1] == 0

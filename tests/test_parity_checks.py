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

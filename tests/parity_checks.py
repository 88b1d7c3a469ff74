"""Element-wise comparators shared by every GPU parity test (and pinned on the CPU by
tests/test_parity_checks.py).

Both treat a non-finite value as a failure unless the reference holds the same value:
  - where the reference is finite, an element passes only if |got - ref| <= bound, which is
    False for a NaN or an infinity in `got`;
  - where the reference is +-inf (LSE of a row with no visible key), `got` must equal it;
  - where the reference is NaN, `got` must be NaN as well.
"""
from __future__ import annotations

import numpy as np


def _nonfinite_bad(got: np.ndarray, ref: np.ndarray, fin: np.ndarray) -> np.ndarray:
    """Mask of failures among the entries where the reference is not finite."""
    nf = ~fin
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    return nf & ~same


def compare(name: str, got, ref, tol) -> dict:
    """numpy-allclose form |got - ref| <= atol + rtol*|ref| with tol = (atol, rtol); returns
    statistics with the failure count `n_bad` (NaN and inf in `got` count as failures)."""
    atol, rtol = tol
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    fin = np.isfinite(ref)
    with np.errstate(invalid="ignore", over="ignore"):
        diff = np.abs(got - ref)
        bound = atol + rtol * np.abs(ref)
        bad = fin & ~(diff <= bound)
    bad |= _nonfinite_bad(got, ref, fin)
    dfin = diff[fin]
    stats = {
        "name": name,
        "max_abs": float(np.nanmax(np.where(np.isnan(dfin), np.inf, dfin))) if dfin.size else 0.0,
        "max_rel": float(np.max(np.where(np.isnan(dfin), np.inf, dfin) /
                                np.maximum(np.abs(ref[fin]), 1e-6))) if dfin.size else 0.0,
        "n_bad": int(bad.sum()),
        "n_nonfinite_got": int((~np.isfinite(got)).sum()),
        "n": int(ref.size),
    }
    if stats["n_bad"]:
        idx = np.argwhere(bad)[:5]
        stats["examples"] = [(tuple(int(i) for i in ix), float(got[tuple(ix)]), float(ref[tuple(ix)]))
                             for ix in idx]
    return stats


def ulp(ref, dtype: str) -> np.ndarray:
    """Spacing of the 16-bit storage type (fp16 or bf16) at |ref| (subnormal spacing below the
    smallest normal)."""
    p, emin = (11, -14) if dtype == "f16" else (8, -126)
    r = np.asarray(ref, np.float64)
    a = np.maximum(np.abs(np.where(np.isfinite(r), r, 0.0)), 2.0 ** (emin - 30))
    return 2.0 ** (np.maximum(np.floor(np.log2(a)), emin) - (p - 1))


def check16_mask(got, ref, dtype: str, n_ulp: float, rel_floor: float) -> np.ndarray:
    """Failure mask of a 16-bit output: |got - ref| <= n_ulp ulps at |ref| plus
    rel_floor * max(1, max|ref|); NaN and inf in `got` fail unless the reference holds them."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (got.shape, ref.shape)
    fin = np.isfinite(ref)
    rmax = float(np.abs(ref[fin]).max(initial=0.0))
    with np.errstate(invalid="ignore", over="ignore"):
        bound = n_ulp * ulp(ref, dtype) + rel_floor * max(1.0, rmax)
        bad = fin & ~(np.abs(got - ref) <= bound)
    return bad | _nonfinite_bad(got, ref, fin)

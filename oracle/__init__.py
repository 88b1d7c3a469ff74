"""ctypes wrapper of the CPU oracles: attention (oracle/attn_ref.c), the qkv-prep
epilogue (oracle/qkv_prep_ref.c) and the plasma epilogues (oracle/plasma_ref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product path
(tokamak_amd/) never imports it.

Input convention (shared by every parity test): one PCG32 stream per tensor,
``seq`` = 1 for Q, 2 for K, 3 for V, 4 for dO; N(0,1) by Box-Muller, times
``mul``, rounded to the compute dtype (ties to even).  Q, K and V are drawn in
[B][S][H][D] order and packed as qkv[B][S][(Hq + 2*Hkv) * D] in Q | K | V
head order (reference: src/tkm_registry.c:736-748).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libattn_ref.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u16p = ctypes.POINTER(ctypes.c_uint16)


def build() -> str:
    """Compile the oracle with its Makefile (gcc + OpenMP)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.ar_pcg32_next.restype = ctypes.c_uint32
        L.ar_fill_normal.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float]
        L.ar_round_f16.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.ar_round_bf16.argtypes = [_f32p, _u16p, ctypes.c_size_t]
        L.ar_widen_f16.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.ar_widen_bf16.argtypes = [_u16p, _f32p, ctypes.c_size_t]
        L.ar_attn_fwd.argtypes = [_f32p, _f32p, _f32p, _i32p] + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.ar_attn_fwd_pround.argtypes = [_f32p, _f32p, _f32p, _i32p] + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_int]
        L.ar_attn_bwd.argtypes = [_f32p, _f32p, _f32p, _f32p, _f32p, _i32p] + [ctypes.c_int] * 5 + [ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.ar_set_threads.argtypes = [ctypes.c_int]
        L.ar_get_threads.restype = ctypes.c_int
        L.ar_online_cpus.restype = ctypes.c_int
        _f64p = ctypes.POINTER(ctypes.c_double)
        L.qp_round.argtypes = [ctypes.c_double, ctypes.c_int]
        L.qp_round.restype = ctypes.c_double
        L.qp_inv_freq.argtypes = [ctypes.c_float] * 5 + [ctypes.c_int, ctypes.c_int]
        L.qp_inv_freq.restype = ctypes.c_float
        L.qp_fwd.argtypes = [_f32p] * 4 + [ctypes.c_int] * 8 + [_f32p] * 3
        L.qp_bwd.argtypes = [_f32p] * 6 + [ctypes.c_int] * 8 + [_f32p, _f64p, _f64p]
        L.pr_op_flags.argtypes = [ctypes.c_int]
        L.pr_op_fwd.argtypes = [ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_double, ctypes.c_double]
        L.pr_op_fwd.restype = ctypes.c_double
        L.pr_op_grad.argtypes = [ctypes.c_int, ctypes.c_double, ctypes.c_double, ctypes.c_double, _f64p]
        L.pr_op_grad.restype = ctypes.c_double
        L.pr_rng_u32.argtypes = [ctypes.c_int, ctypes.c_uint, ctypes.c_uint, ctypes.c_int,
                                 ctypes.POINTER(ctypes.c_uint)]
        L.pr_drop_keep.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint, ctypes.c_int, ctypes.c_int,
                                   ctypes.c_float, ctypes.POINTER(ctypes.c_ubyte)]
        _lib = L
    return _lib


class _Pcg32(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64), ("inc", ctypes.c_uint64)]


def pcg32_sequence(initstate: int, initseq: int, n: int) -> np.ndarray:
    L = lib()
    rng = _Pcg32()
    L.ar_pcg32_seed(ctypes.byref(rng), ctypes.c_uint64(initstate), ctypes.c_uint64(initseq))
    return np.array([L.ar_pcg32_next(ctypes.byref(rng)) for _ in range(n)], dtype=np.uint32)


def _fp(a):
    return a.ctypes.data_as(_f32p)


def normal(n: int, seed: int, seq: int, mul: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().ar_fill_normal(_fp(out), n, seed, seq, mul)
    return out


def round_to(x: np.ndarray, dtype: str):
    """Round float32 array to fp16/bf16 (RNE); returns (rounded float32, uint16 bits)."""
    x = np.ascontiguousarray(x, dtype=np.float32).copy()
    bits = np.empty(x.shape, dtype=np.uint16)
    fn = {"f16": lib().ar_round_f16, "bf16": lib().ar_round_bf16}[dtype]
    fn(_fp(x), bits.ctypes.data_as(_u16p), x.size)
    return x, bits


def widen(bits: np.ndarray, dtype: str) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    fn = {"f16": lib().ar_widen_f16, "bf16": lib().ar_widen_bf16}[dtype]
    fn(bits.ctypes.data_as(_u16p), _fp(out), bits.size)
    return out


def make_inputs(B, S, Hq, Hkv, D, dtype="f16", seed_qkv=0, seed_do=1, mul=1.0, with_dout=True,
                transform=None):
    """Seeded packed qkv (and dO), rounded to dtype.  ``transform(q, k, v)`` may reshape the
    fp32 draws ([B, S, H*D] each) before rounding and returns the new (q, k, v).

    Returns dict with float32 views ``qkv``/``dout`` holding the rounded values
    and ``qkv_bits``/``dout_bits`` (uint16) for upload, or fp32 arrays when
    dtype == "f32"."""
    q = normal(B * S * Hq * D, seed_qkv, 1, mul).reshape(B, S, Hq * D)
    k = normal(B * S * Hkv * D, seed_qkv, 2, mul).reshape(B, S, Hkv * D)
    v = normal(B * S * Hkv * D, seed_qkv, 3, mul).reshape(B, S, Hkv * D)
    if transform is not None:
        q, k, v = transform(q, k, v)
    qkv = np.concatenate([q, k, v], axis=2).astype(np.float32)
    out = {}
    if dtype == "f32":
        out["qkv"] = np.ascontiguousarray(qkv)
    else:
        out["qkv"], out["qkv_bits"] = round_to(qkv, dtype)
    if with_dout:
        do = normal(B * S * Hq * D, seed_do, 4, 1.0).reshape(B, S, Hq * D)
        if dtype == "f32":
            out["dout"] = do
        else:
            out["dout"], out["dout_bits"] = round_to(do, dtype)
    return out


def _kv(kv_len, B):
    if kv_len is None:
        return None, None
    arr = np.ascontiguousarray(np.asarray(kv_len, dtype=np.int32).reshape(B))
    return arr, arr.ctypes.data_as(_i32p)


def set_threads(n: int) -> None:
    lib().ar_set_threads(int(n))


def threads() -> int:
    return lib().ar_get_threads()


def online_cpus() -> int:
    return lib().ar_online_cpus()


def fwd(qkv, B, S, Hq, Hkv, D, scale=None, causal=True, kv_len=None, f64=False, p_f16=False):
    """Returns (O [B][S][Hq*D], LSE [B][Hq][S]) as float32.  p_f16: the reference kernel's
    order of work, with P rounded to fp16 before the PV product (ar_attn_fwd_pround; f64 is
    then ignored: it computes in double apart from that rounding)."""
    qkv = np.ascontiguousarray(qkv, dtype=np.float32)
    assert qkv.size == B * S * (Hq + 2 * Hkv) * D
    scale = 1.0 / np.sqrt(np.float32(D)) if scale is None else scale
    o = np.empty((B, S, Hq * D), dtype=np.float32)
    lse = np.empty((B, Hq, S), dtype=np.float32)
    keep, kvp = _kv(kv_len, B)
    if p_f16:
        rc = lib().ar_attn_fwd_pround(_fp(qkv), _fp(o), _fp(lse), kvp, B, S, Hq, Hkv, D, float(scale),
                                      int(causal))
    else:
        rc = lib().ar_attn_fwd(_fp(qkv), _fp(o), _fp(lse), kvp, B, S, Hq, Hkv, D, float(scale), int(causal), int(f64))
    if rc != 0:
        raise ValueError("ar_attn_fwd rejected its arguments")
    return o, lse


def bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, scale=None, causal=True, kv_len=None, f64=False):
    """Returns dqkv [B][S][(Hq+2Hkv)*D] float32 (dQ | dK | dV)."""
    qkv = np.ascontiguousarray(qkv, dtype=np.float32)
    o = np.ascontiguousarray(o, dtype=np.float32)
    dout = np.ascontiguousarray(dout, dtype=np.float32)
    lse = np.ascontiguousarray(lse, dtype=np.float32)
    scale = 1.0 / np.sqrt(np.float32(D)) if scale is None else scale
    dqkv = np.empty_like(qkv)
    keep, kvp = _kv(kv_len, B)
    rc = lib().ar_attn_bwd(_fp(qkv), _fp(o), _fp(dout), _fp(lse), _fp(dqkv), kvp,
                           B, S, Hq, Hkv, D, float(scale), int(causal), int(f64))
    if rc != 0:
        raise ValueError("ar_attn_bwd rejected its arguments")
    return dqkv


# ---- qkv-prep epilogue (oracle/qkv_prep_ref.c) -------------------------------------------

PREP_DTYPES = {"f16": 0, "bf16": 1, "f32": 2}


def _f32c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a, typ=_f32p):
    return None if a is None else a.ctypes.data_as(typ)


def prep_round(x: float, dtype: str) -> float:
    return lib().qp_round(float(x), PREP_DTYPES[dtype])


def prep_inv_freq(D, theta=10000.0, scale=1.0, low=1.0, high=4.0, ocl=8192.0) -> np.ndarray:
    """fp32 RoPE inverse frequencies of pairs 0..D/2-1 (reference tkm_codegen.c:45-62)."""
    L = lib()
    return np.array([L.qp_inv_freq(theta, scale, low, high, ocl, D, i) for i in range(D // 2)],
                    dtype=np.float32)


def prep_fwd(x, bias, gamma, inv_freq, rows, S, Hq, Hkv, D, qknorm, rope, dtype="f16"):
    """Returns (out [rows][C], xhat [rows][QK] or None, istd [rows][Hq+Hkv] or None), float32."""
    C, QK, NH = (Hq + 2 * Hkv) * D, (Hq + Hkv) * D, Hq + Hkv
    x, bias = _f32c(x).reshape(rows, C), _f32c(bias)
    gamma = _f32c(gamma) if qknorm else None
    inv_freq = _f32c(inv_freq) if rope else None
    out = np.empty((rows, C), np.float32)
    xhat = np.empty((rows, QK), np.float32) if qknorm else None
    istd = np.empty((rows, NH), np.float32) if qknorm else None
    rc = lib().qp_fwd(_ptr(x), _ptr(bias), _ptr(gamma), _ptr(inv_freq), rows, S, Hq, Hkv, D,
                      int(qknorm), int(rope), PREP_DTYPES[dtype], _ptr(out), _ptr(xhat), _ptr(istd))
    if rc:
        raise ValueError("qp_fwd rejected its arguments")
    return out, xhat, istd


def prep_bwd(dout, xhat, istd, gamma, inv_freq, rows, S, Hq, Hkv, D, qknorm, rope, dtype="f16",
             din_prev=None):
    """Returns (din [rows][C] float32, dgamma [QK] float64 or None, dbias [C] float64)."""
    C, QK = (Hq + 2 * Hkv) * D, (Hq + Hkv) * D
    _f64p = ctypes.POINTER(ctypes.c_double)
    dout = _f32c(dout).reshape(rows, C)
    xhat = _f32c(xhat) if qknorm else None
    istd = _f32c(istd) if qknorm else None
    gamma = _f32c(gamma) if qknorm else None
    inv_freq = _f32c(inv_freq) if rope else None
    din_prev = None if din_prev is None else _f32c(din_prev).reshape(rows, C)
    din = np.empty((rows, C), np.float32)
    dgamma = np.empty(QK, np.float64) if qknorm else None
    dbias = np.empty(C, np.float64)
    rc = lib().qp_bwd(_ptr(dout), _ptr(xhat), _ptr(istd), _ptr(gamma), _ptr(inv_freq), _ptr(din_prev),
                      rows, S, Hq, Hkv, D, int(qknorm), int(rope), PREP_DTYPES[dtype], _ptr(din),
                      _ptr(dgamma, _f64p), _ptr(dbias, _f64p))
    if rc:
        raise ValueError("qp_bwd rejected its arguments")
    return din, dgamma, dbias


# ---- plasma epilogues (oracle/plasma_ref.c) ------------------------------------------------

class _PrNode(ctypes.Structure):
    _fields_ = [("op", ctypes.c_int), ("fval", ctypes.c_float)]


class _PrParams(ctypes.Structure):
    _fields_ = [("w", ctypes.POINTER(_f32p)), ("beta", ctypes.POINTER(_f32p)),
                ("bias", ctypes.POINTER(_f32p)), ("branch", ctypes.POINTER(_f32p)),
                ("keep", ctypes.POINTER(ctypes.POINTER(ctypes.c_ubyte)))]


PR_W, PR_BETA, PR_BIAS, PR_NORM, PR_BRANCH, PR_MASK = 1, 2, 4, 8, 16, 32


def rng_u32(rng_type: int, seed: int, idx: int, n: int) -> np.ndarray:
    """n draws of the prelude's generator `rng_type` (1..4) after rng_init(seed, idx)."""
    out = np.zeros(n, np.uint32)
    rc = lib().pr_rng_u32(rng_type, seed & 0xFFFFFFFF, idx & 0xFFFFFFFF, n,
                          out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint)))
    if rc:
        raise ValueError("pr_rng_u32 rejected its arguments")
    return out


def drop_keep(rows: int, C: int, step_seed: int, node_id: int, rng_type: int, p: float) -> np.ndarray:
    """Drop's keep bits [rows][C] (uint8 0/1) for a step seed, node and generator."""
    keep = np.zeros((rows, C), np.uint8)
    rc = lib().pr_drop_keep(rows, C, step_seed & 0xFFFFFFFF, node_id, rng_type, p,
                            keep.ctypes.data_as(ctypes.POINTER(ctypes.c_ubyte)))
    if rc:
        raise ValueError("pr_drop_keep rejected its arguments")
    return keep


def plasma_flags(op: int) -> int:
    return lib().pr_op_flags(op)


def plasma_op(op, fv, x, w=0.0, b=0.0):
    return lib().pr_op_fwd(op, fv, x, w, b)


def plasma_op_grad(op, fv, p, w=0.0):
    dw = ctypes.c_double()
    d = lib().pr_op_grad(op, fv, p, w, ctypes.byref(dw))
    return d, dw.value


def _ptr_array(n, get):
    arr = (_f32p * max(n, 1))()
    keep = []
    for k in range(n):
        a = get(k)
        if a is not None:
            a = _f32c(a)
            keep.append(a)
            arr[k] = a.ctypes.data_as(_f32p)
    return arr, keep


def _params(nodes, params):
    n = len(nodes)
    P = _PrParams()
    keep = []
    for field in ("w", "beta", "bias", "branch"):
        arr, kp = _ptr_array(n, lambda k, f=field: params.get((f, k)))
        keep += kp + [arr]
        setattr(P, field, ctypes.cast(arr, ctypes.POINTER(_f32p)))
    _u8p = ctypes.POINTER(ctypes.c_ubyte)
    karr = (_u8p * max(n, 1))()
    for k in range(n):
        m = params.get(("keep", k))
        if m is not None:
            m = np.ascontiguousarray(m, dtype=np.uint8)
            keep.append(m)
            karr[k] = m.ctypes.data_as(_u8p)
    keep.append(karr)
    P.keep = ctypes.cast(karr, ctypes.POINTER(_u8p))
    return P, keep


def plasma_fwd(x, rows, C, nodes, params, twin=False, n_left=0, n_right=0, dtype="f16"):
    """nodes: [(op, fval)] (twin: left, right, then post); params: {("w"|"beta"|"bias"|"branch", k): array}.
    Returns out [rows][C] and the saved state {k: xhat [rows][C]}, {k: istd [rows][ceil(C/64)]}."""
    n = len(nodes)
    NG = (C + 63) // 64
    arr_nodes = (_PrNode * max(n, 1))(*[_PrNode(op, fv) for op, fv in nodes])
    P, keep = _params(nodes, params)
    xhat = {k: np.zeros((rows, C), np.float32) for k, (op, _) in enumerate(nodes) if plasma_flags(op) & PR_NORM}
    istd = {k: np.zeros((rows, NG), np.float32) for k in xhat}
    xa, _ = _ptr_array(n, lambda k: None)
    ia, _ = _ptr_array(n, lambda k: None)
    for k in xhat:
        xa[k] = xhat[k].ctypes.data_as(_f32p)
        ia[k] = istd[k].ctypes.data_as(_f32p)
    x = _f32c(x)
    out = np.empty((rows, C), np.float32)
    n_main = n - (n_left + n_right if twin else 0)
    rc = lib().pr_fwd(_ptr(x), rows, C, int(twin), arr_nodes, n_left, n_right, n_main, ctypes.byref(P),
                      PREP_DTYPES[dtype], _ptr(out), xa, ia)
    if rc:
        raise ValueError("pr_fwd rejected its arguments")
    return out, xhat, istd


def plasma_bwd(dout, x, rows, C, nodes, params, xhat, istd, twin=False, n_left=0, n_right=0, dtype="f16",
               acc_flags=0, din_prev=None, dbranch_prev=None, grads_prev=None):
    """Returns din, {k: dbranch}, {("dw"|"dbeta"|"dbias", k): float64 array}."""
    _f64p = ctypes.POINTER(ctypes.c_double)
    n = len(nodes)
    arr_nodes = (_PrNode * max(n, 1))(*[_PrNode(op, fv) for op, fv in nodes])
    P, keep = _params(nodes, params)
    W = 2 * C if twin else C
    din = np.zeros((rows, W), np.float32) if din_prev is None else _f32c(din_prev).reshape(rows, W).copy()
    xa, k1 = _ptr_array(n, lambda k: xhat.get(k))
    ia, k2 = _ptr_array(n, lambda k: istd.get(k))
    dbr = {}
    da, _ = _ptr_array(n, lambda k: None)
    grads = {}
    ga = {f: (_f64p * max(n, 1))() for f in ("dw", "dbeta", "dbias")}
    for k, (op, _) in enumerate(nodes):
        fl = plasma_flags(op)
        if fl & PR_BRANCH:
            prev = None if dbranch_prev is None else dbranch_prev.get(k)
            dbr[k] = np.zeros((rows, C), np.float32) if prev is None else _f32c(prev).copy()
            da[k] = dbr[k].ctypes.data_as(_f32p)
        for f, bit in (("dw", PR_W), ("dbeta", PR_BETA), ("dbias", PR_BIAS)):
            if fl & bit:
                prev = None if grads_prev is None else grads_prev.get((f, k))
                grads[(f, k)] = np.zeros(C) if prev is None else np.array(prev, np.float64)
                ga[f][k] = grads[(f, k)].ctypes.data_as(_f64p)
    n_main = n - (n_left + n_right if twin else 0)
    rc = lib().pr_bwd(_ptr(_f32c(dout)), _ptr(_f32c(x)), rows, C, int(twin), arr_nodes, n_left, n_right, n_main,
                      ctypes.byref(P), xa, ia, PREP_DTYPES[dtype], acc_flags, _ptr(din), da,
                      ga["dw"], ga["dbeta"], ga["dbias"])
    if rc:
        raise ValueError("pr_bwd rejected its arguments")
    return din, dbr, grads

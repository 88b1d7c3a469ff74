"""Python binding of the plasma-epilogue C ABI (include/tkm_plasma.h, libtkm_attn.so).

A plasma group is a chain of row-wise ops fused behind a GEMM, generated as HIP C and compiled
with hipRTC (reference src/tkm_codegen.c:297-625, op registry src/tkm_registry.c).  The chain
is given as a list of ``(op_name, fval)`` pairs (fval None = the registry default); tensors
are torch device tensors keyed by argument kind and node index.  Launches go through the C ABI
on the caller's current torch stream; there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
import re

from . import attn, prep
from .attn import AttnError, BF16, F16

HEADER = os.path.join(attn.ROOT, "include", "tkm_plasma.h")

OP_NAMES = ["Bias", "RMSNorm", "LN", "BN", "L2Norm", "SiLU", "ReLU", "ReLU2", "LeakyReLU", "ELU", "GELU",
            "Mish", "HardSwish", "HardSigmoid", "Tanh", "Sigmoid", "SwishBeta", "Sin", "CosGate", "SoftCap",
            "Clamp", "Scale", "LayerScale", "DyT", "PReLU", "xATLU", "Softplus", "Snake", "Add", "Drop",
            # ops whose code only the registry holds (whole-graph generator with the front end
            # linked); the descriptor API rejects them
            "Formula", "FormulaW", "FormulaB"]
FORMULA_OPS = ("Formula", "FormulaW", "FormulaB")
OPS = {n: i for i, n in enumerate(OP_NAMES)}
ARG_KINDS = ["in", "out", "dout", "din", "w", "beta", "bias", "xhat", "istd", "branch", "dbranch",
             "dw", "dbeta", "dbias", "mask", "seed"]
ACC_DIN, ACC_PARAMS, ACC_BRANCH = 1, 2, 4
MAX_NODES = 8

_vp = ctypes.c_void_p
_i = ctypes.c_int
_configured = False


class Node(ctypes.Structure):
    _fields_ = [("op", _i), ("fval", ctypes.c_float), ("rng_type", _i), ("node_id", _i)]


class Desc(ctypes.Structure):
    _fields_ = [("group_id", _i), ("channels", _i), ("twin", _i), ("n_main", _i), ("n_left", _i),
                ("n_right", _i), ("main_ops", Node * MAX_NODES), ("left_ops", Node * MAX_NODES),
                ("right_ops", Node * MAX_NODES), ("dtype", _i)]


def header_functions() -> list:
    with open(HEADER) as f:
        return re.findall(r"TKM_ATTN_API\s+[\w\s\*]+?\b(tkm_\w+)\s*\(", f.read())


def lib() -> ctypes.CDLL:
    global _configured
    L = prep.lib()
    if _configured:
        return L
    L.tkm_plasma_default_fval.argtypes = [_i]
    L.tkm_plasma_default_fval.restype = ctypes.c_float
    L.tkm_plasma_source.argtypes = [ctypes.POINTER(Desc)]
    L.tkm_plasma_source.restype = _vp
    L.tkm_plasma_create.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(_vp)]
    L.tkm_plasma_create.restype = _i
    L.tkm_plasma_destroy.argtypes = [_vp]
    L.tkm_plasma_destroy.restype = None
    L.tkm_plasma_num_args.argtypes = [_vp, _i]
    L.tkm_plasma_num_args.restype = _i
    L.tkm_plasma_arg.argtypes = [_vp, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i)]
    L.tkm_plasma_arg.restype = _i
    L.tkm_plasma_fwd.argtypes = [_vp, ctypes.POINTER(_vp), _i, _vp]
    L.tkm_plasma_fwd.restype = _i
    L.tkm_plasma_bwd_workspace_bytes.argtypes = [_vp, _i]
    L.tkm_plasma_bwd_workspace_bytes.restype = ctypes.c_size_t
    L.tkm_plasma_bwd.argtypes = [_vp, ctypes.POINTER(_vp), _i, _i, _vp, ctypes.c_size_t, _vp]
    L.tkm_plasma_bwd.restype = _i
    _configured = True
    return L


def _check(fn, rc):
    if rc != 0:
        raise AttnError(fn, rc, lib().tkm_attn_last_error().decode())


def _nodes(chain):
    """(op, fval, rng_type, node_id) per item; an item is a name, (name, fval) or, for Drop,
    (name, fval, rng_type, node_id)."""
    out = []
    for item in chain:
        item = (item,) if isinstance(item, str) else tuple(item)
        name, fval = item[0], (item[1] if len(item) > 1 else None)
        rng, node = (item[2], item[3]) if len(item) > 3 else (0, 0)
        op = OPS[name]
        out.append((op, lib().tkm_plasma_default_fval(op) if fval is None else float(fval), int(rng), int(node)))
    return out


def make_desc(channels, chain=(), twin=False, left=(), right=(), dtype="f16", group_id=0) -> Desc:
    d = Desc()
    d.group_id, d.channels, d.twin = group_id, channels, int(twin)
    d.dtype = {"f16": F16, "bf16": BF16}[dtype]
    for field, count, ops in (("main_ops", "n_main", chain), ("left_ops", "n_left", left),
                              ("right_ops", "n_right", right)):
        nodes = _nodes(ops)
        if len(nodes) > MAX_NODES:
            raise ValueError(f"at most {MAX_NODES} ops per chain")
        setattr(d, count, len(nodes))
        arr = getattr(d, field)
        for k, (op, fv, rng, node) in enumerate(nodes):
            arr[k].op, arr[k].fval, arr[k].rng_type, arr[k].node_id = op, fv, rng, node
    return d


def source(d: Desc) -> str:
    L = lib()
    p = L.tkm_plasma_source(ctypes.byref(d))
    if not p:
        raise AttnError("tkm_plasma_source", -1, L.tkm_attn_last_error().decode())
    try:
        return ctypes.string_at(p).decode()
    finally:
        L.tkm_free(p)


class Plasma:
    """One compiled plasma group on the current device."""

    def __init__(self, channels, chain=(), twin=False, left=(), right=(), dtype="f16", group_id=0):
        self.desc = make_desc(channels, chain, twin, left, right, dtype, group_id)
        self.C, self.twin, self.dtype = channels, bool(twin), dtype
        self.nodes = _nodes(left) + _nodes(right) + _nodes(chain) if twin else _nodes(chain)
        h = _vp()
        _check("tkm_plasma_create", lib().tkm_plasma_create(ctypes.byref(self.desc), ctypes.byref(h)))
        self._h = h
        self.fwd_args = self._args(0)
        self.bwd_args = self._args(1)

    def _args(self, pas):
        L = lib()
        n = L.tkm_plasma_num_args(self._h, pas)
        out = []
        for i in range(n):
            k, nd = _i(), _i()
            _check("tkm_plasma_arg", L.tkm_plasma_arg(self._h, pas, i, ctypes.byref(k), ctypes.byref(nd)))
            out.append((ARG_KINDS[k.value], nd.value))
        return out

    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            lib().tkm_plasma_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def norm_groups(self):
        return (self.C + 63) // 64

    def _ptrs(self, spec, tensors):
        arr = (_vp * max(1, len(spec)))()
        for i, key in enumerate(spec):
            name, node = key
            t = tensors.get(name if node < 0 else (name, node))
            if t is None:
                raise KeyError(f"missing tensor {key}")
            arr[i] = t.data_ptr() if t.numel() else None
        return arr

    def fwd(self, tensors: dict, rows: int, stream=None):
        _check("tkm_plasma_fwd", lib().tkm_plasma_fwd(self._h, self._ptrs(self.fwd_args, tensors), rows,
                                                      attn._stream(stream)))

    def bwd_workspace_bytes(self, rows: int) -> int:
        return lib().tkm_plasma_bwd_workspace_bytes(self._h, rows)

    def bwd(self, tensors: dict, rows: int, acc_flags: int, workspace=None, stream=None):
        import torch
        need = self.bwd_workspace_bytes(rows)
        if workspace is None and need:
            dev = next(t.device for t in tensors.values() if t is not None)
            workspace = torch.empty(need, dtype=torch.uint8, device=dev)
        wptr = workspace.data_ptr() if workspace is not None else None
        wbytes = workspace.numel() if workspace is not None else 0
        _check("tkm_plasma_bwd", lib().tkm_plasma_bwd(self._h, self._ptrs(self.bwd_args, tensors), rows, acc_flags,
                                                      wptr, wbytes, attn._stream(stream)))

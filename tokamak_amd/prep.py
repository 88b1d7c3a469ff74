"""Python binding of the qkv-prep / run-time compilation / step-graph C ABI
(include/tkm_prep.h, libtkm_attn.so).

The qkv-prep epilogue is the generated kernel pair that turns the fused QKV GEMM output into
attention input: bias, optional per-head QKNorm, optional RoPE (reference generator
src/tkm_codegen.c:43-70, 211-295; runtime compile/launch src/tkm_gpu.cu:1047-1078, 1166-1174).
``Prep`` generates the HIP source for one descriptor, compiles it with hipRTC and launches it
on the caller's current torch stream.  Step graphs (``Graph``) capture what is enqueued on a
stream once and replay it (reference src/tkm_gpu.cu:1498-1508).  There is no fallback: a
missing library or a failed call raises.
"""
from __future__ import annotations

import ctypes
import os
import re

from . import attn
from .attn import AttnError, BF16, F16

HEADER = os.path.join(attn.ROOT, "include", "tkm_prep.h")

_vp = ctypes.c_void_p
_i = ctypes.c_int
_configured = False


class Desc(ctypes.Structure):
    """tkm_prep_desc (include/tkm_prep.h)."""
    _fields_ = [("group_id", _i), ("seq_len", _i), ("q_heads", _i), ("kv_heads", _i),
                ("head_dim", _i), ("has_qknorm", _i), ("has_rope", _i),
                ("rope_theta", ctypes.c_float), ("rope_scale", ctypes.c_float),
                ("rope_low_freq_factor", ctypes.c_float), ("rope_high_freq_factor", ctypes.c_float),
                ("rope_original_context_length", ctypes.c_float), ("dtype", _i)]


def header_functions() -> list:
    """Names of the functions include/tkm_prep.h declares."""
    with open(HEADER) as f:
        text = f.read()
    return re.findall(r"TKM_ATTN_API\s+[\w\s\*]+?\b(tkm_\w+)\s*\(", text)


def lib() -> ctypes.CDLL:
    global _configured
    L = attn.lib()
    if _configured:
        return L
    L.tkm_prep_desc_init.argtypes = [ctypes.POINTER(Desc)]
    L.tkm_prep_desc_init.restype = None
    L.tkm_prep_source.argtypes = [ctypes.POINTER(Desc)]
    L.tkm_prep_source.restype = _vp
    L.tkm_free.argtypes = [_vp]
    L.tkm_free.restype = None
    L.tkm_prep_create.argtypes = [ctypes.POINTER(Desc), ctypes.POINTER(_vp)]
    L.tkm_prep_create.restype = _i
    L.tkm_prep_destroy.argtypes = [_vp]
    L.tkm_prep_destroy.restype = None
    L.tkm_prep_fwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp]
    L.tkm_prep_fwd.restype = _i
    L.tkm_prep_bwd_workspace_bytes.argtypes = [_vp, _i]
    L.tkm_prep_bwd_workspace_bytes.restype = ctypes.c_size_t
    L.tkm_prep_bwd.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, ctypes.c_size_t, _vp]
    L.tkm_prep_bwd.restype = _i
    L.tkm_hip_prelude.restype = ctypes.c_char_p
    L.tkm_rtc_compile.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(_vp),
                                  ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(_vp)]
    L.tkm_rtc_compile.restype = _i
    L.tkm_graph_begin.argtypes = [_vp]
    L.tkm_graph_begin.restype = _i
    L.tkm_graph_end.argtypes = [_vp, ctypes.POINTER(_vp)]
    L.tkm_graph_end.restype = _i
    L.tkm_graph_launch.argtypes = [_vp, _vp]
    L.tkm_graph_launch.restype = _i
    L.tkm_graph_destroy.argtypes = [_vp]
    L.tkm_graph_destroy.restype = None
    _configured = True
    return L


def _check(fn: str, rc: int) -> None:
    if rc != 0:
        raise AttnError(fn, rc, lib().tkm_attn_last_error().decode())


def make_desc(q_heads, kv_heads, head_dim, seq_len, qknorm=False, rope=False, dtype="f16",
              group_id=0, theta=None, scale=None, low_freq_factor=None, high_freq_factor=None,
              original_context_length=None) -> Desc:
    """A descriptor with the reference's RoPE defaults (src/tkm_core.c:56-60) for unset fields."""
    d = Desc()
    lib().tkm_prep_desc_init(ctypes.byref(d))
    d.group_id, d.seq_len = group_id, seq_len
    d.q_heads, d.kv_heads, d.head_dim = q_heads, kv_heads, head_dim
    d.has_qknorm, d.has_rope = int(qknorm), int(rope)
    d.dtype = {"f16": F16, "bf16": BF16}[dtype]
    for name, v in (("rope_theta", theta), ("rope_scale", scale),
                    ("rope_low_freq_factor", low_freq_factor),
                    ("rope_high_freq_factor", high_freq_factor),
                    ("rope_original_context_length", original_context_length)):
        if v is not None:
            setattr(d, name, v)
    return d


def source(d: Desc) -> str:
    """The generated HIP source (prelude included) for descriptor d."""
    L = lib()
    p = L.tkm_prep_source(ctypes.byref(d))
    if not p:
        raise AttnError("tkm_prep_source", -1, L.tkm_attn_last_error().decode())
    try:
        return ctypes.string_at(p).decode()
    finally:
        L.tkm_free(p)


def prelude() -> str:
    return lib().tkm_hip_prelude().decode()


def rtc_compile(src: str, name: str = "tkm_generated.hip"):
    """hipRTC-compile src for gfx950; returns (status, code object bytes, log)."""
    L = lib()
    code, n, log = _vp(), ctypes.c_size_t(), _vp()
    rc = L.tkm_rtc_compile(src.encode(), name.encode(), ctypes.byref(code), ctypes.byref(n), ctypes.byref(log))
    try:
        blob = ctypes.string_at(code.value, n.value) if code.value else b""
        text = ctypes.string_at(log.value).decode() if log.value else ""
    finally:
        L.tkm_free(code)
        L.tkm_free(log)
    if rc != 0:
        text = text or L.tkm_attn_last_error().decode()
    return rc, blob, text


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


class Prep:
    """One compiled qkv-prep group on the current device."""

    def __init__(self, q_heads, kv_heads, head_dim, seq_len, qknorm=False, rope=False,
                 dtype="f16", group_id=0, **rope_args):
        self.desc = make_desc(q_heads, kv_heads, head_dim, seq_len, qknorm, rope, dtype, group_id,
                              **rope_args)
        self.dtype = dtype
        self.C = (q_heads + 2 * kv_heads) * head_dim
        self.QK = (q_heads + kv_heads) * head_dim
        self.NH = q_heads + kv_heads
        h = _vp()
        _check("tkm_prep_create", lib().tkm_prep_create(ctypes.byref(self.desc), ctypes.byref(h)))
        self._h = h

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            lib().tkm_prep_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _tdtype(self):
        import torch
        return torch.float16 if self.dtype == "f16" else torch.bfloat16

    def fwd(self, x, bias, gamma=None, rows=None, out=None, xhat=None, istd=None, stream=None):
        """out [rows, C] (and, with QKNorm, xhat [rows, QK] and istd [rows, Hq+Hkv])."""
        import torch
        rows = x.numel() // self.C if rows is None else rows
        dev = x.device
        if out is None:
            out = torch.empty((rows, self.C), dtype=self._tdtype(), device=dev)
        if self.desc.has_qknorm:
            if xhat is None:
                xhat = torch.empty((rows, self.QK), dtype=self._tdtype(), device=dev)
            if istd is None:
                istd = torch.empty((rows, self.NH), dtype=torch.float32, device=dev)
        for name, t, n in (("x", x, rows * self.C), ("out", out, rows * self.C), ("bias", bias, self.C)):
            attn._check_tensor(name, t, n, dev)
        if self.desc.has_qknorm:
            attn._check_tensor("gamma", gamma, self.QK, dev, torch.float32)
            attn._check_tensor("xhat", xhat, rows * self.QK, dev, self._tdtype())
            attn._check_tensor("istd", istd, rows * self.NH, dev, torch.float32)
        _check("tkm_prep_fwd", lib().tkm_prep_fwd(
            self._h, _ptr(x), _ptr(out), _ptr(bias), _ptr(gamma), _ptr(istd), _ptr(xhat), rows,
            attn._stream(stream)))
        return out, xhat, istd

    def bwd_workspace_bytes(self, rows: int) -> int:
        return lib().tkm_prep_bwd_workspace_bytes(self._h, rows)

    def bwd(self, dout, xhat=None, istd=None, gamma=None, rows=None, din=None, dgamma=None,
            dbias=None, accumulate=False, workspace=None, stream=None):
        """din [rows, C] (16-bit), dgamma [QK] and dbias [C] (fp32); accumulate adds to them."""
        import torch
        rows = dout.numel() // self.C if rows is None else rows
        dev = dout.device
        if din is None:
            din = torch.empty((rows, self.C), dtype=self._tdtype(), device=dev)
        if dbias is None:
            dbias = torch.empty(self.C, dtype=torch.float32, device=dev)
        if self.desc.has_qknorm and dgamma is None:
            dgamma = torch.empty(self.QK, dtype=torch.float32, device=dev)
        ws_bytes = self.bwd_workspace_bytes(rows)
        if workspace is None:
            workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        attn._check_tensor("dout", dout, rows * self.C, dev)
        attn._check_tensor("din", din, rows * self.C, dev)
        attn._check_tensor("dbias", dbias, self.C, dev, torch.float32)
        if self.desc.has_qknorm:
            attn._check_tensor("xhat", xhat, rows * self.QK, dev, self._tdtype())
            attn._check_tensor("istd", istd, rows * self.NH, dev, torch.float32)
            attn._check_tensor("gamma", gamma, self.QK, dev, torch.float32)
            attn._check_tensor("dgamma", dgamma, self.QK, dev, torch.float32)
        _check("tkm_prep_bwd", lib().tkm_prep_bwd(
            self._h, _ptr(dout), _ptr(din), _ptr(xhat), _ptr(istd), _ptr(gamma), _ptr(dgamma),
            _ptr(dbias), rows, int(accumulate), _ptr(workspace), workspace.numel(),
            attn._stream(stream)))
        return din, dgamma, dbias


class Graph:
    """A captured step: ``with Graph.capture(stream) as g: ...`` then ``g.launch(stream)``."""

    def __init__(self, handle):
        self._h = handle

    @staticmethod
    def begin(stream) -> None:
        _check("tkm_graph_begin", lib().tkm_graph_begin(ctypes.c_void_p(stream.cuda_stream)))

    @staticmethod
    def end(stream) -> "Graph":
        h = _vp()
        _check("tkm_graph_end", lib().tkm_graph_end(ctypes.c_void_p(stream.cuda_stream), ctypes.byref(h)))
        return Graph(h)

    def launch(self, stream) -> None:
        _check("tkm_graph_launch", lib().tkm_graph_launch(self._h, ctypes.c_void_p(stream.cuda_stream)))

    def close(self) -> None:
        if self._h and self._h.value:
            lib().tkm_graph_destroy(self._h)
            self._h = _vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

"""Python binding of the GQA attention C ABI (include/tkm_attn.h, libtkm_attn.so).

Mirrors the reference's GQA op (``GQA(q=, kv=, d=, causal=)``, reference
src/tkm_core.c:83-95) as it is executed by the runtime: forward at
src/tkm_gpu.cu:1252-1265, backward at src/tkm_gpu.cu:1389-1404.  Tensors are
torch device tensors (torch is used only for device memory and streams); every
call goes through ctypes into the HIP library and launches on the caller's
current torch stream.  There is no fallback: if the library is missing or a
call fails, an exception is raised.
"""
from __future__ import annotations

import ctypes
import math
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "libtkm_attn.so")
HEADER = os.path.join(ROOT, "include", "tkm_attn.h")

F16, BF16 = 0, 1
BWD_DELTA, BWD_DKDV, BWD_DQ, BWD_DQ_DELTA = 0, 1, 2, 3

_vp = ctypes.c_void_p
_i = ctypes.c_int
_lib = None


class AttnError(RuntimeError):
    """A tkm_attn_* call returned a non-zero status."""

    def __init__(self, fn: str, status: int, message: str):
        super().__init__(f"{fn} failed with status {status}: {message}")
        self.status = status


def header_functions() -> list:
    """Names of the functions include/tkm_attn.h declares."""
    with open(HEADER) as f:
        text = f.read()
    return re.findall(r"TKM_ATTN_API\s+[\w\s\*]+?\b(tkm_attn_\w+)\s*\(", text)


def lib() -> ctypes.CDLL:
    """Load libtkm_attn.so (built by tokamak_amd.build); raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m tokamak_amd.build` "
            "(the attention path has no non-HIP implementation)")
    L = ctypes.CDLL(LIB_PATH)
    L.tkm_attn_fwd.argtypes = [_vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_float, _i, _i, _vp]
    L.tkm_attn_fwd.restype = _i
    L.tkm_attn_bwd_workspace_bytes.argtypes = [_i, _i, _i]
    L.tkm_attn_bwd_workspace_bytes.restype = ctypes.c_size_t
    bwd_args = [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, ctypes.c_float, _i, _i,
                _vp, ctypes.c_size_t, _vp]
    L.tkm_attn_bwd.argtypes = bwd_args
    L.tkm_attn_bwd.restype = _i
    L.tkm_attn_bwd_stage.argtypes = [_i] + bwd_args
    L.tkm_attn_bwd_stage.restype = _i
    L.tkm_attn_status_string.argtypes = [_i]
    L.tkm_attn_status_string.restype = ctypes.c_char_p
    L.tkm_attn_last_error.restype = ctypes.c_char_p
    L.tkm_attn_version.restype = _i
    L.tkm_attn_init.restype = _i
    L.tkm_attn_asm_available.restype = _i
    L.tkm_attn_last_kernels.restype = ctypes.c_uint
    _lib = L
    return L


# Bits of tkm_attn_last_kernels (include/tkm_attn.h)
KERNEL_BITS = {"fwd_asm": 1, "fwd_hip": 2, "dq_asm": 4, "dq_hip": 8, "dkdv_asm": 16,
               "dkdv_hip": 32, "delta_hip": 64}


def init() -> None:
    """Load the gfx950 assembly kernels on the current device (tkm_attn_init); raises if a
    code object fails to load."""
    _check("tkm_attn_init", lib().tkm_attn_init())


def asm_available() -> bool:
    return bool(lib().tkm_attn_asm_available())


def last_kernels() -> list:
    """Names of the kernels the calling thread's last tkm_attn_* call launched."""
    bits = int(lib().tkm_attn_last_kernels())
    return [n for n, b in KERNEL_BITS.items() if bits & b]


def _check(fn: str, rc: int) -> None:
    if rc != 0:
        raise AttnError(fn, rc, lib().tkm_attn_last_error().decode())


def default_scale(D: int) -> float:
    """1/sqrtf(D) in fp32, as the reference dispatch passes (tkm_gpu.cu:1258)."""
    import numpy as np
    return float(np.float32(1.0) / np.sqrt(np.float32(D)))


def _dtype_code(t) -> int:
    import torch
    if t.dtype == torch.float16:
        return F16
    if t.dtype == torch.bfloat16:
        return BF16
    raise TypeError(f"attention tensors must be float16 or bfloat16, got {t.dtype}")


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    import torch
    s = torch.cuda.current_stream() if stream is None else stream
    return ctypes.c_void_p(s.cuda_stream)


def _check_tensor(name, t, numel, device, dtype=None):
    if not t.is_cuda or t.device != device:
        raise ValueError(f"{name} must be on {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() != numel:
        raise ValueError(f"{name} has {t.numel()} elements, expected {numel}")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")


def gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=True, kv_len=None, scale=None,
            out=None, lse=None, stream=None):
    """O [B,S,Hq*D] and LSE [B,Hq,S] (fp32) of packed qkv [B,S,(Hq+2Hkv)*D]."""
    import torch
    dev = qkv.device
    _check_tensor("qkv", qkv, B * S * (Hq + 2 * Hkv) * D, dev)
    dt = _dtype_code(qkv)
    out = torch.empty((B, S, Hq * D), dtype=qkv.dtype, device=dev) if out is None else out
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=dev) if lse is None else lse
    _check_tensor("out", out, B * S * Hq * D, dev, qkv.dtype)
    _check_tensor("lse", lse, B * Hq * S, dev, torch.float32)
    if kv_len is not None:
        _check_tensor("kv_len", kv_len, B, dev, torch.int32)
    scale = default_scale(D) if scale is None else float(scale)
    rc = lib().tkm_attn_fwd(_ptr(qkv), _ptr(out), _ptr(lse), _ptr(kv_len), B, S, Hq, Hkv, D,
                            scale, int(bool(causal)), dt, _stream(stream))
    _check("tkm_attn_fwd", rc)
    return out, lse


def bwd_workspace_bytes(B, S, Hq) -> int:
    return int(lib().tkm_attn_bwd_workspace_bytes(B, S, Hq))


def gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, causal=True, kv_len=None, scale=None,
            dqkv=None, workspace=None, stream=None, stage=None):
    """dqkv [B,S,(Hq+2Hkv)*D] (dQ | dK | dV); stage selects one backward kernel."""
    import torch
    dev = qkv.device
    _check_tensor("qkv", qkv, B * S * (Hq + 2 * Hkv) * D, dev)
    _check_tensor("o", o, B * S * Hq * D, dev, qkv.dtype)
    _check_tensor("dout", dout, B * S * Hq * D, dev, qkv.dtype)
    _check_tensor("lse", lse, B * Hq * S, dev, torch.float32)
    if kv_len is not None:
        _check_tensor("kv_len", kv_len, B, dev, torch.int32)
    dt = _dtype_code(qkv)
    dqkv = torch.empty_like(qkv) if dqkv is None else dqkv
    _check_tensor("dqkv", dqkv, qkv.numel(), dev, qkv.dtype)
    need = bwd_workspace_bytes(B, S, Hq)
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    wbytes = workspace.numel() * workspace.element_size()
    scale = default_scale(D) if scale is None else float(scale)
    args = (_ptr(qkv), _ptr(o), _ptr(dout), _ptr(lse), _ptr(dqkv), _ptr(kv_len), B, S, Hq, Hkv,
            D, scale, int(bool(causal)), dt, _ptr(workspace), wbytes, _stream(stream))
    if stage is None:
        _check("tkm_attn_bwd", lib().tkm_attn_bwd(*args))
    else:
        _check("tkm_attn_bwd_stage", lib().tkm_attn_bwd_stage(int(stage), *args))
    return dqkv


def attention_flops(B, S, Hq, D, causal, kv_len=None, mode="fwd") -> float:
    """Algorithmic FLOPs (FlashAttention convention): 4*B*Hq*S*Skv*D, halved if causal,
    x2.5 for the backward, x3.5 for forward+backward; with kv_len, S*Skv -> S*mean(kv_len)."""
    skv = S if kv_len is None else sum(int(x) for x in kv_len) / len(kv_len)
    f = 4.0 * B * Hq * S * skv * D * (0.5 if causal else 1.0)
    return {"fwd": f, "bwd": 2.5 * f, "fwdbwd": 3.5 * f}[mode]


__all__ = ["gqa_fwd", "gqa_bwd", "init", "asm_available", "last_kernels", "KERNEL_BITS", "bwd_workspace_bytes", "attention_flops", "default_scale",
           "lib", "header_functions", "AttnError", "F16", "BF16", "BWD_DELTA", "BWD_DKDV",
           "BWD_DQ", "BWD_DQ_DELTA"]

"""The C ABI library (libtkm_attn.so) without a GPU: it loads, exports every function
include/tkm_attn.h declares, and rejects invalid arguments before launching anything."""
import ctypes
import os
import subprocess

import pytest

from tokamak_amd import attn

OK, EINVAL, EUNSUPPORTED, EALIGN, EWORKSPACE = 0, -1, -2, -3, -4
P16 = ctypes.c_void_p(0x10000)   # 16-byte aligned fake device addresses: never dereferenced,
P16B = ctypes.c_void_p(0x20000)  # validation fails (or is not reached) before any HIP call
PODD = ctypes.c_void_p(0x10008)


def test_library_exports_header_functions():
    names = attn.header_functions()
    assert set(names) >= {"tkm_attn_fwd", "tkm_attn_bwd", "tkm_attn_bwd_stage",
                          "tkm_attn_bwd_workspace_bytes", "tkm_attn_status_string",
                          "tkm_attn_last_error", "tkm_attn_version", "tkm_attn_init",
                          "tkm_attn_asm_available", "tkm_attn_last_kernels"}
    L = attn.lib()
    for n in names:
        assert hasattr(L, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", attn.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    assert set(names) <= exported
    # nothing else with C linkage leaks out of the library: the exports are exactly the
    # functions the three public headers declare
    from tokamak_amd import plasma, prep
    both = set(names) | set(prep.header_functions()) | set(plasma.header_functions())
    for n in both:
        assert hasattr(L, n), n
    assert {e for e in exported if e.startswith("tkm_")} == both


def test_version_and_status_strings():
    L = attn.lib()
    assert L.tkm_attn_version() == 200
    assert L.tkm_attn_status_string(OK) == b"ok"
    for st in (EINVAL, EUNSUPPORTED, EALIGN, EWORKSPACE, -5, -6, -7):
        assert L.tkm_attn_status_string(st) not in (b"ok", b"unknown status")
    assert L.tkm_attn_status_string(-99) == b"unknown status"


def fwd(qkv=P16, o=P16B, lse=None, kv=None, B=1, S=8, Hq=2, Hkv=1, D=64, scale=0.125, causal=1, dtype=0):
    return attn.lib().tkm_attn_fwd(qkv, o, lse, kv, B, S, Hq, Hkv, D, scale, causal, dtype, None)


@pytest.mark.parametrize("kw,status,msg", [
    (dict(qkv=None), EINVAL, b"non-null"),
    (dict(o=None), EINVAL, b"non-null"),
    (dict(B=0), EINVAL, b"positive"),
    (dict(S=-3), EINVAL, b"positive"),
    (dict(Hq=3, Hkv=2), EINVAL, b"multiple"),
    (dict(D=96), EUNSUPPORTED, b"head dim"),
    (dict(D=256), EUNSUPPORTED, b"head dim"),
    (dict(dtype=2), EUNSUPPORTED, b"dtype"),
    (dict(causal=2), EINVAL, b"causal"),
    (dict(qkv=PODD), EALIGN, b"aligned"),
    (dict(lse=ctypes.c_void_p(0x10002)), EALIGN, b"aligned"),
    (dict(scale=0.0), EINVAL, b"scale"),
    (dict(scale=-1.0), EINVAL, b"scale"),
    (dict(scale=float("nan")), EINVAL, b"scale"),
    (dict(scale=float("inf")), EINVAL, b"scale"),
    (dict(Hq=40000, Hkv=40000, D=128), EUNSUPPORTED, b"too wide"),
])
def test_fwd_rejects(kw, status, msg):
    assert fwd(**kw) == status
    assert msg in attn.lib().tkm_attn_last_error()
    assert attn.lib().tkm_attn_last_kernels() == 0  # nothing launched


def bwd(stage=None, ws=P16, wsb=None, B=1, S=8, Hq=2, Hkv=1, D=64, lse=P16, dout=P16, scale=0.125):
    L = attn.lib()
    if wsb is None:
        wsb = L.tkm_attn_bwd_workspace_bytes(B, S, Hq)
    args = (P16, P16B, dout, lse, P16B, None, B, S, Hq, Hkv, D, scale, 1, 0, ws, wsb, None)
    return L.tkm_attn_bwd(*args) if stage is None else L.tkm_attn_bwd_stage(stage, *args)


def test_bwd_rejects():
    L = attn.lib()
    assert bwd(lse=None) == EINVAL
    assert bwd(dout=None) == EINVAL
    assert bwd(ws=None) == EWORKSPACE
    assert bwd(wsb=16) == EWORKSPACE and b"workspace" in L.tkm_attn_last_error()
    assert bwd(ws=ctypes.c_void_p(0x10004)) == EALIGN
    assert bwd(D=80) == EUNSUPPORTED
    assert bwd(scale=0.0) == EINVAL
    assert bwd(stage=4) == EINVAL and b"stage" in L.tkm_attn_last_error()
    assert bwd(stage=-1) == EINVAL


def test_workspace_bytes():
    L = attn.lib()
    # D per row (B*Hq*S floats, rounded up to 256 bytes), then 8 bytes per row of the
    # row values (-LSE*log2e, -D) with S padded to a multiple of 32
    assert L.tkm_attn_bwd_workspace_bytes(4, 2048, 16) == 4 * 2048 * 16 * 4 + 4 * 16 * 2048 * 8
    assert L.tkm_attn_bwd_workspace_bytes(1, 3, 1) == 256 + 32 * 8
    assert L.tkm_attn_bwd_workspace_bytes(2, 100, 3) == 2560 + 2 * 3 * 128 * 8
    assert L.tkm_attn_bwd_workspace_bytes(0, 3, 1) == 0


def test_flop_accounting():
    # F_fwd = 4*4*16*2048^2*128/2 = 68.72 GFLOP, fwd+bwd = 3.5x
    assert attn.attention_flops(4, 2048, 16, 128, True) == pytest.approx(68.719476736e9)
    assert attn.attention_flops(4, 2048, 16, 128, True, mode="fwdbwd") == pytest.approx(240.518168576e9)
    # config 5 useful FLOPs with kv_len {8192, 5000}
    assert attn.attention_flops(2, 8192, 32, 128, False, [8192, 5000], "fwd") == pytest.approx(1770.6e9, rel=1e-4)


def test_python_binding_requires_library(tmp_path, monkeypatch):
    monkeypatch.setattr(attn, "_lib", None)
    monkeypatch.setattr(attn, "LIB_PATH", str(tmp_path / "missing.so"))
    with pytest.raises(RuntimeError, match="missing"):
        attn.lib()


def test_header_compiles_as_c():
    src = os.path.join(os.path.dirname(attn.HEADER))
    r = subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-fsyntax-only", "-I", src, "-x", "c", "-"],
                       input='#include "tkm_attn.h"\nint main(void){return TKM_ATTN_OK;}\n',
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


def test_noalloc_rejects_beyond_scratch_without_device():
    """tkm_attn_bwd_noalloc checks its size against the static scratch before it touches the
    device: a workspace need above 16 MiB fails with TKM_ATTN_EWORKSPACE."""
    L = attn.lib()
    L.tkm_attn_bwd_noalloc.restype = ctypes.c_int
    B, S, Hq = 8, 65536, 4
    assert L.tkm_attn_bwd_workspace_bytes(B, S, Hq) > 16 << 20
    rc = L.tkm_attn_bwd_noalloc(P16, P16, P16, P16, P16B, None, B, S, Hq, Hq, 128,
                                ctypes.c_float(0.088), 1, 0, None)
    assert rc == EWORKSPACE and b"scratch" in L.tkm_attn_last_error()
    rc = L.tkm_attn_bwd_noalloc(None, P16, P16, P16, P16B, None, 1, 8, 2, 1, 64,
                                ctypes.c_float(0.125), 1, 0, None)
    assert rc == EINVAL  # argument checks also come before any device call

"""Build libtkm_attn.so: the HIP attention kernels for gfx950, the C ABI of include/tkm_attn.h
and include/tkm_prep.h, and the C host code that generates, compiles (hipRTC) and launches the
qkv-prep kernels.

Usage: python -m tokamak_amd.build   (or build() from Python).  Always recompiles.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
INCLUDE = os.path.join(ROOT, "include")
LIB_NAME = "libtkm_attn.so"
LIB_PATH = os.path.join(PKG, LIB_NAME)
SOURCES = ["attn_fwd.hip", "attn_bwd.hip", "tkm_attn_abi.hip"]
C_SOURCES = ["tkm_error.c", "tkm_prelude.c", "tkm_prep_codegen.c", "tkm_rtc.c", "tkm_plasma_codegen.c",
             "tkm_plasma_rt.c"]
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 in generated code.
HIPFLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", f"-I{INCLUDE}", f"-I{CSRC}",
]


# Host C: -ffp-contract=off keeps the RoPE frequency expression in plain fp32 steps.
CFLAGS = [
    "-O2", "-std=gnu11", "-fPIC", "-fvisibility=hidden", "-ffp-contract=off", "-Wall", "-Wextra",
    "-D__HIP_PLATFORM_AMD__", f"-I{ROCM}/include", f"-I{INCLUDE}", f"-I{CSRC}",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm required to build libtkm_attn.so)")


def _compile(src: str, obj: str, extra) -> None:
    if src.endswith(".c"):
        cmd = [os.environ.get("CC", "gcc"), *CFLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    else:
        cmd = [hipcc(), *HIPFLAGS, *extra, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed for {src}:\n{r.stdout}\n{r.stderr}")
    if r.stderr.strip() and src.endswith(".c"):
        raise RuntimeError(f"warnings in {src} (host C builds warning-free):\n{r.stderr}")


def build(verbose: bool = False, extra=()) -> str:
    objdir = os.path.join(PKG, "_obj")
    os.makedirs(objdir, exist_ok=True)
    srcs = SOURCES + C_SOURCES
    objs = [os.path.join(objdir, s.replace(".", "_") + ".o") for s in srcs]
    with ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        list(ex.map(lambda so: _compile(so[0], so[1], extra), zip(srcs, objs)))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
           f"-L{ROCM}/lib", "-lhiprtc", f"-Wl,-rpath,{ROCM}/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True, extra=sys.argv[1:])

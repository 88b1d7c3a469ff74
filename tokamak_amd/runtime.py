"""Python binding of the HIP runtime behind tkm.h (libtkm_hip.so: tkm_hip.c and the whole-graph
generator tkm_codegen_hip.c) -- the public C API of the reference's tkm.h, section 5
(reference include/tkm.h:214-271), plus this build's extensions (include/tkm_hip.h).

A graph is a ctypes buffer holding a TkmGraph exactly as the reference's front end writes it
(tkm_parse_dsl / tkm_optimize_and_bind / tkm_plan_memory in src/tkm_core.c); ``graph_buffer``
wraps such bytes.  Every call goes through ctypes into the library; there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

from . import attn

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libtkm_hip.so")
HEADERS = [os.path.join(attn.ROOT, "include", "tkm.h"), os.path.join(attn.ROOT, "include", "tkm_hip.h")]

SIZEOF_GRAPH = 1370144          # sizeof(TkmGraph), pinned against the reference header by the CPU tests
GROUP_PREP, GROUP_PLASMA = 0, 1

_vp, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
_lib = None


class Opts(ctypes.Structure):
    _fields_ = [("dtype", _i), ("training", _i), ("token_labels", _i), ("init_seed", ctypes.c_uint64),
                ("verbose", _i), ("dataset_mode", _i), ("clear_all_grads", _i)]


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m tokamak_amd.build`")
    L = ctypes.CDLL(LIB_PATH)
    sig = {
        "tkm_codegen_cuda_string": ([_vp], _vp),
        "tkm_codegen_hip_source": ([_vp, _i], _vp),
        "tkm_hip_group_kind": ([_vp, _i], _i),
        "tkm_hip_prep_desc": ([_vp, _i, _i, _vp], _i),
        "tkm_hip_plasma_desc": ([_vp, _i, _i, _vp, _vp], _i),
        "tkm_hip_plasma_op": ([_vp], _i),
        "tkm_hip_res_flags": ([_vp], ctypes.c_uint32),
        "tkm_runtime_opts_init": ([_vp], None),
        "tkm_runtime_ignite": ([_vp, ctypes.c_char_p], _vp),
        "tkm_runtime_ignite_inference": ([_vp, ctypes.c_char_p], _vp),
        "tkm_runtime_ignite_ex": ([_vp, ctypes.c_char_p, _vp], _vp),
        "tkm_load_string": ([ctypes.c_char_p, _i], _vp),
        "tkm_runtime_step": ([_vp, _vp, _vp, _f], _f),
        "tkm_runtime_step_tokens": ([_vp, _vp, _vp, _f], _f),
        "tkm_runtime_step_device": ([_vp, _f], _i),
        "tkm_runtime_upload": ([_vp, _vp, _vp, _sz], _i),
        "tkm_runtime_last_loss": ([_vp], _f),
        "tkm_runtime_eval": ([_vp, _vp, _vp, _i], _i),
        "tkm_runtime_forward": ([_vp, _vp, _vp, _sz], _sz),
        "tkm_runtime_input_elements": ([_vp], _sz),
        "tkm_runtime_output_elements": ([_vp], _sz),
        "tkm_runtime_weight_bytes": ([_vp], _sz),
        "tkm_save_weights_buffer": ([_vp, _vp, _sz, ctypes.POINTER(_sz)], _i),
        "tkm_load_weights_buffer": ([_vp, _vp, _sz], _i),
        "tkm_save_weights": ([_vp, ctypes.c_char_p], _i),
        "tkm_load_weights": ([_vp, ctypes.c_char_p], _i),
        "tkm_runtime_free": ([_vp], None),
        "tkm_get_grad_sample": ([_vp, _i, _i], _f),
        "tkm_perturb_tensor": ([_vp, _i, _i, _f], None),
        "tkm_eval_current_loss": ([_vp], _f),
        "tkm_dataset_create": ([_vp, _vp, _vp, _sz], _vp),
        "tkm_dataset_free": ([_vp], None),
        "tkm_dataset_is_resident": ([_vp], _i),
        "tkm_runtime_train_epoch": ([_vp, _vp, _vp, _f, _f, _sz, _sz, _sz, ctypes.POINTER(_f)], _i),
        "tkm_runtime_stream": ([_vp], _vp),
        "tkm_runtime_node_device": ([_vp, _i, _i], _vp),
        "tkm_runtime_num_tensors": ([_vp], _i),
        "tkm_runtime_tensor": ([_vp, _i, ctypes.POINTER(_vp), ctypes.POINTER(_vp), ctypes.POINTER(_vp),
                                ctypes.POINTER(_sz), ctypes.POINTER(_i)], _i),
        "tkm_runtime_node_save": ([_vp, _i, _i], _vp),
        "tkm_runtime_step_kernel_count": ([_vp], _i),
        "tkm_attn_last_error": ([], ctypes.c_char_p),
    }
    for name, (args, res) in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = res
    L.free.argtypes = [_vp]
    _lib = L
    return L


def header_functions() -> list:
    """TKM_API functions of include/tkm.h and include/tkm_hip.h that this library defines (the
    front end's -- parsing, fusion, planning, registry -- come from the reference)."""
    front = {"tkm_verify_registry", "tkm_parse_dsl", "tkm_infer_shapes", "tkm_optimize_and_bind",
             "tkm_plan_memory", "tkm_dump_summary"}
    names = []
    for h in HEADERS:
        with open(h) as f:
            names += re.findall(r"TKM_API\s+[\w\s\*]+?\b(tkm_\w+)\s*\(", f.read())
    return [n for n in names if n not in front]


def graph_buffer(raw: bytes):
    """A TkmGraph-sized ctypes buffer holding `raw` (the front end's struct bytes)."""
    if len(raw) != SIZEOF_GRAPH:
        raise ValueError(f"graph of {len(raw)} bytes, expected sizeof(TkmGraph) = {SIZEOF_GRAPH}")
    return ctypes.create_string_buffer(bytes(raw), SIZEOF_GRAPH)


def _take_string(p) -> str:
    if not p:
        raise RuntimeError(lib().tkm_attn_last_error().decode())
    try:
        return ctypes.string_at(p).decode()
    finally:
        lib().free(p)


def codegen(graph, dtype: int = attn.F16) -> str:
    return _take_string(lib().tkm_codegen_hip_source(graph, dtype))


def node_offset(index: int) -> int:
    """Byte offset of nodes[index] in a TkmGraph (sizeof(TkmNode) = 264)."""
    return 264 * index


class Runtime:
    """A runtime ignited from a graph buffer (tkm_runtime_ignite_ex)."""

    def __init__(self, graph, dtype=attn.F16, training=True, token_labels=False, init_seed=0x7417,
                 verbose=False, src=None, dataset_mode=0, clear_all_grads=False):
        L = lib()
        o = Opts()
        L.tkm_runtime_opts_init(ctypes.byref(o))
        o.dtype, o.training, o.token_labels, o.init_seed, o.verbose = (dtype, int(training), int(token_labels),
                                                                         init_seed, int(verbose))
        o.dataset_mode, o.clear_all_grads = dataset_mode, int(clear_all_grads)
        self.graph = graph
        self.rt = L.tkm_runtime_ignite_ex(graph, None if src is None else src.encode(), ctypes.byref(o))
        if not self.rt:
            raise RuntimeError("tkm_runtime_ignite_ex failed (see stderr)")
        self.dtype = dtype
        self.token_labels = token_labels

    def close(self):
        if self.rt:
            lib().tkm_runtime_free(self.rt)
            self.rt = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @property
    def input_elements(self) -> int:
        return int(lib().tkm_runtime_input_elements(self.rt))

    def step(self, x, labels, lr: float) -> float:
        x = np.ascontiguousarray(x, np.float32)
        if self.token_labels:
            lab = np.ascontiguousarray(labels, np.int32)
            return float(lib().tkm_runtime_step_tokens(self.rt, x.ctypes.data, lab.ctypes.data, lr))
        lab = np.ascontiguousarray(labels, np.uint8)
        return float(lib().tkm_runtime_step(self.rt, x.ctypes.data, lab.ctypes.data, lr))

    def upload(self, x, labels=None):
        x = np.ascontiguousarray(x, np.float32)
        lab = None if labels is None else np.ascontiguousarray(labels, np.int32 if self.token_labels else np.uint8)
        rc = lib().tkm_runtime_upload(self.rt, x.ctypes.data, None if lab is None else lab.ctypes.data,
                                      0 if lab is None else lab.size)
        if rc:
            raise RuntimeError("tkm_runtime_upload failed")

    def step_device(self, lr: float):
        if lib().tkm_runtime_step_device(self.rt, lr):
            raise RuntimeError("tkm_runtime_step_device failed")

    def last_loss(self) -> float:
        return float(lib().tkm_runtime_last_loss(self.rt))

    def eval_current_loss(self) -> float:
        return float(lib().tkm_eval_current_loss(self.rt))

    def grad_sample(self, node: int, idx: int) -> float:
        return float(lib().tkm_get_grad_sample(self.rt, node, idx))

    def perturb(self, node: int, idx: int, delta: float):
        lib().tkm_perturb_tensor(self.rt, node, idx, delta)

    def forward(self, x) -> np.ndarray:
        n = int(lib().tkm_runtime_output_elements(self.rt))
        out = np.zeros(n, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        got = lib().tkm_runtime_forward(self.rt, x.ctypes.data, out.ctypes.data, n)
        if got != n:
            raise RuntimeError("tkm_runtime_forward failed")
        return out

    def eval(self, x, labels, count: int) -> int:
        x = np.ascontiguousarray(x, np.float32)
        lab = np.ascontiguousarray(labels, np.uint8)
        return int(lib().tkm_runtime_eval(self.rt, x.ctypes.data, lab.ctypes.data, count))

    def save_weights(self) -> bytes:
        n = int(lib().tkm_runtime_weight_bytes(self.rt))
        buf = ctypes.create_string_buffer(n)
        out = _sz()
        if not lib().tkm_save_weights_buffer(self.rt, buf, n, ctypes.byref(out)):
            raise RuntimeError("tkm_save_weights_buffer failed")
        return buf.raw[:out.value]

    def load_weights(self, data: bytes) -> bool:
        buf = ctypes.create_string_buffer(bytes(data), len(data))
        return bool(lib().tkm_load_weights_buffer(self.rt, buf, len(data)))

    def tensors(self) -> list:
        """[(node_id, element count)] of the learnable tensors, in TKM1 order."""
        L = lib()
        out = []
        for i in range(L.tkm_runtime_num_tensors(self.rt)):
            n, node = _sz(), _i()
            L.tkm_runtime_tensor(self.rt, i, None, None, None, ctypes.byref(n), ctypes.byref(node))
            out.append((node.value, n.value))
        return out

    def stream(self):
        return lib().tkm_runtime_stream(self.rt)

    def node_device(self, node: int, grad: bool = False) -> int:
        p = lib().tkm_runtime_node_device(self.rt, node, int(grad))
        if not p:
            raise ValueError(f"no device buffer for node {node}")
        return p

    def kernel_count(self) -> int:
        return int(lib().tkm_runtime_step_kernel_count(self.rt))


def parse_weights(data: bytes) -> list:
    """The float arrays of a TKM1 weight file (magic 0x544B4D31, count, then size + values)."""
    magic, nt = np.frombuffer(data[:8], np.uint32)
    if magic != 0x544B4D31:
        raise ValueError("not a TKM1 weight buffer")
    out, off = [], 8
    for _ in range(int(nt)):
        n = int(np.frombuffer(data[off:off + 4], np.uint32)[0])
        out.append(np.frombuffer(data[off + 4:off + 4 + 4 * n], np.float32).copy())
        off += 4 + 4 * n
    if off != len(data):
        raise ValueError("trailing bytes in TKM1 buffer")
    return out


def encode_weights(arrays) -> bytes:
    parts = [np.array([0x544B4D31, len(arrays)], np.uint32).tobytes()]
    for a in arrays:
        a = np.ascontiguousarray(a, np.float32)
        parts.append(np.array([a.size], np.uint32).tobytes())
        parts.append(a.tobytes())
    return b"".join(parts)


__all__ = ["lib", "graph_buffer", "codegen", "Runtime", "parse_weights", "encode_weights", "header_functions",
           "GROUP_PREP", "GROUP_PLASMA", "SIZEOF_GRAPH"]

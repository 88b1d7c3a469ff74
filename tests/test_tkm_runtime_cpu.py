"""The tkm.h runtime library (libtkm_hip.so) and its whole-graph generator without a GPU, pinned
to fixtures that the reference's own front end wrote (tests/golden/make_tkm_fixtures.py builds
its unchanged src/tkm_core.c, src/tkm_registry.c, src/tkm_codegen.c in this container):

  - include/tkm.h has the reference header's struct layout, member by member;
  - the runtime's op table agrees with the reference registry (resource flags, user-formula
    indices, default constants, op names);
  - every group's generated kernels take the group's TkmKernelSig parameters in order, with
    the signature's C types and names, then this build's extras;
  - the qkv_prep node maps onto tkm_prep_desc field by field, plain and twin groups onto
    tkm_plasma_desc op by op;
  - the generated source of whole models compiles with hipRTC for gfx950;
  - the library exports the functions its headers declare.
"""
import ctypes
import json
import os
import re
import subprocess

import numpy as np
import pytest

from tokamak_amd import plasma, prep
from tokamak_amd import runtime as R

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
GRAPHS = np.load(os.path.join(HERE, "golden", "tkm_graphs.npz"))
NAMES = sorted({k.split("/")[0] for k in GRAPHS.files})
REGISTRY = json.load(open(os.path.join(HERE, "golden", "tkm_registry.json")))


# seeded random small decoders (tests/golden/make_tkm_fixtures.py: random_decoder)
RANDOM_DECODERS = sorted({k.split("/")[0] for k in GRAPHS.files if k.startswith("rand_decoder_")})


def gjson(name):
    return json.loads(bytes(GRAPHS[name + "/json"]).decode())


def gbuf(name):
    return R.graph_buffer(GRAPHS[name + "/graph"].tobytes())


def test_header_layout_matches_reference():
    """sizeof / offsetof of every struct member of include/tkm.h against the reference
    header's (oracle/tkm_front_dump.c, built once against each header)."""
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "layout_own"], check=True)
    out = subprocess.run([os.path.join(ROOT, "oracle", "_ref", "tkm_layout_own"), "layout"], capture_output=True,
                         text=True, check=True).stdout
    own = json.loads(out)
    ref = json.load(open(os.path.join(HERE, "golden", "tkm_layout.json")))
    assert own == ref
    assert ref["sizeof.TkmGraph"] == R.SIZEOF_GRAPH


def _node(op, spec_id=0):
    """A TkmNode buffer with op and spec_id set (offsets from the layout fixture)."""
    lay = json.load(open(os.path.join(HERE, "golden", "tkm_layout.json")))
    buf = ctypes.create_string_buffer(lay["sizeof.TkmNode"])
    ctypes.c_int.from_buffer(buf, lay["TkmNode.op"][0]).value = op
    ctypes.c_int.from_buffer(buf, lay["TkmNode.spec_id"][0]).value = spec_id
    return buf


def test_resource_flags_match_registry():
    L = R.lib()
    for e in REGISTRY:
        got = L.tkm_hip_res_flags(_node(e["op"], e["index"]))
        assert got == e["res_flags"], e["name"]


def test_op_mapping_matches_registry():
    """Every registry op of the epilogue family maps onto the plasma op of the same name, with the
    registry's default constant; the user-formula ops by their registry index."""
    L = R.lib()
    mapped = set()
    for e in REGISTRY:
        code = L.tkm_hip_plasma_op(_node(e["op"], e["index"]))
        if e["name"] in plasma.OP_NAMES:
            assert code == plasma.OPS[e["name"]], e["name"]
            assert plasma.lib().tkm_plasma_default_fval(code) == pytest.approx(e["default_fval"], rel=1e-6), e["name"]
            mapped.add(e["name"])
        else:
            assert code == -1, e["name"]
    assert mapped == set(plasma.OP_NAMES) - set(plasma.FORMULA_OPS)
    assert REGISTRY[62]["name"] == "Softplus" and REGISTRY[63]["name"] == "Snake"


def _kernel_params(src, name):
    """(c_type, name) pairs of extern "C" kernel `name` in src."""
    m = re.search(r"void %s\((.*?)\)\s*\{" % re.escape(name), src, re.S)
    assert m, name
    out = []
    for p in m.group(1).split(","):
        p = " ".join(p.split())
        t, n = p.rsplit(" ", 1)
        out.append((t, n))
    return out


@pytest.mark.parametrize("name", ["cfg4", "llama_small", "exotic_llama", "fused_check", "numcheck_LayerScale",
                                  "llama3_style"] + RANDOM_DECODERS)
def test_kernels_take_the_signature_parameters(name):
    """tkm_plasma_{fwd,bwd}_g<N> of every group: the TkmKernelSig's arguments first, in order,
    with its C types and names (src/tkm_core.c:289-382), then only this build's extras."""
    js = gjson(name)
    src = R.codegen(gbuf(name))
    extras = {"rows", "part", "band", "acc_flags", "accumulate"}
    for grp in js["groups"]:
        for sig_key, fn in (("fwd_sig", "tkm_plasma_fwd_g%d"), ("bwd_sig", "tkm_plasma_bwd_g%d")):
            sig = grp[sig_key]
            got = _kernel_params(src, fn % grp["id"])
            want = [(" ".join(a["c_type"].split()), a["c_name"]) for a in sig["args"]]
            assert got[:len(want)] == want, (name, grp["id"], sig_key)
            for t, n in got[len(want):]:
                assert n in extras or n.startswith("x_"), (name, grp["id"], n)


def test_prep_descriptor_mapping():
    """The qkv_prep node's fields (written by the reference's 3-way rule,
    src/tkm_registry.c:750-768) become tkm_prep_desc fields; S = H*W of the group."""
    L = R.lib()
    for name in ["cfg4", "llama_small", "exotic_llama", "llama3_style"] + RANDOM_DECODERS:
        js = gjson(name)
        g = gbuf(name)
        seen = 0
        for grp in js["groups"]:
            if not grp["is_qkv_prep"]:
                continue
            n = js["nodes"][grp["nodes"][0]]
            assert L.tkm_hip_group_kind(g, grp["id"]) == R.GROUP_PREP
            d = prep.Desc()
            assert L.tkm_hip_prep_desc(g, grp["id"], 0, ctypes.byref(d)) == 0
            assert (d.group_id, d.seq_len, d.q_heads, d.kv_heads, d.head_dim) == \
                (grp["id"], grp["H"] * grp["W"], n["q_heads"], n["kv_heads"], n["head_dim"])
            assert (d.has_qknorm, d.has_rope) == (n["has_qknorm"], n["has_rope"])
            for f in ("rope_theta", "rope_scale", "rope_low_freq_factor", "rope_high_freq_factor",
                      "rope_original_context_length"):
                assert getattr(d, f) == pytest.approx(n[f], rel=1e-7), (name, f)
            assert n["q_c"] + n["k_c"] + n["v_c"] == grp["C"]
            seen += 1
        assert seen == sum(1 for n in js["nodes"] if n["op"] == 6 and not n["dead"]), name
    # llama3_style: RoPE with the Llama-3 rescaling; exotic: QKNorm with RoPE
    d = prep.Desc()
    js = gjson("llama3_style")
    gid = next(g["id"] for g in js["groups"] if g["is_qkv_prep"])
    R.lib().tkm_hip_prep_desc(gbuf("llama3_style"), gid, 0, ctypes.byref(d))
    assert (d.rope_theta, d.rope_scale, d.has_qknorm, d.q_heads, d.kv_heads, d.head_dim) == (500000.0, 8.0, 0, 32, 8, 128)
    js = gjson("exotic_llama")
    gid = next(g["id"] for g in js["groups"] if g["is_qkv_prep"])
    R.lib().tkm_hip_prep_desc(gbuf("exotic_llama"), gid, 0, ctypes.byref(d))
    assert (d.has_qknorm, d.has_rope, d.q_heads, d.kv_heads, d.head_dim) == (1, 1, 8, 2, 64)


def test_plasma_descriptor_mapping():
    """Plain groups: the group's nodes in order; twin groups: the Mul's left and right gate
    chains, then the ops after the product (src/tkm_core.c:509-537)."""
    L = R.lib()
    names = [e["name"] for e in REGISTRY]
    for name in ("exotic_llama", "llama_small", "fused_check"):
        js = gjson(name)
        g = gbuf(name)
        for grp in js["groups"]:
            if grp["is_qkv_prep"]:
                continue
            d = plasma.Desc()
            chain = (ctypes.c_int * 24)()
            assert L.tkm_hip_plasma_desc(g, grp["id"], 0, ctypes.byref(d), chain) == 0, (name, grp["id"])
            nodes = js["nodes"]
            if grp["is_twin_epilogue"]:
                mul = nodes[grp["nodes"][0]]
                want = mul["left"] + mul["right"] + grp["nodes"][1:]
                assert (d.twin, d.n_left, d.n_right, d.n_main) == (1, len(mul["left"]), len(mul["right"]),
                                                                   len(grp["nodes"]) - 1)
                ops = [d.left_ops[i] for i in range(d.n_left)] + [d.right_ops[i] for i in range(d.n_right)] + \
                    [d.main_ops[i] for i in range(d.n_main)]
            else:
                want = grp["nodes"]
                assert (d.twin, d.n_main) == (0, len(want))
                ops = [d.main_ops[i] for i in range(d.n_main)]
            assert list(chain[:len(want)]) == want
            for o, nid in zip(ops, want):
                n = nodes[nid]
                assert plasma.OP_NAMES[o.op] == names[n["spec_id"]], (name, nid)
                assert o.fval == pytest.approx(n["fval"], rel=1e-7)
                assert (o.rng_type, o.node_id) == (n["rng_type"], nid)
            assert d.channels == grp["C"]


@pytest.mark.parametrize("name,dtype", [("exotic_llama", 0), ("fused_check", 1), ("numcheck_Snake", 0),
                                        ("rand_decoder_1010", 0), ("rand_decoder_1037", 1)])
def test_generated_source_compiles(name, dtype):
    """prelude + tkm_codegen_hip_source compiles with hipRTC for gfx950 (no GPU needed)."""
    src = prep.prelude() + "\n" + R.codegen(gbuf(name), dtype)
    rc, code, log = prep.rtc_compile(src, name + ".hip")
    assert rc == 0, log
    assert len(code) > 0


def test_codegen_cuda_string_is_fp16_and_frees():
    src = R._take_string(R.lib().tkm_codegen_cuda_string(gbuf("numcheck_SiLU")))
    assert "tkm_plasma_fwd_g0" in src and "tkm_plasma_bwd_g0" in src and "fp16" in src


def test_library_exports_runtime_api():
    """libtkm_hip.so defines every function of tkm.h's runtime section and of tkm_hip.h (the
    front end's functions come from the reference's tkm_core.c)."""
    names = R.header_functions()
    assert len([n for n in names if n.startswith(("tkm_runtime_", "tkm_load_", "tkm_save_", "tkm_dataset_",
                                                  "tkm_get_grad", "tkm_perturb", "tkm_eval_current"))]) >= 25
    out = subprocess.run(["nm", "-D", "--defined-only", R.LIB_PATH], capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    undefined = subprocess.run(["nm", "-D", "--undefined-only", R.LIB_PATH], capture_output=True, text=True).stdout
    # the front end is bound weakly: the library loads without it
    for fn in ("tkm_parse_dsl", "tkm_optimize_and_bind", "tkm_plan_memory"):
        line = [ln for ln in undefined.splitlines() if ln.split()[-1] == fn]
        assert line and line[0].split()[0] == "w", (fn, line)


def test_load_without_front_end_fails_cleanly():
    """tkm_load_string needs the reference's front end; without it the call returns NULL."""
    assert not R.lib().tkm_load_string(b"input: 1x1x8\ntest: SiLU -> SoftmaxCE", 2)

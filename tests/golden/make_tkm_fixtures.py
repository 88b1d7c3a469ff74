"""Writes the graph-IR fixtures that pin this build's runtime (tkm_hip.c) and HIP generator
(tkm_codegen_hip.c) to the reference's front end.  Run in the build container only, where the
reference checkout exists:

    python tests/golden/make_tkm_fixtures.py

It builds oracle/_ref/tkm_front_dump (oracle/Makefile, target `ref`: oracle/tkm_front_dump.c
linked with the reference's unchanged src/tkm_core.c, src/tkm_registry.c, src/tkm_codegen.c)
and runs it on each model below, then packs the outputs into:

  tests/golden/tkm_graphs.npz     <name>/graph: the TkmGraph struct the reference's
                                  tkm_parse_dsl -> tkm_optimize_and_bind -> tkm_plan_memory
                                  produce (bytes); <name>/json: its nodes, groups and every
                                  TkmKernelSig (argument kinds, nodes, C types, names, grid)
  tests/golden/tkm_registry.json  the op registry: index, name, op, category, resource
                                  flags, default constant (no code snippets)
  tests/golden/tkm_layout.json    sizeof / offsetof of every struct of the reference's tkm.h

Models: BASELINE config 4's decoder (tests/golden/models/cfg4_llama.tkm, batch 8), a small
two-layer decoder for the chained-oracle parity test (llama_small.tkm, batch 2), a two-layer
head-dim-128 decoder trained on an induction task by the trained-attention test (induction.tkm,
batch 4), the
reference's models/exotic_llama.tkm (batch 2) and models/llama3_style.tkm (batch 1; its
structure only), and the inputs of the reference's GPU gradient check (src/main.c:202-306):
one "input: 1x1x32 / test: <op> -> SoftmaxCE" graph per checked op (batch 2) and its fused
twin-FC graph (batch 4); and nine seeded random small decoders (random_decoder).  The model texts of the reference are read in place, not copied.
"""
from __future__ import annotations

import json
import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
REF = os.environ.get("TKM_REFERENCE", "/root/reference")
DUMP = os.path.join(ROOT, "oracle", "_ref", "tkm_front_dump")

# Ops of the reference's GPU gradient check (src/main.c:59-75: is_numcheck_testable, plus the
# user-formula ops with both expressions); Snake is checked as Snake(1.7) (main.c:259-261).
NUMCHECK_OPS = ["SiLU", "ReLU", "ReLU2", "LeakyReLU", "ELU", "GELU", "Mish", "HardSwish", "HardSigmoid",
                "Tanh", "Sigmoid", "SwishBeta", "Sin", "CosGate", "SoftCap", "Clamp", "Scale", "LayerScale",
                "DyT", "PReLU", "xATLU", "Softplus", "Snake(1.7)"]

# The fused check's graph (src/main.c:78-85): a twin-FC with a user-formula op in one gate.
FUSED_CHECK = ("input: 1x1x8\nflow:\n  trunk: FC(8) -> Softplus -> FC(8) -> Tanh\n  gate: {\n"
               "    branch: FC(8) -> Softplus -> Scale(0.7)\n    skip: FC(8) -> GELU\n"
               "  } -> Mul -> Softplus -> FC(4) -> SoftmaxCE\n")


def random_decoder(seed):
    """A seeded small decoder in the .tkm DSL: width, heads and GQA ratio, head dim (QKNorm only
    with 64, as the reference requires), RoPE, causal or not, SwiGLU or GELU feed-forward,
    one or two layers, vocabulary and batch all drawn.  Returns (text, batch)."""
    import random
    r = random.Random(seed)
    D = r.choice((64, 128))
    hkv = r.choice((1, 2))
    hq = hkv * r.choice((1, 2, 4))
    C, S, V = r.choice((64, 128, 192)), r.choice((16, 32, 48, 64)), r.choice((64, 256))
    hidden = r.choice((96, 128, 192))
    qknorm = D == 64 and r.random() < 0.5
    rope = r.random() < 0.7
    causal = ", causal=true" if r.random() < 0.7 else ""
    post = (" -> QKNorm" if qknorm else "") + (" -> RoPE(theta=10000)" if rope else "")
    if r.random() < 0.6:
        ffn = ["  branch: RMSNorm -> {", f"    gate: FC({hidden}) -> SiLU", f"    up: FC({hidden})",
               f"  }} -> Mul -> FC({C})"]
    else:
        ffn = [f"  branch: RMSNorm -> FC({hidden}) -> GELU -> FC({C})"]
    layer = (["attention: {", "  branch: RMSNorm -> {", f"    q: FC({hq * D}){post}",
              f"    k: FC({hkv * D}){post}", f"    v: FC({hkv * D})",
              f"  }} -> GQA(q={hq}, kv={hkv}, d={D}{causal}) -> FC({C})", "  skip: Identity", "} -> Add", "",
              "ffn: {"] + ffn + ["  skip: Identity", "} -> Add"])
    if r.random() < 0.5:   # two layers (the DSL repeats a block only for counts of 2 and more)
        body = ["layer x 2: {"] + ["  " + ln if ln else "" for ln in layer] + ["}"]
    else:
        body = layer
    lines = ["input: 1x%dx%d" % (S, C), "prng: pcg32", "", "flow:"] + ["  " + ln if ln else "" for ln in body]
    lines += ["", f"  head: RMSNorm -> FC({V}) -> SoftmaxCE"]
    return "\n".join(lines) + "\n", r.choice((1, 2))


# seeds picked to cover both head dims, GQA ratios 1 to 4, QKNorm with and without RoPE, causal
# and not, SwiGLU and GELU, one and two layers; 2021 (one batch of 16 rows) from a sweep of 30
RANDOM_DECODER_SEEDS = (1000, 1005, 1008, 1010, 1015, 1021, 1029, 1037, 2021)


def models():
    out = [("cfg4", os.path.join(HERE, "models", "cfg4_llama.tkm"), 8, None),
           ("llama_small", os.path.join(HERE, "models", "llama_small.tkm"), 2, None),
           ("induction", os.path.join(HERE, "models", "induction.tkm"), 4, None),
           ("exotic_llama", os.path.join(REF, "models", "exotic_llama.tkm"), 2, None),
           ("llama3_style", os.path.join(REF, "models", "llama3_style.tkm"), 1, None),
           ("fused_check", None, 4, FUSED_CHECK)]
    for op in NUMCHECK_OPS:
        name = "numcheck_" + op.split("(")[0]
        out.append((name, None, 2, f"input: 1x1x32\ntest: {op} -> SoftmaxCE"))
    for seed in RANDOM_DECODER_SEEDS:
        text, batch = random_decoder(seed)
        out.append((f"rand_decoder_{seed}", None, batch, text))
    return out


def main() -> int:
    if not os.path.isdir(os.path.join(REF, "src")):
        print(f"reference checkout not found at {REF}; fixtures are generated in the build container only")
        return 1
    subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle"), "ref", f"REF={REF}"], check=True)
    arrays = {}
    with tempfile.TemporaryDirectory() as tmp:
        for name, path, batch, text in models():
            if path is None:
                path = os.path.join(tmp, name + ".tkm")
                with open(path, "w") as f:
                    f.write(text)
            prefix = os.path.join(tmp, name)
            r = subprocess.run([DUMP, "graph", path, str(batch), prefix], capture_output=True, text=True)
            if r.returncode != 0:
                print(r.stdout, r.stderr)
                raise SystemExit(f"front end failed on {name}")
            with open(prefix + ".bin", "rb") as f:
                arrays[f"{name}/graph"] = np.frombuffer(f.read(), dtype=np.uint8)
            with open(prefix + ".json") as f:
                js = json.load(f)
            arrays[f"{name}/json"] = np.frombuffer(json.dumps(js, sort_keys=True).encode(), dtype=np.uint8)
            print(f"{name}: {js['num_nodes']} nodes, {js['num_groups']} groups, "
                  f"arena {js['total_arena_bytes']} bytes")
    np.savez_compressed(os.path.join(HERE, "tkm_graphs.npz"), **arrays)
    reg = json.loads(subprocess.run([DUMP, "registry"], capture_output=True, text=True, check=True).stdout)
    with open(os.path.join(HERE, "tkm_registry.json"), "w") as f:
        json.dump(reg, f, indent=0)
    lay = json.loads(subprocess.run([DUMP, "layout"], capture_output=True, text=True, check=True).stdout)
    with open(os.path.join(HERE, "tkm_layout.json"), "w") as f:
        json.dump(lay, f, indent=0, sort_keys=True)
    print("wrote tkm_graphs.npz, tkm_registry.json, tkm_layout.json")
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Child process of tests/test_graph_gpu.py::test_first_attention_call_inside_capture.

Its very first attention call happens inside a global-mode stream capture, as in the
reference's tkm_runtime_step, which captures its first step (src/tkm_gpu.cu:1498-1508): the
library must load its gfx950 code objects then without recording the load and without
falling back to other kernels.  The captured fp16 D=128 forward + backward is replayed three
times (outputs overwritten with NaN in between) and must equal an eager run bit for bit.
Prints one line per check; exits non-zero on any failure.
"""
import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)


def main() -> int:
    import torch

    from tokamak_amd import attn, prep
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, S, Hq, Hkv, D = 2, 640, 4, 2, 128
    g = torch.Generator(device=dev)
    g.manual_seed(17)
    qkv = torch.randn((B, S, (Hq + 2 * Hkv) * D), generator=g, device=dev).half()
    dout = torch.randn((B, S, Hq * D), generator=g, device=dev).half()
    o = torch.empty((B, S, Hq * D), dtype=torch.float16, device=dev)
    lse = torch.empty((B, Hq, S), dtype=torch.float32, device=dev)
    dqkv = torch.empty_like(qkv)
    ws = torch.empty(attn.bwd_workspace_bytes(B, S, Hq), dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.synchronize()

    def step():
        attn.gqa_fwd(qkv, B, S, Hq, Hkv, D, causal=True, out=o, lse=lse, stream=stream)
        k_fwd = attn.last_kernels()
        attn.gqa_bwd(qkv, o, dout, lse, B, S, Hq, Hkv, D, causal=True, dqkv=dqkv, workspace=ws,
                     stream=stream)
        return k_fwd, attn.last_kernels()

    prep.Graph.begin(stream)
    try:
        k_fwd, k_bwd = step()
    finally:
        graph = prep.Graph.end(stream)
    print(f"captured first call: fwd kernels {k_fwd}, bwd kernels {k_bwd}", flush=True)
    if k_fwd != ["fwd_asm"] or k_bwd != ["dq_asm", "dkdv_asm"]:
        print("FAIL: the captured call did not take the assembly kernels", flush=True)
        return 1
    with torch.cuda.stream(stream):
        step()
    torch.cuda.synchronize()
    eager = [t.clone() for t in (o, lse, dqkv)]
    for rep in range(3):
        with torch.cuda.stream(stream):
            for t in (o, lse, dqkv):
                t.fill_(float("nan"))
        graph.launch(stream)
        stream.synchronize()
        for name, t, e in zip(("o", "lse", "dqkv"), (o, lse, dqkv), eager):
            if not torch.equal(t, e):
                print(f"FAIL: replay {rep}: {name} differs from the eager step", flush=True)
                return 1
        print(f"replay {rep}: o, lse, dqkv bitwise equal to the eager step", flush=True)
    graph.close()
    if not bool(torch.isfinite(o.float()).all()) or not bool(torch.isfinite(dqkv.float()).all()):
        print("FAIL: non-finite outputs", flush=True)
        return 1
    print("OK", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

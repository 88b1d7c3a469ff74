"""CPU checks of the assembly kernel generators (tokamak_amd/asmgen): each kernel generates
(its per-lane address arithmetic is checked against the index formulas while generating),
assembles for gfx950, and reads no register before something writes it in program order."""
import os
import shutil
import subprocess
import tempfile

import pytest

from tokamak_amd import build as tb
from tokamak_amd.asmgen import attn_dkdv, attn_dq, attn_fwd, gfx950

class Gen:
    """A generator with its element type: build() gives that kernel's text."""

    def __init__(self, mod, dt):
        self.mod, self.dt = mod, dt

    def build(self):
        return self.mod.build() if self.dt == "f16" else self.mod.build(dt=self.dt)

    def __repr__(self):
        return f"{self.mod.__name__.split('.')[-1]}-{self.dt}"


# (generator, workgroup-id SGPRs, registers defined on entry: the kernel arguments)
KERNELS = [(Gen(attn_fwd, "f16"), (1, 0, 0), {("s", 8 + i) for i in range(24)}),
           (Gen(attn_fwd, "bf16"), (1, 0, 0), {("s", 8 + i) for i in range(24)}),
           (Gen(attn_dkdv, "f16"), (1, 0, 0), {("s", 8 + i) for i in range(24)} | {("s", 90), ("s", 91)}),
           (Gen(attn_dkdv, "bf16"), (1, 0, 0), {("s", 8 + i) for i in range(24)} | {("s", 90), ("s", 91)}),
           (Gen(attn_dq, "f16"), (1, 0, 0), {("s", 8 + i) for i in range(34)}),
           (Gen(attn_dq, "bf16"), (1, 0, 0), {("s", 8 + i) for i in range(34)})]
IDS = [repr(k[0]) for k in KERNELS]


def _program(gen):
    """The instruction list of the generator's kernel (builds it once more, capturing Prog)."""
    captured = []
    orig = gfx950.Prog.finalize

    def finalize(self):
        captured.append(self)
        return orig(self)

    gfx950.Prog.finalize = finalize
    try:
        text = gen.build()
    finally:
        gfx950.Prog.finalize = orig
    return captured[-1], text


@pytest.mark.parametrize("gen,wg_ids,kernargs", KERNELS, ids=IDS)
def test_no_read_before_write(gen, wg_ids, kernargs):
    prog, _ = _program(gen)
    defined = {("s", 0), ("s", 1), ("v", 0), ("exec", 0)}
    nsys = sum(wg_ids)
    defined |= {("s", 2 + k) for k in range(nsys)}
    defined |= kernargs
    undefined = []
    for ins in prog.ins:
        for r in ins.reads:
            if r[0] in ("s", "v", "a", "m0") and r not in defined:
                undefined.append((ins.text, r))
        defined |= set(ins.writes)
    assert not undefined, undefined[:10]


@pytest.mark.parametrize("gen,wg_ids,kernargs", KERNELS, ids=IDS)
def test_assembles(gen, wg_ids, kernargs):
    try:
        clang = tb.llvm_tool("clang")
    except RuntimeError:
        pytest.skip("ROCm LLVM not installed")
    _, text = _program(gen)
    d = tempfile.mkdtemp()
    try:
        src, obj = os.path.join(d, "k.s"), os.path.join(d, "k.o")
        with open(src, "w") as f:
            f.write(text)
        r = subprocess.run([clang, "-x", "assembler", "-target", "amdgcn-amd-amdhsa", "-mcpu=gfx950",
                            "-c", src, "-o", obj], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
    finally:
        shutil.rmtree(d)


def test_split_scalar_keeps_scc_pairs():
    """Chunks of scalar code are cut only where SCC is dead."""
    p = gfx950.Prog()
    p.salu("s_cmp_eq_u32 s1, 0", [("s", 1)], [("scc", 0)])
    p.salu("s_mov_b32 s3, s4", [("s", 4)], [("s", 3)])
    p.salu("s_cselect_b32 s2, 1, 0", [("scc", 0)], [("s", 2)])
    p.salu("s_add_u32 s5, s5, 1", [("s", 5)], [("s", 5)])
    p.salu("s_addc_u32 s6, s6, 0", [("s", 6), ("scc", 0)], [("s", 6)])
    chunks = attn_dkdv.split_scalar(p.ins, 5)
    assert sum(len(c) for c in chunks) == 5
    flat = []
    for c in chunks:
        if c:
            flat.append([i.text.split()[0] for i in c])
    for c in flat:   # an SCC reader never starts a chunk
        assert c[0] not in ("s_cselect_b32", "s_addc_u32")


def _dead_loads(prog):
    """Loads (LDS reads, buffer loads) whose destination another load overwrites before any
    instruction reads it, within a basic block: the first load's data is lost."""
    pending = {}
    bad = []
    for ins in prog.ins:
        if ins.kind in (gfx950.LABEL, gfx950.BRANCH):
            pending.clear()
            continue
        for r in ins.reads:
            pending.pop(r, None)
        if ins.kind in (gfx950.DS_READ, gfx950.VMEM_LOAD):
            for r in ins.writes:
                if r in pending:
                    bad.append((pending[r], ins.text))
            for r in ins.writes:
                pending[r] = ins.text
        else:
            for r in ins.writes:
                pending.pop(r, None)
    return bad


@pytest.mark.parametrize("gen,wg_ids,kernargs", KERNELS, ids=IDS)
def test_no_dead_loads(gen, wg_ids, kernargs):
    prog, _ = _program(gen)
    bad = _dead_loads(prog)
    assert not bad, bad[:4]


def test_dead_load_check_catches_register_reuse(monkeypatch):
    """Six row reads in flight into four rotating registers (the lookahead above the number
    of read registers): the check must flag it."""
    monkeypatch.setattr(attn_dq, "LK", 6)
    prog, _ = _program(Gen(attn_dq, "f16"))
    assert _dead_loads(prog)

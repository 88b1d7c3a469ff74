"""A small gfx950 (CDNA4) assembly builder for hand-scheduled kernels.

Kernels are written as Python code that appends instructions in issue order, each tagged
with the registers it reads and writes and with its class (MFMA, VALU, transcendental,
LDS, VMEM, SALU, ...).  ``Prog.finalize`` then walks the instruction list once and makes
the code correct for the hardware without changing the order:

* waits: every read or overwrite of a register that is the destination of an outstanding
  LDS read gets an ``s_waitcnt lgkmcnt(n)`` with the largest n that covers it (LDS
  operations complete in order); the same for VMEM loads into VGPRs with ``vmcnt``.
  LDS-DMA loads (``buffer_load ... lds``) have no register destination: kernels wait for
  them explicitly before a barrier.
* hazards: the wait states below, which gfx950 does not enforce in hardware for these
  cases, are padded with ``s_nop``.  The figures are the ones the ROCm 7.2 compiler itself
  inserts for the same pairs of instructions on gfx950 (32x32x16 16-bit MFMA, 8 passes):

    MFMA writes r, then a non-MFMA instruction reads or writes r         12
    MFMA writes r, then an MFMA reads r as A/B, or as C unless it is the
      same accumulator range (back-to-back accumulation needs none)       12
    MFMA reads r as C, then a non-MFMA instruction writes r               12
    MFMA reads r as A/B, then a non-MFMA instruction writes r              4
    VALU writes r, then an MFMA reads r                                    2
    transcendental (v_exp/v_log/v_rcp) writes r, then anything reads r     2
    VALU writes r, then v_permlane32_swap reads r                          2
    VALU writes r, then v_readfirstlane / v_readlane reads r              2 (compiler: 1)
    SALU writes M0, then an LDS-DMA load                                   1
    SALU writes an SGPR, then a VMEM instruction reads it                  1
    VALU writes an SGPR (v_readfirstlane, v_cmp), then a non-VALU reads it 5
    VMEM store of more than 8 bytes, then anything writes its data VGPRs   2

  (A wait state is one issued instruction; ``s_nop N`` counts N+1.)
* before every branch, outstanding LDS reads and VMEM loads into registers are waited for
  and the MFMA/transcendental hazards are settled, so a jump target needs no state from
  the jump source.  Two exceptions, both the caller's promise about every path into a
  target: ``branch(..., keep_lgkm=True)`` leaves LDS reads in flight, and every target then
  starts with ``assume_lgkm`` naming exactly those reads (oldest first); ``skip_xdl``
  names MFMA destinations left unpadded because every target only accumulates into them
  with MFMAs (no wait states needed) or pads for them itself.
* v_mov_b32_dpp and v_permlane* are PERMLANE-class: they read a VGPR a VALU wrote no
  earlier than 2 wait states before.

Nothing here writes through the scalar data cache: the builder has no scalar store.
"""
from __future__ import annotations

from dataclasses import dataclass, field

XDL, VALU, TRANS, SALU, DS_READ, DS_WRITE, VMEM_LOAD, VMEM_STORE, DMA, SMEM, NOP, WAIT, BRANCH, \
    LABEL, BARRIER, PERMLANE, READLANE, ASSUME = range(18)

# hazard wait states (see module docstring)
W_XDL_RAW = 12
W_XDL_WAR_C = 12
W_XDL_WAR_AB = 4
W_VALU_XDL = 2
W_TRANS = 2
W_PERMLANE = 2
W_READLANE = 2
W_M0_DMA = 1
W_SALU_VMEM = 1
W_VALU_SGPR = 5
W_STORE_DATA = 2


def vr(i: int, n: int = 1) -> str:
    return f"v{i}" if n == 1 else f"v[{i}:{i + n - 1}]"


def ar(i: int, n: int = 1) -> str:
    return f"a{i}" if n == 1 else f"a[{i}:{i + n - 1}]"


def sr(i: int, n: int = 1) -> str:
    return f"s{i}" if n == 1 else f"s[{i}:{i + n - 1}]"


def V(i, n=1):
    return [("v", i + k) for k in range(n)]


def A(i, n=1):
    return [("a", i + k) for k in range(n)]


def S(i, n=1):
    return [("s", i + k) for k in range(n)]


@dataclass
class Ins:
    text: str
    kind: int
    reads: list = field(default_factory=list)
    writes: list = field(default_factory=list)
    # MFMA only: register lists of the A/B operands and the C operand, and the destination
    ab: list = field(default_factory=list)
    c: list = field(default_factory=list)
    dst: list = field(default_factory=list)
    # BRANCH: leave LDS reads in flight / MFMA destinations not to pad; ASSUME: reads in flight
    keep_lgkm: bool = False
    skip_xdl: object = None
    pending: list = field(default_factory=list)
    # VMEM_LOAD: not tracked by the automatic waits (the kernel waits for it explicitly)
    untracked: bool = False


class Prog:
    def __init__(self, coalesce_lgkm: bool = False):
        """coalesce_lgkm: an LDS wait in front of an MFMA also covers the reads the next MFMA
        needs that are already in flight (one wait per two MFMAs instead of one each)."""
        self.ins: list[Ins] = []
        self.coalesce_lgkm = coalesce_lgkm

    # ---- raw emission -------------------------------------------------------------------
    def emit(self, text, kind, reads=(), writes=(), **kw):
        self.ins.append(Ins(text, kind, list(reads), list(writes), **kw))

    def label(self, name):
        self.emit(f"{name}:", LABEL)

    def comment(self, text):
        self.emit(f"; {text}", LABEL)

    # ---- typed helpers ------------------------------------------------------------------
    def salu(self, text, reads=(), writes=()):
        self.emit(text, SALU, reads, writes)

    def valu(self, text, reads=(), writes=()):
        self.emit(text, VALU, reads, writes)

    def trans(self, text, reads=(), writes=()):
        self.emit(text, TRANS, reads, writes)

    def readlane(self, text, reads=(), writes=()):
        self.emit(text, READLANE, reads, writes)

    def mfma(self, op, dst, a, b, c, dst_acc=False, a_acc=False, b_acc=False, c_acc=None):
        """op vdst, srcA, srcB, srcC: dst and c are first registers of 16-register ranges;
        c is None for the inline constant 0."""
        c_acc = dst_acc if c_acc is None else c_acc
        R = A if dst_acc else V
        dl = R(dst, 16)
        al = (A if a_acc else V)(a, 4)
        bl = (A if b_acc else V)(b, 4)
        if c is None:
            cl, ctext = [], "0"
        else:
            cl = (A if c_acc else V)(c, 16)
            ctext = (ar if c_acc else vr)(c, 16)
        text = (f"{op} {(ar if dst_acc else vr)(dst, 16)}, {(ar if a_acc else vr)(a, 4)}, "
                f"{(ar if b_acc else vr)(b, 4)}, {ctext}")
        self.emit(text, XDL, al + bl + cl, dl, ab=al + bl, c=cl, dst=dl)

    def ds_read(self, text, dst, addr):
        self.emit(text, DS_READ, addr, dst)

    def ds_write(self, text, addr_data):
        self.emit(text, DS_WRITE, addr_data, [])

    def vmem_load(self, text, dst, reads, untracked=False):
        """untracked: no automatic wait for the destination (nor at branches); the kernel
        itself waits (vmcnt) before anything touches it."""
        self.emit(text, VMEM_LOAD, reads, dst, untracked=untracked)

    def vmem_store(self, text, reads):
        self.emit(text, VMEM_STORE, reads, [])

    def dma(self, text, reads):
        self.emit(text, DMA, reads + [("m0", 0)], [])

    def smem(self, text, dst, reads):
        self.emit(text, SMEM, reads, dst)

    def waitcnt(self, vm=None, lgkm=None):
        parts = []
        if vm is not None:
            parts.append(f"vmcnt({vm})")
        if lgkm is not None:
            parts.append(f"lgkmcnt({lgkm})")
        self.emit("s_waitcnt " + " ".join(parts), WAIT)

    def barrier(self):
        self.emit("s_barrier", BARRIER)

    def branch(self, text, reads=(), keep_lgkm=False, skip_xdl=None):
        self.emit(text, BRANCH, reads, keep_lgkm=keep_lgkm, skip_xdl=skip_xdl)

    def assume_lgkm(self, pending):
        """At a branch target: the LDS reads in flight on every path into it (register lists,
        oldest first)."""
        self.emit("", ASSUME, pending=[set(d) for d in pending])

    def permlane(self, text, reads=(), writes=()):
        self.emit(text, PERMLANE, reads, writes)

    def nop(self, n):
        while n > 0:
            k = min(n, 8)
            self.emit(f"s_nop {k - 1}", NOP)
            n -= k

    # ---- finalize: waits and hazard padding ---------------------------------------------
    def finalize(self) -> list[str]:
        out: list[str] = []
        ws = 0                     # running wait-state count (position of the next instruction)
        last_xdl_w = {}            # reg -> (ws after the MFMA, dst tuple)
        last_xdl_rc = {}           # reg -> ws after an MFMA read it as C
        last_xdl_rab = {}          # reg -> ws after an MFMA read it as A/B
        last_valu_w = {}           # reg -> ws after a VALU wrote it
        last_trans_w = {}          # reg -> ws after a transcendental wrote it
        last_salu_w = {}           # sgpr/m0 -> ws after a SALU wrote it
        last_valu_sw = {}          # sgpr -> ws after a VALU wrote it
        last_store_data = {}       # vgpr -> ws after a wide VMEM store read it as data
        lgkm = []                  # outstanding LDS reads: list of dst register sets
        vm = []                    # outstanding VMEM loads/DMAs: list of dst register sets

        def put(text, cost=1):
            nonlocal ws
            out.append(text)
            ws += cost

        def pad(need):
            nonlocal ws
            while need > 0:
                k = min(need, 8)
                put(f"\ts_nop {k - 1}", k)
                need -= k

        def settle_all(keep_lgkm=False, skip_xdl=None):
            # wait for every register-writing memory op, pad every pending hazard
            if lgkm and not keep_lgkm:
                put("\ts_waitcnt lgkmcnt(0)")
                lgkm.clear()
            if any(d for d in vm):
                put("\ts_waitcnt vmcnt(0)")
                vm.clear()
            need = 0
            for r, t in last_xdl_w.items():
                if skip_xdl is not None and r in skip_xdl:
                    continue
                need = max(need, t[0] + W_XDL_RAW - ws)
            for r, t in last_xdl_rc.items():
                if skip_xdl is not None and r in skip_xdl:
                    continue
                need = max(need, t + W_XDL_WAR_C - ws)
            for t in last_trans_w.values():
                need = max(need, t + W_TRANS - ws)
            for t in last_valu_sw.values():
                need = max(need, t + W_VALU_SGPR - ws)
            pad(need)

        for pos, ins in enumerate(self.ins):
            k = ins.kind
            if k == LABEL:
                out.append(ins.text if not ins.text.startswith(";") else "\t" + ins.text)
                continue
            if k == BRANCH:
                settle_all(ins.keep_lgkm, ins.skip_xdl)
                put("\t" + ins.text)
                continue
            if k == ASSUME:
                lgkm[:] = [set(d) for d in ins.pending]
                continue
            regs_r = set(ins.reads)
            regs_w = set(ins.writes)
            touched = regs_r | regs_w
            # --- memory-count waits
            if k != WAIT:
                idx = -1
                for i, d in enumerate(lgkm):
                    if d & touched:
                        idx = i
                if idx >= 0 and k == XDL and self.coalesce_lgkm:
                    for nxt in self.ins[pos + 1:]:
                        if nxt.kind in (BRANCH, LABEL, ASSUME, BARRIER):
                            break
                        if nxt.kind == XDL:
                            nt = set(nxt.reads) | set(nxt.writes)
                            for i, d in enumerate(lgkm):
                                if d & nt:
                                    idx = max(idx, i)
                            break
                if idx >= 0:
                    put(f"\ts_waitcnt lgkmcnt({len(lgkm) - 1 - idx})")
                    del lgkm[:idx + 1]
                idx = -1
                for i, d in enumerate(vm):
                    if d & touched:
                        idx = i
                if idx >= 0:
                    put(f"\ts_waitcnt vmcnt({len(vm) - 1 - idx})")
                    del vm[:idx + 1]
            else:
                # explicit waits: apply them to the model
                if "lgkmcnt(" in ins.text:
                    n = int(ins.text.split("lgkmcnt(")[1].split(")")[0])
                    del lgkm[:max(0, len(lgkm) - n)]
                if "vmcnt(" in ins.text:
                    n = int(ins.text.split("vmcnt(")[1].split(")")[0])
                    del vm[:max(0, len(vm) - n)]
            # --- hazards
            need = 0
            if k == XDL:
                dst_t = tuple(ins.dst)
                for r in ins.ab:
                    if r in last_xdl_w:
                        need = max(need, last_xdl_w[r][0] + W_XDL_RAW - ws)
                    if r in last_valu_w:
                        need = max(need, last_valu_w[r] + W_VALU_XDL - ws)
                    if r in last_trans_w:
                        need = max(need, last_trans_w[r] + W_TRANS - ws)
                for r in ins.c:
                    if r in last_xdl_w and last_xdl_w[r][1] != tuple(ins.c):
                        need = max(need, last_xdl_w[r][0] + W_XDL_RAW - ws)
                    if r in last_valu_w:
                        need = max(need, last_valu_w[r] + W_VALU_XDL - ws)
                    if r in last_trans_w:
                        need = max(need, last_trans_w[r] + W_TRANS - ws)
                for r in ins.dst:
                    if r in last_xdl_w and last_xdl_w[r][1] != dst_t:
                        need = max(need, last_xdl_w[r][0] + W_XDL_RAW - ws)
                    if r in last_valu_w:
                        need = max(need, last_valu_w[r] + W_VALU_XDL - ws)
            elif k not in (WAIT, NOP):
                for r in touched:
                    if r in last_xdl_w:
                        need = max(need, last_xdl_w[r][0] + W_XDL_RAW - ws)
                    if r in last_trans_w:
                        need = max(need, last_trans_w[r] + W_TRANS - ws)
                    if (r[0] == "s" or r[0] in ("vcc", "exec")) and k not in (VALU, TRANS, PERMLANE, READLANE):
                        if r in last_valu_sw:
                            need = max(need, last_valu_sw[r] + W_VALU_SGPR - ws)
                for r in regs_w:
                    if r in last_store_data:
                        need = max(need, last_store_data[r] + W_STORE_DATA - ws)
                    if r in last_xdl_rc:
                        need = max(need, last_xdl_rc[r] + W_XDL_WAR_C - ws)
                    if r in last_xdl_rab:
                        need = max(need, last_xdl_rab[r] + W_XDL_WAR_AB - ws)
                if k in (PERMLANE, READLANE):
                    w = W_PERMLANE if k == PERMLANE else W_READLANE
                    for r in regs_r:
                        if r in last_valu_w:
                            need = max(need, last_valu_w[r] + w - ws)
                if k in (DMA,):
                    if ("m0", 0) in last_salu_w:
                        need = max(need, last_salu_w[("m0", 0)] + W_M0_DMA - ws)
                if k in (DMA, VMEM_LOAD, VMEM_STORE):
                    for r in regs_r:
                        if r[0] == "s" and r in last_salu_w:
                            need = max(need, last_salu_w[r] + W_SALU_VMEM - ws)
            pad(need)
            # --- issue
            cost = 1
            if k == NOP:
                cost = int(ins.text.split()[1]) + 1
            put("\t" + ins.text, cost)
            # --- record
            if k == XDL:
                for r in ins.dst:
                    last_xdl_w[r] = (ws, tuple(ins.dst))
                    last_valu_w.pop(r, None)
                    last_trans_w.pop(r, None)
                for r in ins.c:
                    last_xdl_rc[r] = ws
                for r in ins.ab:
                    last_xdl_rab[r] = ws
            elif k in (VALU, TRANS, PERMLANE, READLANE):
                for r in regs_w:
                    last_xdl_w.pop(r, None)
                    if r[0] in ("v", "a"):
                        if k == TRANS:
                            last_trans_w[r] = ws
                            last_valu_w[r] = ws
                        else:
                            last_valu_w[r] = ws
                            last_trans_w.pop(r, None)
                    else:
                        last_valu_sw[r] = ws
            elif k == SALU:
                for r in regs_w:
                    last_salu_w[r] = ws
                    last_valu_sw.pop(r, None)
            elif k == DS_READ:
                for r in regs_w:
                    last_xdl_w.pop(r, None)
                    last_valu_w.pop(r, None)
                    last_trans_w.pop(r, None)
                lgkm.append(set(regs_w))
            elif k == DS_WRITE:
                lgkm.append(set())
            elif k == VMEM_STORE:
                data = [r for r in ins.reads if r[0] == "v"]
                if len(data) > 3:   # address + more than two data dwords
                    for r in data:
                        last_store_data[r] = ws
            elif k in (VMEM_LOAD, DMA):
                for r in regs_w:
                    last_xdl_w.pop(r, None)
                    last_valu_w.pop(r, None)
                    last_trans_w.pop(r, None)
                vm.append(set() if ins.untracked else set(regs_w))
            elif k == SMEM:
                for r in regs_w:
                    last_valu_sw.pop(r, None)
                    last_salu_w[r] = ws
                lgkm.append(set(regs_w))
            if len(lgkm) > 15:
                del lgkm[0]
            if len(vm) > 63:
                del vm[0]
        return out


def kernel_descriptor(name, *, lds_bytes, kernarg_bytes, next_free_sgpr, wg_ids=(1, 1, 1)):
    """Kernel descriptor for a kernel with 512 registers per lane (256 VGPR + 256 AGPR), one
    wave per SIMD, a kernarg pointer in s[0:1] and the workgroup ids after it."""
    return f"""
\t.rodata
\t.p2align 6
\t.amdhsa_kernel {name}
\t\t.amdhsa_group_segment_fixed_size {lds_bytes}
\t\t.amdhsa_private_segment_fixed_size 0
\t\t.amdhsa_kernarg_size {kernarg_bytes}
\t\t.amdhsa_user_sgpr_count 2
\t\t.amdhsa_user_sgpr_kernarg_segment_ptr 1
\t\t.amdhsa_enable_private_segment 0
\t\t.amdhsa_system_sgpr_workgroup_id_x {wg_ids[0]}
\t\t.amdhsa_system_sgpr_workgroup_id_y {wg_ids[1]}
\t\t.amdhsa_system_sgpr_workgroup_id_z {wg_ids[2]}
\t\t.amdhsa_system_vgpr_workitem_id 0
\t\t.amdhsa_next_free_vgpr 512
\t\t.amdhsa_next_free_sgpr {next_free_sgpr}
\t\t.amdhsa_accum_offset 256
\t\t.amdhsa_reserve_vcc 1
\t\t.amdhsa_float_round_mode_32 0
\t\t.amdhsa_float_round_mode_16_64 0
\t\t.amdhsa_float_denorm_mode_32 3
\t\t.amdhsa_float_denorm_mode_16_64 3
\t\t.amdhsa_dx10_clamp 1
\t\t.amdhsa_ieee_mode 1
\t\t.amdhsa_fp16_overflow 0
\t\t.amdhsa_tg_split 0
\t.end_amdhsa_kernel
"""


def metadata(name, *, args, lds_bytes, kernarg_bytes, sgpr_count, wg_size=256):
    """Code-object v5 metadata; args = [(offset, size, kind)] with kind 'ptr' or 'val'."""
    lines = ["\t.amdgpu_metadata", "---", "amdhsa.kernels:", "  - .agpr_count:     256",
             "    .args:"]
    for off, size, kind in args:
        if kind == "ptr":
            lines += [f"      - .address_space:  global", f"        .offset:         {off}",
                      f"        .size:           {size}", "        .value_kind:     global_buffer"]
        else:
            lines += [f"      - .offset:         {off}", f"        .size:           {size}",
                      "        .value_kind:     by_value"]
    lines += [
        f"    .group_segment_fixed_size: {lds_bytes}",
        "    .kernarg_segment_align: 8",
        f"    .kernarg_segment_size: {kernarg_bytes}",
        "    .language:       OpenCL C",
        "    .language_version:",
        "      - 2",
        "      - 0",
        f"    .max_flat_workgroup_size: {wg_size}",
        f"    .name:           {name}",
        "    .private_segment_fixed_size: 0",
        f"    .sgpr_count:     {sgpr_count}",
        "    .sgpr_spill_count: 0",
        f"    .symbol:         {name}.kd",
        "    .uniform_work_group_size: 1",
        "    .uses_dynamic_stack: false",
        "    .vgpr_count:     512",
        "    .vgpr_spill_count: 0",
        "    .wavefront_size: 64",
        "amdhsa.target:   amdgcn-amd-amdhsa--gfx950",
        "amdhsa.version:",
        "  - 1",
        "  - 2",
        "...",
        "\t.end_amdgpu_metadata",
    ]
    return "\n".join(lines) + "\n"


def kernel_text(name, body_lines, *, lds_bytes, kernarg_bytes, next_free_sgpr, args, wg_ids=(1, 1, 1)):
    head = [
        '\t.amdgcn_target "amdgcn-amd-amdhsa--gfx950"',
        "\t.text",
        f"\t.globl {name}",
        "\t.p2align 8",
        f"\t.type {name},@function",
        f"{name}:",
    ]
    tail = [f".Lfunc_end_{name}:", f"\t.size {name}, .Lfunc_end_{name}-{name}"]
    return ("\n".join(head + body_lines + tail) + "\n"
            + kernel_descriptor(name, lds_bytes=lds_bytes, kernarg_bytes=kernarg_bytes,
                                next_free_sgpr=next_free_sgpr, wg_ids=wg_ids)
            + metadata(name, args=args, lds_bytes=lds_bytes, kernarg_bytes=kernarg_bytes,
                       sgpr_count=next_free_sgpr + 6))

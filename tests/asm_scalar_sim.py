"""CPU interpreter of the scalar side of a generated attention kernel (test infrastructure).

It runs every workgroup of a launch wave by wave: scalar ALU, scalar loads from the kernel
arguments and kv_len, branches, M0, barriers, and the buffer descriptors of every DMA and
store.  Vector work is skipped: the vector results the scalar code consumes are the wave index
(v_readfirstlane of v0 >> 6) and lane masks of vector compares (the forward's rescale test:
every lane, or none, as the caller chooses).  Waves of a workgroup run until each reaches its next s_barrier, so
a barrier that not all four waves reach fails the run instead of hanging a GPU.

What the kernels under test must show: every workgroup terminates; each DMA and store
descriptor stays inside its tensor; and, through '; <event>' comment lines the generators
emit, the LDS tile a wave is about to read was written by DMA in an earlier barrier phase
with the expected rows, and is not written by any wave in the phase that reads it.

Lane reach: where the caller names, for a VGPR that holds per-lane offsets, the largest
offset any lane adds (lane_max: vgpr -> bytes, or a tuple of bytes per wave), an instruction `v_add_u32_e32 vX, sY, vZ`
records vX = sY + lanes(vZ); a buffer access through vX with `offen` must then touch no byte
past the end of the tensor the descriptor covers.  Lanes are taken to touch rows 0..k of the
tensor's pitch at columns up to lanes(vZ) mod pitch; offsets at or past num_records are
dropped by the hardware.
"""
from __future__ import annotations

import re

M32 = 0xFFFFFFFF
M64 = (1 << 64) - 1
_OPND = re.compile(r"^([sva])\[(\d+):(\d+)\]$|^([sva])(\d+)$")


def _operand(tok):
    m = _OPND.match(tok)
    if m:
        if m.group(1):
            lo, hi = int(m.group(2)), int(m.group(3))
            return (m.group(1), lo, hi - lo + 1)
        return (m.group(4), int(m.group(5)), 1)
    if tok in ("m0", "vcc", "exec", "scc", "off"):
        return (tok, 0, 1)
    try:
        return ("k", int(tok, 0), 1)
    except ValueError:
        return ("x", tok, 1)


def parse(lines):
    """Instruction list [(op, operands, text)] and label -> index."""
    ins, labels = [], {}
    for raw in lines:
        t = raw.strip()
        if not t:
            continue
        if t.endswith(":") and not t.startswith(";"):
            labels[t[:-1]] = len(ins)
            continue
        if t.startswith(";"):
            ins.append(("event", t[1:].strip().split(), t))
            continue
        parts = t.split(None, 1)
        op = parts[0]
        args = []
        if len(parts) > 1:
            for a in parts[1].split(","):
                a = a.strip()
                args.append(_operand(a.split()[0]) if a else None)
                # trailing modifiers (offen, lds, offset:N) of the last operand
                if " " in a:
                    for mod in a.split()[1:]:
                        args.append(("mod", mod, 1))
        ins.append((op, args, t))
    return ins, labels


class Fail(AssertionError):
    pass


class Wave:
    def __init__(self, wg, wave):
        self.s = {}
        self.scc = 0
        self.m0 = 0
        self.pc = 0
        self.wg, self.wave = wg, wave
        self.done = False
        self.loads = []         # (destination operand, descriptor base) of plain buffer loads
        self.load_nrec = {}     # descriptor base -> num_records of the plain buffer loads
        self.vscal = {}         # vgpr -> (scalar offset, largest lane offset) (lane reach)

    def get(self, o, w64=False):
        kind, i, n = o
        if kind == "s":
            v = self.s.get(i, None)
            if v is None:
                raise Fail(f"s{i} read before written")
            if w64 or n == 2:
                hi = self.s.get(i + 1, None)
                if hi is None:
                    raise Fail(f"s{i + 1} read before written")
                return v | (hi << 32)
            return v
        if kind == "k":
            return i & (M64 if w64 else M32)
        if kind == "m0":
            return self.m0
        if kind == "exec":
            return M64
        raise Fail(f"cannot read operand {o}")

    def put(self, o, v, w64=False):
        kind, i, n = o
        if kind == "s":
            self.s[i] = v & M32
            if w64 or n == 2:
                self.s[i + 1] = (v >> 32) & M32
        elif kind == "m0":
            self.m0 = v & M32
        elif kind == "exec":
            if (v & M64) != M64 and (v & M64) != 1:
                raise Fail("exec changed")
        else:
            raise Fail(f"cannot write operand {o}")


def _s32(x):
    x &= M32
    return x - (1 << 32) if x & 0x80000000 else x


class Sim:
    """kernarg: bytes of the argument segment; mem: name -> (base, bytes, row pitch, bytes a
    lane row touches) of the tensors the descriptors may cover; kv_len: list or None (its pointer in the arguments is nonzero then);
    n_wg: grid; vcmp_lanes: the lane mask every v_cmp_*_e64 writes; expect: a
    callable (wave, event words) -> list of checks [(lds_base, base, nrec)] of LDS tiles
    the wave reads at that event, or None; on_event(wave, words) for bookkeeping; wave_vgpr:
    the VGPR holding v0 >> 6 when the prologue reads the wave index from it."""

    def __init__(self, lines, kernarg, mem, kv_len, n_wg, expect, on_event=None, vcmp_lanes=M64,
                 tile_bytes=16384, max_steps=2_000_000, wave_vgpr=64, lane_max=None):
        self.ins, self.labels = parse(lines)
        self.lane_max = dict(lane_max or {})
        self.wave_vgpr = wave_vgpr
        self.kernarg = kernarg
        self.mem = mem
        self.kv_len = kv_len
        self.n_wg = n_wg
        self.expect = expect
        self.on_event = on_event
        self.vcmp_lanes = vcmp_lanes
        self.tile_bytes = tile_bytes
        self.max_steps = max_steps
        self.stores = []
        self.clock = 0

    # ---------------------------------------------------------------- memory checks
    def _desc(self, w, o):
        kind, i, n = o
        w0, w1, w2, w3 = (w.get(("s", i + k, 1)) for k in range(4))
        return w0 | ((w1 & 0xFFFF) << 32), w2, w3

    def _reach(self, w, vop, base, nrec, text):
        """Lane reach of a buffer access with offen through VGPR vop (see the module notes)."""
        if vop is None or vop[0] != "v":
            return
        got = w.vscal.get(vop[1])
        if got is None:
            return
        scal, lanes = got
        for name, (b0, size, pitch, _) in self.mem.items():
            if b0 <= base < b0 + size:
                # lanes touch rows 0..k of `pitch` bytes at columns up to `col`; offsets at or
                # past num_records are dropped
                k_top, col = divmod(lanes, pitch)
                if scal + lanes < nrec:
                    last = base + scal + lanes
                else:
                    k = (nrec - 1 - scal) // pitch
                    if k < 0:
                        return
                    last = base + min(scal + min(k, k_top) * pitch + col, nrec - 1)
                if last >= b0 + size:
                    raise Fail(f"{text}: a lane reaches {last - (b0 + size) + 1} bytes past the end of {name} "
                               f"(offset {scal:#x} + lanes {lanes:#x}, num_records {nrec:#x})")
                return

    def _inside(self, base, nrec, what):
        """The tensor a descriptor lies in: every byte of [base, base + num_records) must be
        inside it, so that no request through the descriptor, whatever its lane offsets, can
        reach memory past the tensor's end (the hardware drops only offsets at or past
        num_records)."""
        if nrec == 0:
            return None
        for name, (b0, size, pitch, row_bytes) in self.mem.items():
            if b0 <= base and base + nrec <= b0 + size:
                return name
        raise Fail(f"{what}: descriptor [{base:#x}, +{nrec}) outside every tensor")

    def run(self):
        for wg in range(self.n_wg):
            self._run_wg(wg)

    def _run_wg(self, wg):
        waves = [Wave(wg, w) for w in range(4)]
        for w in waves:
            w.s[2] = wg
            w.s[0], w.s[1] = 0, 0          # kernarg "pointer": offsets into self.kernarg
        self.lds = {}        # 1 KB slot -> (phase, base, nrec)
        self.reads = {}      # (phase) -> set of slots read
        self.writes = {}     # (phase) -> set of slots written
        phase = 0
        steps = 0
        while True:
            states = []
            for w in waves:
                if not w.done:
                    steps += self._run_until_barrier(w, phase)
                states.append(w.done)
            if all(states):
                break
            if any(states):
                raise Fail(f"wg {wg}: some waves ended while others wait at a barrier (phase {phase})")
            r = self.reads.get(phase, set()) & self.writes.get(phase, set())
            if r:
                raise Fail(f"wg {wg}: LDS slots {sorted(r)[:4]} read and written in one phase {phase}")
            phase += 1
            if steps > self.max_steps:
                raise Fail(f"wg {wg}: no end after {steps} instructions")

    def _run_until_barrier(self, w, phase):
        ins, labels = self.ins, self.labels
        n = 0
        while True:
            if w.pc >= len(ins):
                raise Fail("ran off the end of the program")
            op, a, text = ins[w.pc]
            w.pc += 1
            n += 1
            if n > self.max_steps:
                raise Fail(f"wave {w.wave} of wg {w.wg}: no barrier or end after {n} instructions")
            if op == "s_barrier":
                return n
            if op == "s_endpgm":
                w.done = True
                return n
            if op == "event":
                self._event(w, a, phase)
                continue
            if op.startswith("s_cbranch_") or op == "s_branch":
                tgt = a[0][1]
                if op == "s_branch" or (op == "s_cbranch_scc1" and w.scc) or (op == "s_cbranch_scc0" and not w.scc):
                    w.pc = labels[tgt]
                continue
            self._exec(w, op, a, text, phase)

    def _event(self, w, words, phase):
        if self.on_event is not None:
            self.on_event(w, words)
        checks = self.expect(w, words) if self.expect else None
        for lds_base, base, nrec in checks or ():
            for k in range(self.tile_bytes // 1024):
                slot = lds_base // 1024 + k
                got = self.lds.get(slot)
                if got is None:
                    raise Fail(f"{' '.join(words)}: LDS slot {slot} never written")
                ph, gb, gn, lrow = got
                if ph >= phase:
                    raise Fail(f"{' '.join(words)}: LDS slot {slot} written in the reading phase")
                if (gb, gn) != (base, nrec) or lrow != 4 * k:
                    raise Fail(f"{' '.join(words)} (wave {w.wave}, wg {w.wg}): LDS slot {slot} holds "
                               f"[{gb:#x}, +{gn}) row {lrow}, expected [{base:#x}, +{nrec}) row {4 * k}")
                self.reads.setdefault(phase, set()).add(slot)

    def _exec(self, w, op, a, text, phase):
        g = w.get
        if op == "v_add_u32_e32" and a[0][0] == "v" and a[1][0] == "s" and a[2][0] == "v":
            if a[2][1] in self.lane_max:
                lm = self.lane_max[a[2][1]]
                w.vscal[a[0][1]] = (g(a[1]), lm[w.wave] if isinstance(lm, (tuple, list)) else lm)
            else:
                w.vscal.pop(a[0][1], None)
            return
        if op in ("s_waitcnt", "s_nop", "s_setprio") or op.startswith("v_") and not (
                op == "v_readfirstlane_b32" or (op.startswith("v_cmp") and op.endswith("_e64"))):
            if op.startswith("v_") and a and a[0] and a[0][0] == "v":
                for k in range(a[0][2]):
                    w.vscal.pop(a[0][1] + k, None)
            return
        if op == "v_readfirstlane_b32":
            src = a[1]
            if src != ("v", self.wave_vgpr, 1):
                raise Fail(f"v_readfirstlane of an unmodelled register: {text}")
            w.put(a[0], w.wave)           # wave index (v0 >> 6 in the prologue)
            return
        if op.startswith("v_cmp") and op.endswith("_e64"):
            w.put(a[0], self.vcmp_lanes, True)
            return
        if op.startswith("s_load_dword"):
            cnt = {"s_load_dword": 1, "s_load_dwordx2": 2, "s_load_dwordx4": 4, "s_load_dwordx8": 8,
                   "s_load_dwordx16": 16}[op]
            base = g(a[1], True)
            off = g(a[2]) if a[2][0] == "s" else a[2][1]
            for k in range(cnt):
                addr = base + off + 4 * k
                if a[1][1] == 0:
                    v = int.from_bytes(self.kernarg[addr:addr + 4], "little")
                else:
                    idx = (addr - self.mem["kv_len"][0]) // 4
                    if self.kv_len is None or not 0 <= idx < len(self.kv_len):
                        raise Fail(f"kv_len load out of range: {idx}")
                    v = self.kv_len[idx] & M32
                w.s[a[0][1] + k] = v
            return
        if op.startswith("buffer_load") and any(x and x[0] == "mod" and x[1] == "lds" for x in a):
            base, nrec, w3 = self._desc(w, a[1])
            self._inside(base, nrec, text)
            if any(x and x[0] == "mod" and x[1] == "offen" for x in a):
                self._reach(w, a[0], base, nrec, text)
            slot = w.m0 // 1024
            self.lds[slot] = (phase, base, nrec, (w.m0 % self.tile_bytes) // 256)
            self.writes.setdefault(phase, set()).add(slot)
            return
        if op.startswith("buffer_load"):
            base, nrec, _ = self._desc(w, a[2])
            self._inside(base, nrec, text)
            w.loads.append((a[0], base))
            w.load_nrec[base] = nrec
            return
        if op.startswith("buffer_store"):
            base, nrec, _ = self._desc(w, a[2])
            self.stores.append((w.wg, w.wave, self._inside(base, nrec, text), base, nrec))
            return
        if op in ("s_memtime", "s_memrealtime"):
            self.clock += 1000
            w.put(a[0], self.clock, True)
            return
        if op.startswith("ds_"):
            return
        b64 = op.endswith("_b64") or op.endswith("_u64")
        if op in ("s_mov_b32", "s_mov_b64"):
            w.put(a[0], g(a[1], b64), b64)
        elif op in ("s_add_u32", "s_addc_u32"):
            r = g(a[1]) + g(a[2]) + (w.scc if op == "s_addc_u32" else 0)
            w.scc = int(r > M32)
            w.put(a[0], r)
        elif op == "s_sub_u32":
            x, y = g(a[1]), g(a[2])
            w.scc = int(y > x)
            w.put(a[0], x - y)
        elif op == "s_sub_i32":
            w.put(a[0], _s32(g(a[1])) - _s32(g(a[2])))
        elif op in ("s_lshl1_add_u32", "s_lshl2_add_u32"):
            r = (g(a[1]) << (1 if op == "s_lshl1_add_u32" else 2)) + g(a[2])
            w.scc = int(r > M32)
            w.put(a[0], r)
        elif op == "s_mul_i32":
            w.put(a[0], g(a[1]) * g(a[2]))
        elif op == "s_mul_hi_u32":
            w.put(a[0], (g(a[1]) * g(a[2])) >> 32)
        elif op in ("s_lshl_b32", "s_lshr_b32"):
            x, n = g(a[1]), g(a[2]) & 31
            r = ((x << n) if op == "s_lshl_b32" else (x >> n)) & M32
            w.scc = int(r != 0)
            w.put(a[0], r)
        elif op in ("s_and_b32", "s_or_b32", "s_andn2_b32", "s_xor_b32",
                    "s_and_b64", "s_or_b64", "s_andn2_b64"):
            x, y = g(a[1], b64), g(a[2], b64)
            kind = op[2:].split("_")[0]
            r = {"and": x & y, "or": x | y, "andn2": x & ~y, "xor": x ^ y}[kind] & (M64 if b64 else M32)
            w.scc = int(r != 0)
            w.put(a[0], r, b64)
        elif op in ("s_min_i32", "s_max_i32"):
            x, y = _s32(g(a[1])), _s32(g(a[2]))
            w.put(a[0], min(x, y) if op == "s_min_i32" else max(x, y))
        elif op in ("s_min_u32", "s_max_u32"):
            x, y = g(a[1]), g(a[2])
            w.put(a[0], min(x, y) if op == "s_min_u32" else max(x, y))
        elif op.startswith("s_cmp_"):
            _, _, rel, ty = op.split("_")
            x, y = g(a[0], ty == "u64"), g(a[1], ty == "u64")
            if ty == "i32":
                x, y = _s32(x), _s32(y)
            w.scc = int({"eq": x == y, "lg": x != y, "lt": x < y, "le": x <= y, "gt": x > y,
                         "ge": x >= y}[rel])
        elif op == "s_cselect_b32":
            w.put(a[0], g(a[1]) if w.scc else g(a[2]))
        elif op == "s_bitcmp1_b32":
            w.scc = (g(a[0]) >> (g(a[1]) & 31)) & 1
        else:
            raise Fail(f"instruction not modelled: {text}")

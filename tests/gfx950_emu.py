"""Test infrastructure: a CPU emulator of one wave of a gfx950 kernel's
generated assembly, for the integer and address part of the code.

Kernels that load weights into registers with inline asm (so that the
compiler's own conservative waits do not drain the prefetch) rely on the
register allocator never copying or reusing a destination register while its
load is in flight: such a copy reads a stale value, and a register reused for
an address is overwritten when the late load lands (a wild address, a GPU
memory fault). The compiler cannot see this hazard; this emulator does.

It runs one wave with concrete kernel arguments and tracks:
- scalar and vector integer values (unknown where they come from memory the
  test does not describe, from LDS written by DMA, or from float data ops);
- the in-order queue of outstanding vector memory operations (s_waitcnt
  vmcnt(N) retires all but the N youngest) and, per register, whether it may
  hold a stale or clobbered value ("poisoned"), propagated through every
  instruction that reads it;
- every global, buffer and LDS access, checked against the buffers and LDS
  size of the launch, and whether any address, stored value or MFMA operand
  is poisoned.
Barriers are counted, not waited on: the waves of a workgroup run one after
another, sharing LDS (the code checked here publishes only routing scalars and
row tables through LDS), and a test compares the waves' barrier counts."""
import re, struct, sys
import numpy as np

M32 = 0xFFFFFFFF
NL = 64

class Unknown(Exception):
    pass

def f2u(x): return struct.unpack("<I", struct.pack("<f", x))[0]
INLINE_F = {"0.5": f2u(0.5), "-0.5": f2u(-0.5), "1.0": f2u(1.0), "-1.0": f2u(-1.0), "2.0": f2u(2.0),
            "-2.0": f2u(-2.0), "4.0": f2u(4.0), "-4.0": f2u(-4.0)}

def load_kernel(asm_path, fn):
    lines = open(asm_path).read().split("\n")
    i0 = next(i for i, l in enumerate(lines) if l.startswith(fn + ":"))
    ins, labels = [], {}
    for l in lines[i0 + 1:]:
        if l.startswith(".Lfunc_end"): break
        s = l.split(";")[0].strip()
        if not s: continue
        if s.endswith(":"):
            labels[s[:-1]] = len(ins); continue
        if s.startswith("."): continue
        ins.append(s)
    return ins, labels

class Wave:
    def __init__(self, mem, kernarg, wg_id, wave_in_wg, buffers, lds_size):
        self.s = [0] * 128; self.sk = [True] * 128
        self.v = np.zeros((256, NL), dtype=np.uint64); self.vk = np.ones((256, NL), dtype=bool)
        self.exec = (1 << 64) - 1; self.vcc = 0; self.scc = 0; self.m0 = 0
        self.mem = mem; self.buffers = buffers; self.lds_size = lds_size
        self.s[0], self.s[1] = kernarg & M32, kernarg >> 32
        self.s[2] = wg_id
        self.v[0] = np.arange(NL, dtype=np.uint64) + wave_in_wg * 64
        self.lds = {}  # byte address -> (value byte, known)
        self.errors = []; self.accesses = 0; self.cur_poison = False; self.m0poison = False; self.trace = []
        self.vmq = []  # outstanding vmem ops: [dest vgpr set, set of dests written since issue]
        self.poison = np.zeros(256, dtype=bool)  # register may hold a stale or clobbered value
        self.spoison = [False] * 128
        self.barriers = 0  # s_barrier instructions executed (all waves of a workgroup must agree)
    # ---- operand helpers
    def sreg(self, t):
        m = re.match(r"s\[(\d+):(\d+)\]$", t)
        if m: return list(range(int(m.group(1)), int(m.group(2)) + 1))
        m = re.match(r"s(\d+)$", t)
        if m: return [int(m.group(1))]
        return None
    def vreg(self, t):
        m = re.match(r"v\[(\d+):(\d+)\]$", t)
        if m: return list(range(int(m.group(1)), int(m.group(2)) + 1))
        m = re.match(r"v(\d+)$", t)
        if m: return [int(m.group(1))]
        return None
    def lit(self, t):
        if t in INLINE_F: return INLINE_F[t]
        if re.match(r"-?0x[0-9a-fA-F]+$", t) or re.match(r"-?\d+$", t):
            return int(t, 0) & 0xFFFFFFFFFFFFFFFF
        return None
    def sget(self, t, n=1):
        """scalar value (n dwords) of operand t"""
        if t == "vcc": return self.vcc
        if t == "exec": return self.exec
        if t == "m0": return self.m0
        if t == "scc": return self.scc
        if t in ("vcc_lo",): return self.vcc & M32
        if t in ("vcc_hi",): return self.vcc >> 32
        r = self.sreg(t)
        if r is not None:
            for i in r:
                if not self.sk[i]: raise Unknown(f"unknown {t}")
            val = 0
            for k, i in enumerate(r): val |= self.s[i] << (32 * k)
            return val
        m = re.match(r"([\w.$]+)@rel32@(lo|hi)[+-]\d+$", t)
        if m:
            # PC-relative address of a device symbol: s_getpc_b64 reads as 0,
            # so the relocation halves are the symbol's own address (a buffer
            # registered under its mangled name)
            a = self.buffers[m.group(1)][0]
            return a & M32 if m.group(2) == "lo" else a >> 32
        L = self.lit(t)
        if L is not None:
            if n == 2 and L < 0x100000000 and t.startswith("-"): return L
            return L if n == 2 else L & M32
        raise ValueError("scalar operand " + t)
    def sset(self, t, val, n=1, known=True):
        if t == "vcc": self.vcc = val & 0xFFFFFFFFFFFFFFFF; return
        if t == "exec": self.exec = val & 0xFFFFFFFFFFFFFFFF; return
        if t == "m0": self.m0 = val & M32; return
        if t == "vcc_lo": self.vcc = (self.vcc & ~M32) | (val & M32); return
        if t == "vcc_hi": self.vcc = (self.vcc & M32) | ((val & M32) << 32); return
        r = self.sreg(t)
        for k, i in enumerate(r):
            self.s[i] = (val >> (32 * k)) & M32; self.sk[i] = known
    def vget(self, t, n=1):
        """per-lane value array (uint64) of operand t, n dwords"""
        r = self.vreg(t)
        if r is not None:
            val = np.zeros(NL, dtype=np.uint64); kn = np.ones(NL, dtype=bool)
            for k, i in enumerate(r[:n] if n else r):
                val |= self.v[i] << np.uint64(32 * k); kn &= self.vk[i]
            return val, kn
        if t.startswith("s") or t in ("vcc", "exec", "m0") or t.startswith("-") or t[0].isdigit() or t in INLINE_F:
            try:
                sv = self.sget(t, n)
            except Unknown:
                return np.zeros(NL, dtype=np.uint64), np.zeros(NL, dtype=bool)
            return np.full(NL, sv, dtype=np.uint64), np.ones(NL, dtype=bool)
        raise ValueError("vector operand " + t)
    def vset(self, t, val, kn, n=None):
        r = self.vreg(t)
        act = self.act()
        for k, i in enumerate(r):
            part = (val >> np.uint64(32 * k)) & np.uint64(M32)
            self.v[i] = np.where(act, part, self.v[i]); self.vk[i] = np.where(act, kn, self.vk[i])
            for q in self.vmq:
                if i in q[0]: q[1].add(i)  # written while a load to it is pending
            self.poison[i] = self.cur_poison
    def act(self):
        return np.array([(self.exec >> l) & 1 for l in range(NL)], dtype=bool)
    def mask_from(self, b):  # bool array -> 64-bit mask (active lanes only)
        m = 0
        for l in range(NL):
            if b[l]: m |= 1 << l
        return m
    def check_inflight_read(self, t):
        """True if operand t may read a stale / clobbered value"""
        r = self.vreg(t)
        bad = False
        if r:
            for i in r:
                if self.poison[i]: bad = True
                for q in self.vmq:
                    if i in q[0]: bad = True  # pending load: old or new value
        r = self.sreg(t)
        if r:
            for i in r:
                if self.spoison[i]: bad = True
        if bad and len(self.trace) < 8:
            rv = self.vreg(t) or []
            self.trace.append((self.cur, t, [i for i in rv if self.poison[i]], [i for i in rv for q in self.vmq if i in q[0]]))
        return bad
    def check_addr(self, addr, kn, size, what, lanes):
        for l in range(NL):
            if not lanes[l]: continue
            if not kn[l]:
                self.errors.append((what, "unknown address", l, self.cur)); return
            a = int(addr[l])
            ok = any(lo <= a and a + size <= hi for (lo, hi) in self.buffers.values())
            if not ok:
                self.errors.append((what, hex(a), size, l, self.cur)); return
        self.accesses += 1

def signed32(x): return x - (1 << 32) if x & 0x80000000 else x
def signed64(x): return x - (1 << 64) if x & (1 << 63) else x

def run(ins, labels, w, max_steps=2_000_000):
    pc = 0; steps = 0
    U64 = np.uint64
    while True:
        steps += 1
        if steps > max_steps: raise RuntimeError("too many steps")
        s = ins[pc]; w.cur = (pc, s)
        parts = s.split(None, 1); op = parts[0]; args = parts[1] if len(parts) > 1 else ""
        t = [x for x in re.split(r",\s*|\s+", args) if x]
        pc += 1
        if op == "s_endpgm": return
        if op.startswith("s_waitcnt"):
            m = re.search(r"vmcnt\((\d+)\)", args)
            if m:
                k = int(m.group(1))
                while len(w.vmq) > k:
                    dests, written = w.vmq.pop(0)
                    for r in dests:
                        w.poison[r] = r in written  # a landing after a newer write clobbers it
                        if r in written and len(w.trace) < 8: w.trace.append(("CLOBBER at wait", w.cur, r))
            continue
        if op == "s_barrier":
            w.barriers += 1; continue
        if op in ("s_nop", "s_setprio", "s_sleep") : continue
        if op == "s_branch": pc = labels[t[0]]; continue
        if op.startswith("s_cbranch"):
            cond = op[len("s_cbranch_"):]
            take = {"scc0": w.scc == 0, "scc1": w.scc == 1, "vccz": (w.vcc & w.exec) == 0,
                    "vccnz": (w.vcc & w.exec) != 0, "execz": w.exec == 0, "execnz": w.exec != 0}[cond]
            if take: pc = labels[t[0]]
            continue
        # ---- scalar ALU
        if op.startswith("s_") and not op.startswith("s_load") and not op.startswith("s_buffer"):
            pz = any(w.check_inflight_read(x) for x in t[1:]) if len(t) > 1 else False
            if op.startswith("s_cmp"): pz = any(w.check_inflight_read(x) for x in t)
            try:
                sop(w, op, t)
            except Unknown:
                w.sset(t[0], 0, known=False)
            if not op.startswith("s_cmp"):
                if t and t[0] == "m0": w.m0poison = pz
                r = w.sreg(t[0]) if t else None
                if r:
                    for i in r: w.spoison[i] = pz
            continue
        if op.startswith("s_load"):
            n = {"s_load_dword": 1, "s_load_dwordx2": 2, "s_load_dwordx4": 4, "s_load_dwordx8": 8}[op]
            base = w.sget(t[1], 2)
            off = w.sget(t[2]) if t[2].startswith("s") else int(t[2], 0)  # soffset register or immediate
            for x in t[3:]:
                if x.startswith("offset:"): off += int(x[7:], 0)
            addr = (base + off) & 0xFFFFFFFFFFFFFFFF
            ok = any(lo <= addr and addr + 4 * n <= hi for (lo, hi) in w.buffers.values()) or addr in w.mem
            vals = [w.mem.get(addr + 4 * k) for k in range(n)]
            for k, r in enumerate(w.sreg(t[0])):
                w.s[r] = vals[k] if vals[k] is not None else 0; w.sk[r] = vals[k] is not None
            if not ok: w.errors.append(("s_load OOB", hex(addr), w.cur))
            continue
        # ---- vector memory
        if op.startswith("global_load_lds"):
            addr, kn = gaddr(w, t[0], t[1])
            if w.check_inflight_read(t[0]): w.errors.append(("POISONED ADDRESS lds_dma", w.cur))
            if getattr(w, "m0poison", False): w.errors.append(("POISONED M0", w.cur))
            w.check_addr(addr, kn, 16, "lds_dma", w.act())
            lds = w.m0
            act_l = [l for l in range(NL) if (w.exec >> l) & 1]
            if act_l and lds + (max(act_l) + 1) * 16 > w.lds_size: w.errors.append(("lds dma beyond LDS", lds, w.cur))
            for l in range(NL):
                if (w.exec >> l) & 1:
                    for b in range(16): w.lds.pop(lds + 16 * l + b, None)
            w.vmq.append([set(), set()]); continue
        if op.startswith("global_load"):
            n = {"global_load_dword": 1, "global_load_dwordx2": 2, "global_load_dwordx4": 4,
                 "global_load_ushort": 1}[op]
            addr, kn = gaddr(w, t[1], t[2])
            off = 0
            for x in t[3:]:
                if x.startswith("offset:"): off = int(x[7:], 0)
            addr = (addr.astype(object) + off)
            addr = np.array([int(x) & 0xFFFFFFFFFFFFFFFF for x in addr], dtype=U64); off = 0
            if w.check_inflight_read(t[1]): w.errors.append(("POISONED ADDRESS load", w.cur))
            w.check_addr(addr + U64(off), kn, 4 * n, op, w.act())
            kn_addr = kn
            r = w.vreg(t[0])
            act = w.act()
            for j, i in enumerate(r):
                vals = np.zeros(NL, dtype=np.uint64); kn = np.zeros(NL, dtype=bool)
                for l in range(NL):
                    if act[l] and kn_addr[l]:
                        m = w.mem.get(int(addr[l]) + off + 4 * j)
                        if m is not None: vals[l] = m; kn[l] = True
                w.v[i] = np.where(act, vals, w.v[i])
                w.vk[i] = np.where(act, kn, w.vk[i])
                for q in w.vmq:
                    if i in q[0]: q[1].add(i)
                w.poison[i] = False
            w.vmq.append([set(r), set()]); continue
        if op.startswith("scratch_store") or op.startswith("scratch_load"):
            # register spills: private per-lane memory, dword granular
            store = op.startswith("scratch_store")
            size = {"byte": 1, "short": 2, "dword": 4, "dwordx2": 8, "dwordx3": 12, "dwordx4": 16}[op.split("_", 2)[2]
                                                                                                 .replace("ubyte", "byte").replace("ushort", "short").replace("sbyte", "byte").replace("sshort", "short")
                                                                                                 .replace("short_d16_hi", "short").replace("short_d16", "short")]
            data, vaddr, saddr = (t[1], t[0], t[2]) if store else (t[0], t[1], t[2])
            off = 0
            for x in t[3:]:
                if x.startswith("offset:"): off = int(x[7:], 0)
            base = np.zeros(NL, dtype=np.uint64); kb = np.ones(NL, dtype=bool)
            if vaddr != "off": base, kb = w.vget(vaddr)
            if saddr != "off": base = base + np.uint64(w.sget(saddr))
            if not hasattr(w, "scratch"): w.scratch = {}
            act = w.act()
            nd = max(1, size // 4)
            if store:
                if w.check_inflight_read(data): w.errors.append(("STALE DATA spilled", w.cur))
                vals, kn = w.vget(data, nd)
                regs = w.vreg(data)
                pz = any(w.poison[i] for i in regs)
                for l in range(NL):
                    if not act[l]: continue
                    if not kb[l]: w.errors.append(("scratch unknown address", w.cur)); continue
                    a = int(base[l]) + off
                    for k in range(nd):
                        v = int(w.v[regs[k]][l]) if k < len(regs) else 0
                        w.scratch[(l, a + 4 * k)] = (v, bool(w.vk[regs[k]][l]) and size >= 4, pz)
                w.vmq.append([set(), set()]); continue
            r = w.vreg(data)
            for k, i in enumerate(r):
                vals = np.zeros(NL, dtype=np.uint64); kn = np.zeros(NL, dtype=bool); pz = False
                for l in range(NL):
                    if act[l] and kb[l]:
                        e = w.scratch.get((l, int(base[l]) + off + 4 * k))
                        if e is not None:
                            vals[l], kn[l] = e[0], e[1] and size >= 4
                            pz = pz or e[2]
                w.v[i] = np.where(act, vals, w.v[i])
                w.vk[i] = np.where(act, kn, w.vk[i])
                for q in w.vmq:
                    if i in q[0]: q[1].add(i)
                w.poison[i] = pz
            w.vmq.append([set(r), set()]); continue
        if op.startswith("global_store"):
            size = {"global_store_byte": 1, "global_store_short": 2, "global_store_dword": 4,
                    "global_store_dwordx2": 8, "global_store_dwordx4": 16}[op]
            if w.check_inflight_read(t[1]): w.errors.append(("STALE DATA stored", w.cur))
            if w.check_inflight_read(t[0]): w.errors.append(("POISONED ADDRESS store", w.cur))
            addr, kn = gaddr(w, t[0], t[2])
            off = 0
            for x in t[3:]:
                if x.startswith("offset:"): off = int(x[7:], 0)
            addr = np.array([(int(a) + off) & 0xFFFFFFFFFFFFFFFF for a in addr], dtype=U64)
            w.check_addr(addr, kn, size, op, w.act())
            w.vmq.append([set(), set()]); continue
        if op.startswith("buffer_store"):
            n = {"buffer_store_dword": 1, "buffer_store_dwordx2": 2, "buffer_store_dwordx4": 4}[op]
            if w.check_inflight_read(t[0]): w.errors.append(("STALE DATA stored", w.cur))
            if w.check_inflight_read(t[1]) or w.check_inflight_read(t[2]): w.errors.append(("POISONED ADDRESS store", w.cur))
            rs = w.sreg(t[2]); base = w.s[rs[0]] | ((w.s[rs[1]] & 0xFFFF) << 32); nrec = w.s[rs[2]]
            voff, kn = w.vget(t[1], 1)
            soff = int(t[3], 0)
            act = w.act()
            for l in range(NL):
                if not act[l]: continue
                if not kn[l]: w.errors.append(("store unknown offset", l, w.cur)); break
                o = int(voff[l]) + soff
                if o + 4 * n <= nrec:
                    a = base + o
                    if not any(lo <= a and a + 4 * n <= hi for (lo, hi) in w.buffers.values()):
                        w.errors.append(("store OOB", hex(a), l, w.cur)); break
            w.vmq.append([set(), set()]); continue
        if op.startswith("ds_") or op.startswith("v_mfma") or op.startswith("v_pk_") or op.startswith("v_cvt_pk_f16") \
                or op in ("v_add_f16_e32", "v_and_or_b32") and False:
            if op.startswith("ds_write2") or op.startswith("ds_read2"):
                # two accesses of one element size (b32 / b64): offset0 / offset1
                # in elements (x64 for the st64 forms)
                es = 8 if op.endswith("b64") else 4
                unit = es * (64 if "st64" in op else 1)
                o0 = o1 = 0
                for x in t:
                    if x.startswith("offset0:"): o0 = int(x[8:], 0)
                    if x.startswith("offset1:"): o1 = int(x[8:], 0)
                write = op.startswith("ds_write2")
                av = t[0] if write else t[1]
                if w.check_inflight_read(av): w.errors.append(("POISONED ADDRESS ds", w.cur))
                a, ka = w.vget(av); act = w.act()
                if write:
                    if any(w.check_inflight_read(x) for x in t[1:3]): w.errors.append(("STALE DATA to LDS", w.cur))
                    for half, (dreg, oo) in enumerate(((t[1], o0), (t[2], o1))):
                        regs = w.vreg(dreg)
                        for l in range(NL):
                            if not act[l]: continue
                            if not ka[l]: w.errors.append(("ds_write unknown address", w.cur)); break
                            base = int(a[l]) + oo * unit
                            if base + es > w.lds_size: w.errors.append(("ds_write beyond LDS", base, w.cur))
                            for b in range(es):
                                i = regs[b // 4]
                                w.lds[base + b] = ((int(w.v[i][l]) >> (8 * (b % 4))) & 0xFF, bool(w.vk[i][l]))
                    continue
                r = w.vreg(t[0]); nd = es // 4
                for half, oo in enumerate((o0, o1)):
                    for j in range(nd):
                        i = r[half * nd + j]
                        vals = np.zeros(NL, dtype=np.uint64); kn = np.zeros(NL, dtype=bool)
                        for l in range(NL):
                            if not act[l] or not ka[l]: continue
                            base = int(a[l]) + oo * unit + 4 * j
                            if base + 4 > w.lds_size: w.errors.append(("ds_read beyond LDS", base, w.cur))
                            v = 0; k = True
                            for b in range(4):
                                e = w.lds.get(base + b)
                                if e is None: k = False; break
                                v |= e[0] << (8 * b); k &= e[1]
                            vals[l] = v; kn[l] = k
                        w.v[i] = np.where(act, vals, w.v[i]); w.vk[i] = np.where(act, kn, w.vk[i])
                        for q in w.vmq:
                            if i in q[0]: q[1].add(i)
                        w.poison[i] = False
                continue
            if op.startswith("ds_write"):
                if w.check_inflight_read(t[0]): w.errors.append(("POISONED ADDRESS ds", w.cur))
                if any(w.check_inflight_read(x) for x in t[1:]): w.errors.append(("STALE DATA to LDS", w.cur))
                nb = {"ds_write_b32": 4, "ds_write_b64": 8, "ds_write_b96": 12, "ds_write_b128": 16,
                      "ds_write_b16": 2}[op]
                off = 0
                for x in t[2:]:
                    if x.startswith("offset:"): off = int(x[7:], 0)
                a, ka = w.vget(t[0])
                # data dword by dword (a uint64 lane value holds two)
                dr = w.vreg(t[1])
                nd = max(1, nb // 4)
                if dr is not None:
                    dws = [(w.v[i], w.vk[i]) for i in dr[:nd]]
                else:
                    d0, k0 = w.vget(t[1]); dws = [(d0, k0)]
                act = w.act()
                for l in range(NL):
                    if not act[l]: continue
                    if not ka[l]: w.errors.append(("ds_write unknown address", w.cur)); break
                    base = int(a[l]) + off
                    if base + nb > w.lds_size: w.errors.append(("ds_write beyond LDS", base, w.cur))
                    for b in range(nb):
                        dv, dk = dws[min(b // 4, len(dws) - 1)]
                        w.lds[base + b] = ((int(dv[l]) >> (8 * (b % 4))) & 0xFF, bool(dk[l]))
                continue
            if op in ("ds_read_b32", "ds_read_b64", "ds_read_b96", "ds_read_u16", "ds_read_b128", "ds_read_u8",
                      "ds_bpermute_b32"):
                nb = {"ds_read_b32": 4, "ds_read_b64": 8, "ds_read_b96": 12, "ds_read_u16": 2, "ds_read_b128": 16,
                      "ds_read_u8": 1, "ds_bpermute_b32": 4}[op]
                off = 0
                for x in t[2:]:
                    if x.startswith("offset:"): off = int(x[7:], 0)
                pz = w.check_inflight_read(t[1])
                if pz: w.errors.append(("POISONED ADDRESS ds", w.cur))
                a, ka = w.vget(t[1]); act = w.act()
                r = w.vreg(t[0])
                if op == "ds_bpermute_b32":
                    d, kd = w.vget(t[2]); pzd = w.check_inflight_read(t[2])
                    src = ((a + np.uint64(off)) >> np.uint64(2)) % np.uint64(64)
                    val = np.array([d[int(x)] for x in src], dtype=np.uint64); kn = np.array([kd[int(x)] for x in src]) & ka
                    w.cur_poison = pzd or pz
                    w.vset(t[0], val, kn); continue
                vals = np.zeros(NL, dtype=object); kn = np.zeros(NL, dtype=bool)
                for l in range(NL):
                    if not act[l] or not ka[l]: continue
                    base = int(a[l]) + off
                    if base + nb > w.lds_size: w.errors.append(("ds_read beyond LDS", base, w.cur))
                    v = 0; k = True
                    for b in range(nb):
                        e = w.lds.get(base + b)
                        if e is None: k = False; break
                        v |= e[0] << (8 * b); k &= e[1]
                    vals[l] = v; kn[l] = k
                w.cur_poison = pz
                for j, i in enumerate(r):
                    part = np.array([(int(vals[l]) >> (32 * j)) & M32 for l in range(NL)], dtype=np.uint64)
                    w.v[i] = np.where(act, part, w.v[i]); w.vk[i] = np.where(act, kn, w.vk[i])
                    for q in w.vmq:
                        if i in q[0]: q[1].add(i)
                    w.poison[i] = pz
                continue
            if op.startswith("ds_"):
                if w.check_inflight_read(t[1]): w.errors.append(("POISONED ADDRESS ds", w.cur))
                pz = any(w.check_inflight_read(x) for x in t[2:])
            else:
                pz = any(w.check_inflight_read(x) for x in t[1:])
                if pz and op.startswith("v_mfma"): w.errors.append(("STALE DATA mfma", w.cur))
            w.cur_poison = pz
            r = w.vreg(t[0])
            act = w.act()
            for i in r:
                w.vk[i] = np.where(act, False, w.vk[i])
                for q in w.vmq:
                    if i in q[0]: q[1].add(i)
                w.poison[i] = pz
            continue
        if op.startswith("v_"):
            w.cur_poison = any(w.check_inflight_read(x) for x in t[1:])
            vop(w, op, t)
            if op.startswith("v_readfirstlane") or op.startswith("v_readlane"):
                for i in (w.sreg(t[0]) or []): w.spoison[i] = w.cur_poison  # (vcc_lo, m0: not tracked)
            if op.startswith("v_cmp") and not op.endswith("_e32") and w.sreg(t[0]):
                w.cur_poison = any(w.check_inflight_read(x) for x in t[1:])
                for i in w.sreg(t[0]): w.spoison[i] = w.cur_poison
            continue
        raise NotImplementedError(s)

def sop(w, op, t):
    g = lambda x, n=1: w.sget(x, n)
    if op in ("s_mov_b32", "s_movk_i32"): w.sset(t[0], g(t[1])); return
    if op == "s_mov_b64": w.sset(t[0], g(t[1], 2) if not t[1].lstrip("-").isdigit() else int(t[1]) & 0xFFFFFFFFFFFFFFFF, 2); return
    if op == "s_add_i32": w.sset(t[0], (g(t[1]) + g(t[2])) & M32); return
    if op == "s_addk_i32": w.sset(t[0], (g(t[0]) + (int(t[1], 0) if int(t[1], 0) < 0x8000 else int(t[1], 0) - 0x10000)) & M32); return
    if op == "s_mulk_i32": w.sset(t[0], (g(t[0]) * int(t[1], 0)) & M32); return
    if op == "s_sub_i32": w.sset(t[0], (g(t[1]) - g(t[2])) & M32); return
    if op == "s_add_u32":
        r = g(t[1]) + g(t[2]); w.sset(t[0], r & M32); w.scc = int(r > M32); return
    if op == "s_addc_u32":
        r = g(t[1]) + g(t[2]) + w.scc; w.sset(t[0], r & M32); w.scc = int(r > M32); return
    if op == "s_sub_u32":
        r = g(t[1]) - g(t[2]); w.sset(t[0], r & M32); w.scc = int(r < 0); return
    if op == "s_subb_u32":
        r = g(t[1]) - g(t[2]) - w.scc; w.sset(t[0], r & M32); w.scc = int(r < 0); return
    if op == "s_mul_i32": w.sset(t[0], (signed32(g(t[1])) * signed32(g(t[2]))) & M32); return
    if op == "s_mul_hi_u32": w.sset(t[0], (g(t[1]) * g(t[2])) >> 32); return
    if op == "s_mul_hi_i32": w.sset(t[0], ((signed32(g(t[1])) * signed32(g(t[2]))) >> 32) & M32); return
    if op == "s_lshl_b32": w.sset(t[0], (g(t[1]) << (g(t[2]) & 31)) & M32); w.scc = int(w.s[w.sreg(t[0])[0]] != 0); return
    if op == "s_lshr_b32": w.sset(t[0], g(t[1]) >> (g(t[2]) & 31)); w.scc = int(w.s[w.sreg(t[0])[0]] != 0); return
    if op == "s_ashr_i32": w.sset(t[0], (signed32(g(t[1])) >> (g(t[2]) & 31)) & M32); return
    if op == "s_lshl_b64": w.sset(t[0], (g(t[1], 2) << (g(t[2]) & 63)) & 0xFFFFFFFFFFFFFFFF, 2); return
    if op == "s_lshr_b64": w.sset(t[0], g(t[1], 2) >> (g(t[2]) & 63), 2); return
    if op == "s_ashr_i64": w.sset(t[0], (signed64(g(t[1], 2)) >> (g(t[2]) & 63)) & 0xFFFFFFFFFFFFFFFF, 2); return
    if op == "s_and_b32": r = g(t[1]) & g(t[2]); w.sset(t[0], r); w.scc = int(r != 0); return
    if op == "s_or_b32": r = g(t[1]) | g(t[2]); w.sset(t[0], r); w.scc = int(r != 0); return
    if op == "s_andn2_b32": r = g(t[1]) & ~g(t[2]) & M32; w.sset(t[0], r); w.scc = int(r != 0); return
    if op == "s_orn2_b32": r = (g(t[1]) | ~g(t[2])) & M32; w.sset(t[0], r); w.scc = int(r != 0); return
    if op == "s_xor_b32": r = g(t[1]) ^ g(t[2]); w.sset(t[0], r); w.scc = int(r != 0); return
    if op == "s_not_b32": r = (~g(t[1])) & M32; w.sset(t[0], r); w.scc = int(r != 0); return
    if op == "s_and_b64": r = g(t[1], 2) & g(t[2], 2); w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_or_b64": r = g(t[1], 2) | g(t[2], 2); w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_xor_b64": r = (g(t[1], 2) ^ g(t[2], 2)) & 0xFFFFFFFFFFFFFFFF; w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_nor_b64": r = ~(g(t[1], 2) | g(t[2], 2)) & 0xFFFFFFFFFFFFFFFF; w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_nand_b64": r = ~(g(t[1], 2) & g(t[2], 2)) & 0xFFFFFFFFFFFFFFFF; w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_xnor_b64": r = ~(g(t[1], 2) ^ g(t[2], 2)) & 0xFFFFFFFFFFFFFFFF; w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_not_b64": r = ~g(t[1], 2) & 0xFFFFFFFFFFFFFFFF; w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_andn2_b64": r = g(t[1], 2) & ~g(t[2], 2) & 0xFFFFFFFFFFFFFFFF; w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_orn2_b64": r = (g(t[1], 2) | ~g(t[2], 2)) & 0xFFFFFFFFFFFFFFFF; w.sset(t[0], r, 2); w.scc = int(r != 0); return
    if op == "s_and_saveexec_b64":
        src, old = g(t[1], 2), w.exec; w.sset(t[0], old, 2); w.exec = old & src; w.scc = int(w.exec != 0); return
    if op == "s_andn2_saveexec_b64":
        src, old = g(t[1], 2), w.exec; w.sset(t[0], old, 2); w.exec = src & ~old & 0xFFFFFFFFFFFFFFFF; w.scc = int(w.exec != 0); return
    if op == "s_or_saveexec_b64":
        src, old = g(t[1], 2), w.exec; w.sset(t[0], old, 2); w.exec = src | old; w.scc = int(w.exec != 0); return
    if op == "s_brev_b32": w.sset(t[0], int(f"{g(t[1]) & M32:032b}"[::-1], 2)); return
    if op == "s_abs_i32": r = abs(signed32(g(t[1]))) & M32; w.sset(t[0], r); w.scc = int(r != 0); return
    if op in ("s_min_i32", "s_max_i32"):
        a, b = signed32(g(t[1])), signed32(g(t[2])); r = min(a, b) if op == "s_min_i32" else max(a, b)
        w.sset(t[0], r & M32); w.scc = int(r == a); return
    if op in ("s_min_u32", "s_max_u32"):
        a, b = g(t[1]), g(t[2]); r = min(a, b) if op == "s_min_u32" else max(a, b); w.sset(t[0], r); return
    if op.startswith("s_cmpk_"):  # 16-bit immediate: sign-extended for _i32, zero-extended for _u32
        kind = op[7:]
        a, b = g(t[0]), int(t[1], 0) & 0xFFFF
        if kind.endswith("i32"): a, b = signed32(a), (b - 0x10000 if b & 0x8000 else b)
        w.scc = int({"eq": a == b, "lg": a != b, "lt": a < b, "le": a <= b, "gt": a > b, "ge": a >= b}[kind[:2]]); return
    if op.startswith("s_cmp_"):
        kind = op[6:]
        a, b = g(t[0]), g(t[1])
        if kind.endswith("i32"): a, b = signed32(a), signed32(b)
        c = kind[:2]
        w.scc = int({"eq": a == b, "lg": a != b, "lt": a < b, "le": a <= b, "gt": a > b, "ge": a >= b}[c]); return
    if op == "s_cselect_b32": w.sset(t[0], g(t[1]) if w.scc else g(t[2])); return
    if op == "s_cselect_b64":
        a = g(t[1], 2) if not t[1].lstrip("-").isdigit() else int(t[1]) & 0xFFFFFFFFFFFFFFFF
        b = g(t[2], 2) if not t[2].lstrip("-").isdigit() else int(t[2]) & 0xFFFFFFFFFFFFFFFF
        w.sset(t[0], a if w.scc else b, 2); return
    if op == "s_bfe_u32":
        v = g(t[2]); off, wd = v & 31, (v >> 16) & 127; w.sset(t[0], (g(t[1]) >> off) & ((1 << wd) - 1)); return
    if op in ("s_bcnt1_i32_b64", "s_bcnt1_i32_b32"):
        r = bin(g(t[1], 2 if op.endswith("b64") else 1)).count("1"); w.sset(t[0], r); w.scc = int(r != 0); return
    if op in ("s_ff1_i32_b64", "s_ff1_i32_b32"):
        v = g(t[1], 2 if op.endswith("b64") else 1)
        w.sset(t[0], (v & -v).bit_length() - 1 if v else M32); return
    if op == "s_getreg_b32": w.sset(t[0], 0); return
    if op == "s_getpc_b64": w.sset(t[0], 0, 2); return
    raise NotImplementedError(op + " " + " ".join(t))

def gaddr(w, vaddr, saddr):
    """Per-lane address of a global memory instruction: a 64-bit vector
    address (saddr "off"), or a scalar base plus a 32-bit vector offset."""
    if saddr == "off":
        return w.vget(vaddr, 2)
    vo, kn = w.vget(vaddr)
    try:
        sb = w.sget(saddr, 2)
    except Unknown:
        return np.zeros(NL, dtype=np.uint64), np.zeros(NL, dtype=bool)
    return np.array([(int(sb) + int(x)) & 0xFFFFFFFFFFFFFFFF for x in vo], dtype=np.uint64), kn

def vop(w, op, t):
    U = np.uint64; MM = U(M32)
    g = lambda x, n=1: w.vget(x, n)
    act = w.act()
    def setv(val, kn, dst=None): w.vset(dst or t[0], val & U(0xFFFFFFFFFFFFFFFF), kn)
    base = op.replace("_e32", "").replace("_e64", "").replace("_sdwa", "")
    def s32(a): return np.where(a & U(0x80000000), a.astype(np.int64) - (1 << 32), a.astype(np.int64))
    if base in ("v_mov_b32",): a, k = g(t[1]); setv(a & MM, k); return
    if base == "v_mov_b64": a, k = g(t[1], 2); setv(a, k); return
    if base in ("v_add_u32", "v_sub_u32", "v_subrev_u32"):
        a, ka = g(t[1]); b, kb = g(t[2])
        r = (a + b) if base == "v_add_u32" else ((a - b) if base == "v_sub_u32" else (b - a))
        setv(r & MM, ka & kb); return
    if base in ("v_add_co_u32", "v_sub_co_u32", "v_subrev_co_u32"):
        # dst, carry(sdst or vcc), a, b
        if op.endswith("_e32"):
            cdst = "vcc"
            a_, b_ = (t[2], t[3]) if len(t) > 3 and t[1] == "vcc" else (t[1], t[2])
        else: cdst, a_, b_ = t[1], t[2], t[3]
        a, ka = g(a_); b, kb = g(b_)
        ai, bi = a.astype(object), b.astype(object)
        if base == "v_add_co_u32": r = [int(x) + int(y) for x, y in zip(a, b)]; c = [int(v > M32) for v in r]
        elif base == "v_sub_co_u32": r = [int(x) - int(y) for x, y in zip(a, b)]; c = [int(v < 0) for v in r]
        else: r = [int(y) - int(x) for x, y in zip(a, b)]; c = [int(v < 0) for v in r]
        setv(np.array([v & M32 for v in r], dtype=U), ka & kb)
        m = 0
        for l in range(NL):
            if act[l] and c[l]: m |= 1 << l
        w.sset(cdst, m, 2); return
    if base in ("v_addc_co_u32", "v_subb_co_u32"):
        # dst, carry out, a, b, carry in
        a, ka = g(t[2]); b, kb = g(t[3]); cin = w.sget(t[4], 2)
        m = 0; out = []
        for l in range(NL):
            ci = (cin >> l) & 1
            v = int(a[l]) + int(b[l]) + ci if base == "v_addc_co_u32" else int(a[l]) - int(b[l]) - ci
            out.append(v & M32)
            if act[l] and (v > M32 or v < 0): m |= 1 << l
        setv(np.array(out, dtype=U), ka & kb); w.sset(t[1], m, 2); return
    if base == "v_lshl_add_u64":
        a, ka = g(t[1], 2); sh = int(t[2], 0) if t[2].isdigit() else None
        if sh is None: shv, ks = g(t[2]); sh = int(shv[0])
        b, kb = g(t[3], 2)
        setv(((a << U(sh)) + b) & U(0xFFFFFFFFFFFFFFFF), ka & kb); return
    if base == "v_mad_u64_u32":
        a, ka = g(t[2]); b, kb = g(t[3]); c, kc = g(t[4], 2)
        r = np.array([(int(x) * int(y) + int(z)) & 0xFFFFFFFFFFFFFFFF for x, y, z in zip(a, b, c)], dtype=U)
        setv(r, ka & kb & kc); w.sset(t[1], 0, 2); return
    if base == "v_mad_i64_i32":
        a, ka = g(t[2]); b, kb = g(t[3]); c, kc = g(t[4], 2)
        r = np.array([(signed32(int(x)) * signed32(int(y)) + signed64(int(z))) & 0xFFFFFFFFFFFFFFFF for x, y, z in zip(a, b, c)], dtype=U)
        setv(r, ka & kb & kc); w.sset(t[1], 0, 2); return
    if base in ("v_lshlrev_b64", "v_lshrrev_b64"):
        a, ka = g(t[1]); b, kb = g(t[2], 2); sh = a & U(63)
        r = (b << sh) if base == "v_lshlrev_b64" else (b >> sh)
        setv(r & U(0xFFFFFFFFFFFFFFFF), ka & kb); return
    if base in ("v_lshlrev_b32", "v_lshrrev_b32", "v_ashrrev_i32"):
        a, ka = g(t[1]); b, kb = g(t[2]); sh = a & U(31)
        if base == "v_lshlrev_b32": r = (b << sh) & MM
        elif base == "v_lshrrev_b32": r = b >> sh
        else: r = (s32(b) >> sh.astype(np.int64)).astype(np.int64) & M32; r = r.astype(U)
        setv(r, ka & kb); return
    if base in ("v_and_b32", "v_or_b32", "v_xor_b32"):
        a, ka = g(t[1]); b, kb = g(t[2])
        r = {"v_and_b32": a & b, "v_or_b32": a | b, "v_xor_b32": a ^ b}[base]; setv(r & MM, ka & kb); return
    if base in ("v_and_or_b32", "v_lshl_or_b32", "v_lshl_add_u32", "v_add_lshl_u32", "v_or3_b32", "v_add3_u32"):
        a, ka = g(t[1]); b, kb = g(t[2]); c, kc = g(t[3])
        if base == "v_and_or_b32": r = (a & b) | c
        elif base == "v_lshl_or_b32": r = ((a << (b & U(31))) & MM) | c
        elif base == "v_lshl_add_u32": r = ((a << (b & U(31))) + c) & MM
        elif base == "v_add_lshl_u32": r = (((a + b) & MM) << (c & U(31))) & MM
        elif base == "v_or3_b32": r = a | b | c
        else: r = (a + b + c) & MM
        setv(r & MM, ka & kb & kc); return
    if base == "v_bitop3_b32":
        a, ka = g(t[1]); b, kb = g(t[2]); c, kc = g(t[3])
        lut = int([x for x in t if x.startswith("bitop3:")][0][7:], 0)
        r = np.zeros(NL, dtype=U)
        for bit in range(32):
            ab = (a >> U(bit)) & U(1); bb = (b >> U(bit)) & U(1); cb = (c >> U(bit)) & U(1)
            idx = (ab << U(2)) | (bb << U(1)) | cb
            r |= ((U(lut) >> idx) & U(1)) << U(bit)
        setv(r, ka & kb & kc); return
    if base == "v_bfe_u32":
        a, ka = g(t[1]); o, ko = g(t[2]); wd, kw = g(t[3])
        r = (a >> (o & U(31))) & ((U(1) << (wd & U(31))) - U(1)); setv(r, ka & ko & kw); return
    if base == "v_bfrev_b32":
        a, ka = g(t[1]); r = np.array([int(f"{int(x):032b}"[::-1], 2) for x in a], dtype=U); setv(r, ka); return
    if base == "v_mad_u32_u24":
        a, ka = g(t[1]); b, kb = g(t[2]); c, kc = g(t[3])
        setv(((a & U(0xFFFFFF)) * (b & U(0xFFFFFF)) + c) & MM, ka & kb & kc); return
    if base in ("v_mul_lo_u32", "v_mul_u32_u24", "v_mul_hi_u32"):
        a, ka = g(t[1]); b, kb = g(t[2])
        if base == "v_mul_u32_u24": r = ((a & U(0xFFFFFF)) * (b & U(0xFFFFFF))) & MM
        elif base == "v_mul_lo_u32": r = np.array([(int(x) * int(y)) & M32 for x, y in zip(a, b)], dtype=U)
        else: r = np.array([(int(x) * int(y)) >> 32 for x, y in zip(a, b)], dtype=U)
        setv(r, ka & kb); return
    if base in ("v_min_i32", "v_max_i32", "v_min_u32", "v_max_u32"):
        a, ka = g(t[1]); b, kb = g(t[2])
        if base.endswith("i32"): a2, b2 = s32(a), s32(b)
        else: a2, b2 = a.astype(np.int64), b.astype(np.int64)
        r = np.minimum(a2, b2) if "min" in base else np.maximum(a2, b2)
        setv((r & M32).astype(U), ka & kb); return
    if base == "v_cndmask_b32":
        if op.endswith("_e32"): a, ka = g(t[1]); b, kb = g(t[2]); m = w.vcc
        else: a, ka = g(t[1]); b, kb = g(t[2]); m = w.sget(t[3], 2)
        sel = np.array([(m >> l) & 1 for l in range(NL)], dtype=bool)
        setv(np.where(sel, b, a) & MM, np.where(sel, kb, ka)); return
    if base.startswith("v_cmp_") and not re.search(r"_(f32|f16|bf16)$", base):
        kind = base[6:]
        c, ty = kind.split("_")
        if op.endswith("_e32"):
            dst = "vcc"
            a_, b_ = (t[1], t[2]) if t[0] == "vcc" else (t[0], t[1])
        else: dst, a_, b_ = t[0], t[1], t[2]
        a, ka = g(a_); b, kb = g(b_)
        if ty == "i32": a2, b2 = s32(a), s32(b)
        else: a2, b2 = a.astype(np.int64), b.astype(np.int64)
        r = {"eq": a2 == b2, "ne": a2 != b2, "lt": a2 < b2, "le": a2 <= b2, "gt": a2 > b2, "ge": a2 >= b2}[c]
        if not (ka & kb)[act].all(): raise Unknown("cmp on unknown")
        w.sset(dst, w.mask_from(r & act), 2); return
    if base == "v_writelane_b32":  # one lane, whatever exec (SGPR spill slots)
        r = w.vreg(t[0])[0]
        lane = int(w.sget(t[2])) & (NL - 1)
        try:
            val, known = w.sget(t[1]), True
        except Unknown:
            val, known = 0, False
        w.v[r][lane] = U(val & M32); w.vk[r][lane] = known
        w.poison[r] = w.poison[r] or w.cur_poison
        return
    if base == "v_readlane_b32":
        a, ka = g(t[1])
        lane = int(w.sget(t[2])) & (NL - 1)
        w.sset(t[0], int(a[lane]) & M32, known=bool(ka[lane])); return
    if base == "v_readfirstlane_b32":
        a, ka = g(t[1])
        lanes = [l for l in range(NL) if act[l]]
        l0 = lanes[0] if lanes else 0
        w.sset(t[0], int(a[l0]) & M32, known=bool(ka[l0])); return
    if base == "v_mbcnt_lo_u32_b32":
        m, _ = g(t[1]); c, kc = g(t[2])
        r = np.array([bin(int(m[l]) & ((1 << min(l, 32)) - 1)).count("1") for l in range(NL)], dtype=U) + c
        setv(r & MM, kc); return
    if base == "v_mbcnt_hi_u32_b32":
        m, _ = g(t[1]); c, kc = g(t[2])
        r = np.array([bin(int(m[l]) & ((1 << max(l - 32, 0)) - 1)).count("1") for l in range(NL)], dtype=U) + c
        setv(r & MM, kc); return
    if base == "v_cvt_f32_u32":
        a, ka = g(t[1]); r = np.array([f2u(float(np.float32(int(x)))) for x in a], dtype=U); setv(r, ka); return
    if base == "v_rcp_iflag_f32":
        a, ka = g(t[1])
        with np.errstate(all="ignore"):  # lanes of unknown value may hold any bits
            r = np.array([f2u(float(np.float32(1.0) / np.frombuffer(struct.pack('<I', int(x)), np.float32)[0])) if int(x) else 0x7f800000 for x in a], dtype=U)
        setv(r, ka); return
    if base == "v_mul_f32":
        a, ka = g(t[1]); b, kb = g(t[2])
        fa = np.array([np.frombuffer(struct.pack('<I', int(x) & M32), np.float32)[0] for x in a], dtype=np.float32)
        fb = np.array([np.frombuffer(struct.pack('<I', int(x) & M32), np.float32)[0] for x in b], dtype=np.float32)
        with np.errstate(all="ignore"):
            r = np.array([f2u(float(x)) for x in (fa * fb)], dtype=U)
        setv(r, ka & kb); return
    if base == "v_cvt_u32_f32":
        a, ka = g(t[1])
        fa = [np.frombuffer(struct.pack('<I', int(x) & M32), np.float32)[0] for x in a]
        r = np.array([min(max(int(x), 0), M32) if np.isfinite(x) else M32 for x in fa], dtype=U); setv(r, ka); return
    # data ops: result unknown
    if base in ("v_add_f16", "v_cvt_pk_f16_f32", "v_add_f32", "v_fma_f32", "v_cvt_f16_f32", "v_mul_f16", "v_sub_f16",
                "v_pk_add_f16", "v_pk_mul_f16", "v_pk_fma_f16", "v_accvgpr_read_b32", "v_accvgpr_write_b32", "v_exp_f32",
                "v_max_f32", "v_min_f32", "v_cvt_f32_f16", "v_perm_b32", "v_pack_b32_f16", "v_fmac_f32", "v_sub_f32",
                "v_cvt_pk_bf16_f32", "v_div_scale_f32", "v_rcp_f32", "v_fma_mix_f32", "v_fma_mixlo_f16",
                "v_fma_mixhi_f16", "v_pk_mul_f32", "v_pk_add_f32", "v_pk_fma_f32"):
        r = w.vreg(t[0])
        for i in r:
            w.vk[i] = np.where(act, False, w.vk[i])
            for q in w.vmq:
                if i in q[0]: q[1].add(i)
            w.poison[i] = w.cur_poison
        return
    # other floating-point data ops (the activation epilogues): result unknown;
    # a float compare only selects data (v_cndmask), never a branch or address
    if re.search(r"_(f32|f16|bf16)$", base) or re.search(r"_(f32|f16)_", base):
        if base.startswith("v_cmp"):
            dst = "vcc" if t[0] == "vcc" or op.endswith("_e32") else t[0]
            w.sset(dst, 0, 2); return
        r = w.vreg(t[0])
        for i in r:
            w.vk[i] = np.where(act, False, w.vk[i])
            for q in w.vmq:
                if i in q[0]: q[1].add(i)
            w.poison[i] = w.cur_poison
        return
    raise NotImplementedError(op + " " + " ".join(t))

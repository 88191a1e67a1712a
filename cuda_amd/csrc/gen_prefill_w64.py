#!/usr/bin/env python3
"""Generator of the 64-row prefill kernel body: hand-scheduled gfx950 assembly.

The 16-bit head-dim-128 prefill (`prefill_w64.hip`) runs one wave per SIMD,
64 query rows per wave. In the steady state each iteration issues 64
v_mfma_f32_32x32x16_bf16 (PV of the previous key tile, QK of the next) and
between them the whole softmax of the current tile, so the wave's own MFMAs
hide its VALU work, and every K/V fragment read from LDS feeds two MFMAs.
That walk needs O^T and Q in AGPRs and S^T, P in VGPRs with no copies; the
register assignment is fixed here, by hand, and the instruction order with it.

The same run writes an fp16 body beside the bf16 one (`configure_f16`):
v_mfma_f32_32x32x16_f16, v_cvt_pk_f16_f32 for P, and a redo bound of 2^15
on a tile sum so that no weight passes fp16's 65504.

With --mx it writes the MXFP8 form of the same walk (`prefill_w64_mx.hip`):
QK on v_mfma_scale_f32_32x32x64_f8f6f4 (16 passes, e4m3 codes with per-lane
e8m0 scale bytes picked by op_sel), K and V^T fragments in one AGPR ring,
K scale words travelling in the K ring slot, and row sums over the
bf16-rounded weights; `configure(mx)` rebinds the register map.

This script writes the kernel body as one string-literal macro per variant
(causal, non-causal; bf16 and fp16) for an inline-asm statement, plus the
clobber list. It
also checks its own output before writing it:

* hazards: a forward dataflow over the body's control-flow graph tracks, for
  every register, the wait states since its last MFMA / VALU / transcendental
  / permlane write and since MFMA reads of it, and rejects any instruction
  closer than the gfx950 requirement (taken conservatively: the 16-pass
  figures of the MFMA tables, which are longer than what the 8-pass
  32x32x16 needs);
* counters: the LDS and vector-memory operations in flight are tracked in
  order, and a use of a register whose load has not been waited on by an
  s_waitcnt is rejected; at a control-flow join the in-flight lists of all
  predecessors must agree;
* SCC: every SCC reader's producer is the instruction it was written for;
* schedule: every placed instruction reads each register from the same
  writer as in program order.

Usage: gen_prefill_w64.py [--mx] OUT.inc
"""
import sys

# ---------------------------------------------------------------------------
# operands
# ---------------------------------------------------------------------------


class Reg:
    """Contiguous register range: file 'v', 'a' or 's', first index, count."""

    __slots__ = ("f", "i", "n")

    def __init__(self, f, i, n=1):
        self.f, self.i, self.n = f, i, n

    def __str__(self):
        return f"{self.f}{self.i}" if self.n == 1 else f"{self.f}[{self.i}:{self.i + self.n - 1}]"

    def __getitem__(self, k):
        assert 0 <= k < self.n, (self, k)
        return Reg(self.f, self.i + k)

    def sl(self, k, n):
        assert 0 <= k and k + n <= self.n, (self, k, n)
        return Reg(self.f, self.i + k, n)

    def keys(self):
        return [(self.f, self.i + j) for j in range(self.n)]


class Sym:
    """An operand of the inline-asm statement (a compiler-placed register)."""

    def __init__(self, name):
        self.name = name

    def __str__(self):
        return "%[" + self.name + "]"

    def keys(self):
        return [("in", self.name)]


class Spec:
    """vcc, m0, scc."""

    def __init__(self, name):
        self.name = name

    def __str__(self):
        return self.name

    def keys(self):
        return [("x", self.name)]


VCC, M0 = Spec("vcc"), Spec("m0")


def _keys(x):
    return x.keys() if hasattr(x, "keys") and not isinstance(x, dict) else []


def _txt(x):
    if isinstance(x, int):
        return hex(x) if (x < -16 or x > 64) else str(x)
    return str(x)


# ---------------------------------------------------------------------------
# instructions
# ---------------------------------------------------------------------------


class Ins:
    __slots__ = ("kind", "text", "defs", "uses", "ws", "mdst", "mc", "mab", "mem", "wvm", "wlgkm",
                 "target", "cond", "trans", "perm", "dot", "m0use", "std", "cost", "frag")

    def __init__(self, kind, text, defs=(), uses=(), **kw):
        self.kind = kind
        self.text = text
        self.defs = [k for r in defs for k in _keys(r)]
        self.uses = [k for r in uses for k in _keys(r)]
        self.ws = kw.get("ws", 1)
        self.mdst = kw.get("mdst")
        self.mc = kw.get("mc")
        self.mab = kw.get("mab", [])
        self.mem = kw.get("mem")        # 'lgkm' or 'vm'
        self.wvm = kw.get("wvm")
        self.wlgkm = kw.get("wlgkm")
        self.target = kw.get("target")
        self.cond = kw.get("cond", False)
        self.trans = kw.get("trans", False)
        self.perm = kw.get("perm", False)
        self.dot = kw.get("dot", False)
        self.m0use = kw.get("m0use", False)
        self.std = kw.get("std", [])
        self.cost = kw.get("cost", 0)
        self.frag = None


def MFMA(d, a, b, c, op=None):
    op = op or MFMA_OP
    uses = [a, b] + ([c] if c is not None else [])
    return Ins("mfma", f"{op} {d}, {a}, {b}, {c if c is not None else 0}", defs=[d], uses=uses,
               mdst=tuple(d.keys()), mc=tuple(c.keys()) if c is not None else None,
               mab=a.keys() + b.keys())


def V(op, d, *s, trans=False, perm=False):
    """VALU instruction; d may be a Reg, VCC or an SGPR pair (v_cmp)."""
    ops = ", ".join(_txt(x) for x in ([d] if d is not None else []) + list(s))
    defs = [d] if d is not None else []
    uses = list(s)
    if perm:
        uses = uses + [d]
        defs = defs + list(s)
    return Ins("valu", f"{op} {ops}", defs=defs, uses=uses, trans=trans, perm=perm,
               dot=op.startswith("v_dot2"), cost=12 if trans else 6)


def ACCR(d, a):
    return Ins("valu", f"v_accvgpr_read_b32 {d}, {a}", defs=[d], uses=[a], cost=6)


def ACCW(a, s):
    return Ins("valu", f"v_accvgpr_write_b32 {a}, {_txt(s)}", defs=[a], uses=[s], cost=6)


def S(op, d, *s, scc_def=True):
    ops = ", ".join(_txt(x) for x in ([d] if d is not None else []) + list(s))
    return Ins("salu", f"{op} {ops}", defs=[d] if d is not None else [], uses=list(s), cost=2)


def SLOAD(op, d, base, off):
    return Ins("smem", f"{op} {d}, {base}, {_txt(off)}", defs=[d], uses=[base], mem="lgkm", cost=2)


def DSR(op, d, addr, off=0):
    t = f"{op} {d}, {addr}" + (f" offset:{off}" if off else "")
    return Ins("lds", t, defs=[d], uses=[addr], mem="lgkm", cost=4)


def DSW(op, addr, data, off=0):
    t = f"{op} {addr}, {data}" + (f" offset:{off}" if off else "")
    return Ins("lds", t, defs=[], uses=[addr, data], mem="lgkm", cost=4)


def BLOAD(op, d, voff, rsrc, off=0):
    t = f"{op} {d}, {voff}, {rsrc}, 0 offen" + (f" offset:{off}" if off else "")
    return Ins("vmem", t, defs=[d], uses=[voff, rsrc], mem="vm", cost=4)


def BLOAD_LDS(voff, rsrc, off=0):
    """16 bytes per lane into LDS at M0 + off + 16 lane; the instruction
    offset adds to the global address as well."""
    t = f"buffer_load_dwordx4 {voff}, {rsrc}, 0 offen" + (f" offset:{off}" if off else "") + " lds"
    return Ins("vmem", t, defs=[], uses=[voff, rsrc, M0], mem="vm", m0use=True, cost=4)


def BLOAD_LDS_DW(voff, rsrc, off=0):
    """4 bytes per lane into LDS at M0 + off + 4 lane."""
    t = f"buffer_load_dword {voff}, {rsrc}, 0 offen" + (f" offset:{off}" if off else "") + " lds"
    return Ins("vmem", t, defs=[], uses=[voff, rsrc, M0], mem="vm", m0use=True, cost=4)


def GLOAD(op, d, voff, base, off=0):
    """Global load at base (64-bit SGPR pair) + voff (32-bit VGPR offset)."""
    t = f"{op} {d}, {voff}, {base}" + (f" offset:{off}" if off else "")
    return Ins("vmem", t, defs=[d], uses=[voff, base], mem="vm", cost=4)


def BSTORE(op, data, voff, rsrc, off=0):
    t = f"{op} {data}, {voff}, {rsrc}, 0 offen" + (f" offset:{off}" if off else "")
    return Ins("vmem", t, defs=[], uses=[data, voff, rsrc], mem="vm", std=data.keys(), cost=4)


def WAIT(vm=None, lgkm=None):
    parts = []
    if vm is not None:
        parts.append(f"vmcnt({vm})")
    if lgkm is not None:
        parts.append(f"lgkmcnt({lgkm})")
    return Ins("wait", "s_waitcnt " + " ".join(parts), wvm=vm, wlgkm=lgkm, cost=1)


def NOP(n):
    assert 0 <= n <= 7
    return Ins("nop", f"s_nop {n}", ws=n + 1, cost=n + 1)


def NOPS(n):
    """n wait states of s_nop."""
    out = []
    while n > 0:
        k = min(n, 8)
        out.append(NOP(k - 1))
        n -= k
    return out


def BAR():
    return Ins("barrier", "s_barrier", cost=1)


def LABEL(name):
    return Ins("label", f"{name}:", ws=0)


def BR(target):
    return Ins("br", f"s_branch {target}", target=target, cost=1)


def CBR(op, target):
    return Ins("br", f"{op} {target}", target=target, cond=True, cost=1)


# ---------------------------------------------------------------------------
# hazard and counter checker
# ---------------------------------------------------------------------------

MFMA_WS = 20       # MFMA result -> any other read or write (16-pass figure + gfx950)
MFMA_SRCC_WAR = 18  # MFMA reads srcC -> VALU overwrites it
MFMA_AB_WAR = 1     # MFMA reads srcA/B at issue (only srcC has a listed WAR window)
VALU_TO_MFMA = 3    # VALU write -> MFMA read (2 required)
TRANS_FWD = 2       # transcendental result -> VALU read (1 required)
DOT_FWD = 3         # v_dot2 result -> read by any instruction but a v_dot2 accumulating it
                    # (measured: one instruction between reads the old value, two do not)
PERM_WS = 4         # around v_permlane32_swap (conservative)
VALU_SGPR_VMEM = 5  # VALU writes SGPR -> VMEM / SALU reads it
VALU_SGPR_VALU = 2  # VALU writes SGPR or VCC -> VALU reads it (v_cndmask mask)
M0_WS = 1           # SALU writes M0 -> LDS DMA
STORE_DATA = 2      # wide store data -> VALU overwrite
CAP = 32
# v_mfma_f32_32x32x16_bf16 takes 8 passes: an MFMA issues at least 8 wait
# states (32 cycles; measured 32.1 cycles apart back to back) after the one
# before it, so whatever preceded an MFMA is 8 wait states older by the next.
MFMA_ISSUE = 8


class CheckError(Exception):
    pass


def _is_vec(k):
    return k[0] in ("v", "a")


def check(prog, name):
    """Dataflow over `prog` (list of Ins); raises CheckError on a violation."""
    labels = {ins.text[:-1]: i for i, ins in enumerate(prog) if ins.kind == "label"}
    n = len(prog)
    succ = []
    for i, ins in enumerate(prog):
        s = []
        if ins.kind == "br":
            assert ins.target in labels, f"{name}: unknown label {ins.target}"
            s.append(labels[ins.target])
            if ins.cond and i + 1 < n:
                s.append(i + 1)
        elif i + 1 < n:
            s.append(i + 1)
        succ.append(s)

    # state: (dist dict, lgkm tuple, vm tuple); dist: (cat, key) -> (d, tag, dm),
    # dm: d at the last MFMA issue on the path (None: the entry is younger)
    instate = [None] * n
    instate[0] = ({}, (), ())
    work = [0]
    errors = []

    def merge(la, lb):
        """In-flight lists of two paths, aligned at their most recent end:
        entry j of the result holds the registers of entry j of either."""
        if la == lb:
            return la
        n_ = max(len(la), len(lb))
        out = []
        for j in range(1, n_ + 1):
            ea = la[-j] if j <= len(la) else frozenset()
            eb = lb[-j] if j <= len(lb) else frozenset()
            out.append(ea | eb)
        return tuple(reversed(out))

    def join(a, b, where):
        if a is None:
            return b
        da, la, va = a
        db, lb, vb = b
        la, va = merge(la, lb), merge(va, vb)
        d = dict(da)
        for k, (dist, tag, dm) in db.items():
            if k in d:
                d0, t0, m0 = d[k]
                d[k] = (min(d0, dist), t0 if t0 == tag else None, None if m0 is None or dm is None else min(m0, dm))
            else:
                d[k] = (dist, tag, dm)
        return (d, la, va)

    def err(i, msg):
        errors.append(f"{name}: #{i} `{prog[i].text}`: {msg}")

    def transfer(i, st):
        ins = prog[i]
        dist, lg, vm = st
        g = dist.get

        def dd(cat, k):
            e = g((cat, k))
            return e[0] if e else CAP

        # --- counters: uses / defs of registers with loads in flight
        pend_l = set().union(*lg) if lg else set()
        pend_v = set().union(*vm) if vm else set()
        for k in set(ins.uses) | set(ins.defs):
            if k in pend_l:
                err(i, f"{k} has an LDS operation in flight")
            if k in pend_v:
                err(i, f"{k} has a vector-memory load in flight")
        # --- hazards
        if ins.kind == "mfma":
            for k in ins.uses:
                if dd("dw", k) < DOT_FWD:
                    err(i, f"reads {k} {dd('dw', k)} wait states after a v_dot2 wrote it")
            for k in ins.mab:
                if dd("mw", k) < MFMA_WS:
                    err(i, f"srcA/B {k} written by an MFMA {dd('mw', k)} wait states before")
                if dd("vw", k) < VALU_TO_MFMA:
                    err(i, f"srcA/B {k} written by VALU {dd('vw', k)} wait states before")
            for k in (ins.mc or ()):
                e = g(("mw", k))
                if e and e[0] < MFMA_WS and e[1] != ins.mdst:
                    err(i, f"srcC {k} written by a different MFMA {e[0]} wait states before")
                if dd("vw", k) < VALU_TO_MFMA:
                    err(i, f"srcC {k} written by VALU {dd('vw', k)} wait states before")
            for k in ins.mdst:
                e = g(("mw", k))
                if e and e[0] < MFMA_WS and e[1] != ins.mdst:
                    err(i, f"dst {k} written by a different MFMA {e[0]} wait states before")
                if dd("vw", k) < VALU_TO_MFMA:
                    err(i, f"dst {k} written by VALU {dd('vw', k)} wait states before")
        elif ins.kind in ("valu", "lds", "vmem"):
            for k in ins.uses:
                if _is_vec(k) and dd("mw", k) < MFMA_WS:
                    err(i, f"reads {k} {dd('mw', k)} wait states after an MFMA wrote it")
                if ins.kind == "valu" and not ins.trans and dd("tw", k) < TRANS_FWD:
                    err(i, f"reads {k} {dd('tw', k)} wait states after a transcendental wrote it")
                if dd("pw", k) < PERM_WS:
                    err(i, f"reads {k} {dd('pw', k)} wait states after a permlane wrote it")
                if not ins.dot and dd("dw", k) < DOT_FWD:
                    err(i, f"reads {k} {dd('dw', k)} wait states after a v_dot2 wrote it")
                if ins.perm and dd("vw", k) < PERM_WS:
                    err(i, f"permlane reads {k} {dd('vw', k)} wait states after a VALU write")
                if ins.kind in ("vmem", "lds") and k[0] == "s" and dd("vws", k) < VALU_SGPR_VMEM:
                    err(i, f"memory op reads {k} written by VALU {dd('vws', k)} wait states before")
                if ins.kind == "valu" and dd("vws", k) < VALU_SGPR_VALU:
                    err(i, f"VALU reads {k} written by VALU {dd('vws', k)} wait states before")
            for k in ins.defs:
                if not _is_vec(k):
                    continue
                if dd("mw", k) < MFMA_WS:
                    err(i, f"overwrites {k} {dd('mw', k)} wait states after an MFMA wrote it")
                if dd("mrc", k) < MFMA_SRCC_WAR:
                    err(i, f"overwrites {k} {dd('mrc', k)} wait states after an MFMA read it as srcC")
                if dd("mrab", k) < MFMA_AB_WAR:
                    err(i, f"overwrites {k} {dd('mrab', k)} wait states after an MFMA read it")
                if dd("std", k) < STORE_DATA:
                    err(i, f"overwrites {k} {dd('std', k)} wait states after a store read it")
            if ins.m0use and dd("sm0", ("x", "m0")) < M0_WS:
                err(i, "LDS DMA right after M0 was written")
        elif ins.kind in ("salu", "smem"):
            for k in ins.uses:
                if k[0] == "s" and dd("vws", k) < VALU_SGPR_VMEM:
                    err(i, f"scalar op reads {k} written by VALU {dd('vws', k)} wait states before")

        # --- advance distances
        w = ins.ws
        nd = {}
        mf = ins.kind == "mfma"
        for k, (d0, tag, dm) in dist.items():
            d1 = d0 + w
            if mf:
                if dm is not None:
                    d1 = max(d1, dm + MFMA_ISSUE)
                dm = d1
            if d1 < CAP:
                nd[k] = (d1, tag, dm)
        if mf:
            for k in ins.mdst:
                nd[("mw", k)] = (0, ins.mdst, 0)
            for k in (ins.mc or ()):
                nd[("mrc", k)] = (0, None, 0)
            for k in ins.mab:
                nd[("mrab", k)] = (0, None, 0)
        elif ins.kind == "valu":
            for k in ins.defs:
                nd[("vw", k)] = (0, None, None)
                nd.pop(("mw", k), None)   # later reads see this write (its WAW was checked)
                if ins.trans:
                    nd[("tw", k)] = (0, None, None)
                if ins.perm:
                    nd[("pw", k)] = (0, None, None)
                if ins.dot:
                    nd[("dw", k)] = (0, None, None)
                if k[0] == "s" or k == ("x", "vcc"):
                    nd[("vws", k)] = (0, None, None)
        elif ins.kind == "salu":
            for k in ins.defs:
                if k == ("x", "m0"):
                    nd[("sm0", k)] = (0, None, None)
        if ins.kind == "vmem" and ins.std:
            for k in ins.std:
                nd[("std", k)] = (0, None, None)
        # --- counters
        if ins.mem == "lgkm":
            lg = lg + (frozenset(ins.defs),)
        if ins.mem == "vm":
            vm = vm + (frozenset(ins.defs),)
        if ins.kind == "wait":
            if ins.wlgkm is not None:
                lg = lg[len(lg) - ins.wlgkm:] if ins.wlgkm < len(lg) else lg
                if ins.wlgkm == 0:
                    lg = ()
            if ins.wvm is not None:
                vm = vm[len(vm) - ins.wvm:] if ins.wvm < len(vm) else vm
                if ins.wvm == 0:
                    vm = ()
        if len(lg) > 15:
            # the counter holds 15: an older read could not be waited for exactly
            if any(lg[:len(lg) - 15]):
                err(i, "a read is more than 15 LDS operations deep (lgkmcnt saturates)")
            lg = lg[len(lg) - 15:]
        if len(vm) > 63:
            vm = vm[-63:]
        return (nd, lg, vm)

    iters = 0
    while work:
        iters += 1
        if iters > 200 * n:
            raise CheckError(f"{name}: checker did not converge")
        i = work.pop()
        errs0 = len(errors)
        out = transfer(i, instate[i])
        if len(errors) > errs0:
            raise CheckError("\n".join(errors))
        for s in succ[i]:
            new = join(instate[s], out, s)
            if new != instate[s]:
                instate[s] = new
                work.append(s)
    return True


# ---------------------------------------------------------------------------
# register map
# ---------------------------------------------------------------------------


def v(i, n=1):
    return Reg("v", i, n)


def a(i, n=1):
    return Reg("a", i, n)


def s(i, n=1):
    return Reg("s", i, n)


# VGPRs (v0..v239; v240..v255 hold the compiler-placed per-lane inputs)
SACC = [[[v(64 * p + 32 * mb + 16 * nb, 16) for nb in range(2)] for mb in range(2)] for p in range(2)]
PB = [[v(128 + 8 * kk + 4 * nb, 4) for nb in range(2)] for kk in range(4)]
TMP = [v(160 + 8 * t, 8) for t in range(3)]
# K / V^T fragments read from LDS: NSLOT slots, each read LOOK fragments (2 LOOK
# MFMAs) ahead of its first use; slots 4-7 share v224-v239 with SCR, which the
# steady walk does not use (the output, the first tile's max and the redo path
# keep their temporaries elsewhere while fragments are in flight).
NSLOT, LOOK = 8, 6
STEADY_SPAN = 55   # the steady softmax spreads its 64 elements over gaps 0..STEADY_SPAN
LDS_SLOTS = 1      # issue slots the slot scheduler charges for an LDS read
# slot caps of the other iterations slot_schedule places (measured per tile
# of C2: fill 1500 cycles at 5, last 2611 and drain at 10; the first tile's
# iteration is faster under the greedy schedule, 2315 against 2386)
OTHER_CAP = {"fill": 5, "last": 10, "drain": 10}
GAP_CAP = 5        # issue slots per MFMA gap (5 measured best: 2220 cycles per steady iteration, 7 gave 2307)
FRAG = [v(184 + 4 * t, 4) for t in range(4)] + [v(224 + 4 * t, 4) for t in range(4)]
MRUN = [v(200), v(201)]
LRUN = [v(202), v(203)]
MSUB = [v(204), v(205)]
PSUM = [[v(206), v(207)], [v(208), v(209)]]
NINF = v(210)
KA = v(211)
KX = v(212)
VA = [[v(213 + 2 * ob + j) for j in range(2)] for ob in range(4)]   # v213..v220
DREM = v(221)
QOFF = [v(222), v(223)]
SCR = v(224, 16)                                                    # v224..v239
N_VGPR_OWN = 240

# AGPRs
OACC = [[a(16 * (2 * ob + nb), 16) for nb in range(2)] for ob in range(4)]
QA = [[a(128 + 4 * (8 * nb + ks), 4) for ks in range(8)] for nb in range(2)]

# per-lane inputs (placed by the compiler in v240..v255)
IN_V = ["kofs", "vofs1", "vofs2", "loff0", "loff1", "loff2", "loff3", "qlane", "dl", "h8",
        "wbase", "wx", "rdl", "stl", "lsel"]
INV = {nm: Sym(nm) for nm in IN_V}

# SGPRs: kernel arguments
KARG = dict(QP=s(0, 2), KP=s(2, 2), VP=s(4, 2), OP=s(6, 2), LP=s(8, 2), SEQ=s(10), NQT=s(11),
            NWORK=s(12), PAIRED=s(13), QSHIFT=s(14), SCALE=s(15), NBH=s(16), NFULL=s(17),
            HALF=s(18), HQ=s(19), HKV=s(20), MNQT=s(21), SHNQT=s(22), MHALF=s(23), SHHALF=s(24),
            MHQ=s(25), SHHQ=s(26), MRATIO=s(27), SHRATIO=s(28), XQ=s(29), XR=s(30))
globals().update(KARG)
DIVP = s(34, 2)        # 64-bit product of the magic divisions
RQ = s(36, 4)
RK = s(40, 4)
RV = s(44, 4)
RO = s(48, 4)
RL = s(52, 4)
KH = s(56, 2)
VH = s(58, 2)
ITEMV, WORK, BH0, QT0, BH1, QT1, BH, QT = (s(60 + j) for j in range(8))
NXT = WORK            # after the decode: the next tile's flags
Q0, KVEND, NT, WT, QW0, KVB, ITER, WOFF = (s(68 + j) for j in range(8))
T = [s(76 + j) for j in range(8)]
CMPA = s(84, 2)
CMPB = s(86, 2)
OQW, BOUND, PASS, WAVE, GRID, LDSB = (s(88 + j) for j in range(6))
# the finished tile's O resource while the next tile is set up: the redo
# check's registers, idle between walks
ORO = s(84, 4)
# s31 (the kernel-argument block's pad) and temporaries the query-tile setup
# uses only before the walk. WOFF = LDS base + 4 KB x wave: this wave's quarter
# of a ring slot.
LIM = s(31)           # the steady walk runs while ITER < LIM = WT - 1
SVLD = T[6]           # idle iterations: V load destination (tile i + 2)
SKLD = T[7]           # idle iterations: K load destination (tile i + 4)
N_SGPR_OWN = 94       # s0..s93 (except s32, s33, which the compiler reserves)

IN_S = ["ka", "wg", "ng", "wv", "lb"]
INS_ = {nm: Sym(nm) for nm in IN_S}

# ---------------------------------------------------------------------------
# MXFP8 variant (configure(True)): Q and K are e4m3 codes with one e8m0 scale
# byte per 32 elements along D, V the bf16 dequantisation. QK runs on
# v_mfma_scale_f32_32x32x64_f8f6f4: per 64-d k-step s2 lane half h supplies
# d = 64 s2 + 16 h + [0, 16) in bytes 0-15 and 64 s2 + 32 + 16 h + [0, 16) in
# bytes 16-31, with the scale of MX block 2 s2 + h, for K rows from LDS and
# Q rows from AGPRs alike. A lane's scale bytes sit in one register, byte
# 2 b + s2 for row block b (key block mb / query block nb), picked by the
# MFMA's op_sel. The K tile is 64 rows of 128 code bytes (8 KB, 128-byte-row
# swizzle), then at +8 KB the tile's 64 scale words; V as in the bf16 walk.
# ---------------------------------------------------------------------------
MX = False
_BF16_STATE = None
# vector-memory loads per walk iteration, per query tile's Q, and of the
# prologue after K(0) and Q (bf16: K 4 + V 4; Q 16; K(1), K(2), V(0))
NLD_IT, NLD_Q, NLD_PRO = 8, 16, 12
KTILE = 16384              # bytes of a K tile in HBM (64 rows)
CLOB_SKIP_V = ()           # VGPRs below N_VGPR_OWN left to the compiler's inputs


def configure(mx):
    """Rebinds the register map and limits of the bf16 (mx False) or the
    MXFP8 (mx True) kernel body."""
    global MX, FRAG, IN_V, INV, STEADY_SPAN, NLD_IT, NLD_Q, NLD_PRO, KTILE, CLOB_SKIP_V, _BF16_STATE
    global QA_MX, KSW, KSWT, QSC, QSW, KXM, QSO, RKS, QSP, KSP, WOFFK, OUTF16, MASKHI
    names = ("FRAG", "IN_V", "INV", "STEADY_SPAN", "NLD_IT", "NLD_Q", "NLD_PRO", "KTILE", "CLOB_SKIP_V")
    g = globals()
    if _BF16_STATE is None:
        _BF16_STATE = {nm: g[nm] for nm in names}
    MX = mx
    if not mx:
        g.update(_BF16_STATE)
        return
    # all fragments in AGPRs, 8 per slot (a K fragment is two b128 reads, a
    # V^T fragment uses the first 4); the VGPRs the bf16 map gives them are
    # the scale words' and the Q scale loads'
    FRAG = [a(160 + 8 * t, 8) for t in range(8)]
    QA_MX = [[a(128 + 16 * nb + 8 * s2, 8) for s2 in range(2)] for nb in range(2)]
    KSW = v(184)               # scale bytes of the lane's key rows, byte 2 mb + s2
    KSWT = [v(185), v(186)]    # scale words of rows krow, krow + 32 as read
    QSC = v(187)               # scale bytes of the lane's query rows, byte 2 nb + s2
    QSW = [v(188), v(189)]     # their words, loaded with the tile's Q
    KXM = [KA, KX, v(190), v(191)]   # K read bases of the 32-byte chunk pairs 0..3 (KA ^ 32 cp)
    QSO = [v(192), v(193)]     # Q scale word offsets of the lane's two rows
    CLOB_SKIP_V = tuple(range(194, 200))
    IN_V = ["kofs", "vofs1", "vofs2", "loff0", "loff1", "loff2", "loff3", "kl0", "kl1", "sl", "ksr",
            "psel", "qlane", "dl", "h8", "wbase", "wx", "rdl", "stl"]
    INV = {nm: Sym(nm) for nm in IN_V}
    STEADY_SPAN = 33
    NLD_IT, NLD_Q, NLD_PRO = 7, 10, 10
    KTILE = 8192
    # SGPRs the MX kernel frees: no LSE (RL, LP), no GQA (HKV, MHQ, SHHQ,
    # MRATIO, SHRATIO); the argument block carries the scale pointers there
    RKS = s(52, 4)             # K scale resource, stepped like RK
    QSP = s(8, 2)              # Q scale words (LP's slot)
    KSP = [s(27), s(28)]       # K scale words (MRATIO, SHRATIO's slots)
    OUTF16 = s(25)             # flags (MHQ's slot): bit 0 fp16 output (else bf16), bit 1 negate Q
    MASKHI = s(26)             # 0xffff0000: the high bf16 of a packed pair as fp32 (SHHQ's slot)
    WOFFK = s(20)              # LDS base + 2 KB x wave: this wave's K rows of a slot (HKV's slot)


def MFMA_SCALE(d, a_, b_, c, sa, sb, opa, opb):
    """v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 x e4m3) with scale bytes opa of
    register sa (A) and opb of sb (B)."""
    cc = c if c is not None else 0
    t = (f"v_mfma_scale_f32_32x32x64_f8f6f4 {d}, {a_}, {b_}, {cc}, {sa}, {sb}"
         f" op_sel:[{opa & 1},{opb & 1},0] op_sel_hi:[{opa >> 1},{opb >> 1},0]")
    uses = [a_, b_, sa, sb] + ([c] if c is not None else [])
    return Ins("mfma", t, defs=[d], uses=uses, mdst=tuple(d.keys()), mc=tuple(c.keys()) if c is not None else None,
               mab=a_.keys() + b_.keys() + sa.keys() + sb.keys())


RSRC3 = 0x00020000     # buffer resource word 3: raw 32-bit dwords
LDS_V = 65536          # V ring offset in LDS
LDS_STG = 131072       # output staging offset in LDS
SLOT = 16384           # bytes per K (or V) tile of 64 rows x 256 bytes
BOUND_F = 0x57800000   # 2^48: the stale-max bound of a tile sum with bf16 P
# element type of Q, K, V, P and O: bf16, or fp16 (configure_f16): its MFMA,
# the P / O pack and the stale-max bound (2^15, the largest power of two below
# fp16's 65504, so no weight of a tile that passes the check overflows)
F16 = False
MFMA_OP = "v_mfma_f32_32x32x16_bf16"
PK_OP = "v_cvt_pk_bf16_f32"


def configure_f16(on):
    global F16, MFMA_OP, PK_OP, BOUND_F
    F16 = on
    MFMA_OP = "v_mfma_f32_32x32x16_f16" if on else "v_mfma_f32_32x32x16_bf16"
    PK_OP = "v_cvt_pk_f16_f32" if on else "v_cvt_pk_bf16_f32"
    BOUND_F = 0x47000000 if on else 0x57800000
LN2 = 0x3F317218


# ---------------------------------------------------------------------------
# building blocks
# ---------------------------------------------------------------------------


def div_magic(dst, x, m, sh):
    """dst = x / d for 0 <= x < 2^31 (m, sh from the host: magic division)."""
    return [S("s_mul_i32", DIVP[0], x, m), S("s_mul_hi_u32", DIVP[1], x, m),
            S("s_lshr_b64", DIVP, DIVP, sh), S("s_mov_b32", dst, DIVP[0])]


def rsrc_at(r, head, off_s, size_s):
    """Resource over bytes [off, size) of the head at `head` (64-bit SGPR
    pair); off_s, size_s SGPRs (off may exceed size: empty resource)."""
    return [S("s_add_u32", r[0], head[0], off_s), S("s_addc_u32", r[1], head[1], 0),
            S("s_and_b32", r[1], r[1], 0xFFFF), S("s_sub_i32", r[2], size_s, off_s),
            S("s_max_i32", r[2], r[2], 0), S("s_mov_b32", r[3], RSRC3)]


def k_frag_reads(f_slot, ks, mb, first_of_ks, kslot):
    """K fragment (ks, mb) of the tile in ring slot kslot: one ds_read_b128 of
    the lane's key row krow + 32 mb, logical 16-byte chunk 2 ks + h (the XOR
    32 ks on the lane's base)."""
    out = []
    addr = KA if ks == 0 else KX
    if first_of_ks and ks > 0:
        out.append(V("v_xor_b32", KX, 32 * ks, KA))
    out.append(DSR("ds_read_b128", FRAG[f_slot], addr, SLOT * kslot + 8192 * mb))
    return out


def k_frag_reads_mx(f_slot, s2, mb, kslot):
    """MX K fragment (k-step s2, key block mb) of the tile in ring slot kslot:
    the lane's key row krow + 32 mb, chunk pairs 2 s2 and 2 s2 + 1 (bytes
    0-15 and 16-31 of the A operand)."""
    return [DSR("ds_read_b128", FRAG[f_slot].sl(4 * j, 4), KXM[2 * s2 + j], SLOT * kslot + 4096 * mb)
            for j in range(2)]


def ksw_reads(kslot):
    """The scale words of the lane's key rows krow and krow + 32 in ring slot
    kslot (the tile's 64 words follow its 8 KB of codes)."""
    return [DSR("ds_read_b32", KSWT[j], INV["ksr"], SLOT * kslot + 8192 + 128 * j) for j in range(2)]


def ksw_perm():
    """KSW byte 2 mb + s2 = scale byte 2 s2 + h of key row krow + 32 mb."""
    return V("v_perm_b32", KSW, KSWT[1], KSWT[0], INV["psel"])


def v_frag_reads(f_slot, kk, ob, vslot):
    """V^T fragment (O^T block ob, P^T k-step kk) of the tile in ring slot
    vslot: two ds_read_b64_tr_b16."""
    return [DSR("ds_read_b64_tr_b16", FRAG[f_slot].sl(0, 2), VA[ob][0], SLOT * vslot + 4096 * kk),
            DSR("ds_read_b64_tr_b16", FRAG[f_slot].sl(2, 2), VA[ob][1], SLOT * vslot + 4096 * kk)]


def rsrc_base(r, head, size_s):
    """Resource over bytes [0, size) of the head at `head` (64-bit SGPR pair)."""
    return [S("s_mov_b32", r[0], head[0]), S("s_and_b32", r[1], head[1], 0xFFFF), S("s_max_i32", r[2], size_s, 0),
            S("s_mov_b32", r[3], RSRC3)]


def rsrc_step(r, step=SLOT):
    """Resource r moved on by one tile: base + step, size - step (at least 0).
    The carry pair is one bundle, so no SCC writer lands between."""
    return [[S("s_add_u32", r[0], r[0], step), S("s_addc_u32", r[1], r[1], 0)],
            [S("s_sub_i32", r[2], r[2], step)], [S("s_max_i32", r[2], r[2], 0)]]


class VOp:
    __slots__ = ("ins", "deps", "nb_gap", "cost", "idx", "done", "emitted_at")

    def __init__(self, ins, deps=(), nb_gap=-1):
        self.ins = ins if isinstance(ins, list) else [ins]
        self.deps = list(deps)     # (VOp, min index distance)
        self.nb_gap = nb_gap       # not before this gap
        self.cost = sum(x.cost for x in self.ins)
        self.done = False
        self.emitted_at = None


class Softmax:
    """The VALU program of one tile's softmax (ops in program order)."""

    def __init__(self):
        self.ops = []

    def add(self, ins, deps=(), nb_gap=-1):
        op = VOp(ins, deps, nb_gap)
        self.ops.append(op)
        return op


def mask_kind(causal, mb, nb):
    """How the masked tile treats S^T block (mb, nb): causal diagonal tile,
    key block below the query block 'none', above it 'all', on it 'cmp';
    the last tile of a non-causal walk (keys >= S) 'cmp'."""
    if not causal:
        return "cmp"
    return {-1: "none", 0: "cmp", 1: "all"}[mb - nb]


def mask_cmp(causal, mb, nb, r):
    """v_cmp setting VCC for the masked logits of S^T block (mb, nb), register
    r: causal, key > query within the diagonal tile (block on the diagonal);
    else key >= S. The v_cndmask reading VCC must follow 2 wait states later."""
    kc = 16 * (r // 8) + (r % 8)
    if causal:
        assert mb == nb
        return V("v_cmp_gt_i32", VCC, kc, INV["dl"])
    return V("v_cmp_ge_i32", VCC, 32 * mb + kc, DREM)


def masked_select(causal, mb, nb, r, dst, src):
    """dst = src, or -inf where masked (as a bundle)."""
    kind = mask_kind(causal, mb, nb)
    if kind == "none":
        return [V("v_mov_b32", dst, src)] if dst.i != src.i else []
    if kind == "all":
        return [V("v_mov_b32", dst, NINF)]
    return [mask_cmp(causal, mb, nb, r), NOP(VALU_SGPR_VALU - 1), V("v_cndmask_b32", dst, src, NINF, VCC)]


def softmax_exp_program(sm, p, masked, causal, kk_release, first_sum_init=True, msub_deps=()):
    """Exponentials, P and row sums of S^T[p] against MSUB: groups g = (kk, nb).
    kk_release[kk]: gap from which P[kk] may be overwritten. The row sums add
    the fp32 exponentials (v_add_f32, chains (nb, e % 2)): a v_dot2 of the
    packed weights would occupy the matrix pipe (it costs an MFMA ~16
    cycles each on gfx950)."""
    last_read = {}    # (g, e): the last op reading group g's temp e
    last_sum = {}
    for g in range(8):
        kk, nb = g // 2, g % 2
        mb, hf = kk // 2, kk % 2
        tb = TMP[g % 3]
        src = SACC[p][mb][nb]
        fmas, exps = [], []
        for e in range(8):
            deps = list(msub_deps)
            if (g - 3, e) in last_read:
                deps.append((last_read[(g - 3, e)], 1))
            if masked and mask_kind(causal, mb, nb) == "all":
                ins = [V("v_mov_b32", tb[e], NINF)]
            else:
                ins = [V("v_fma_f32", tb[e], src[8 * hf + e], SCALE, "-" + str(MSUB[nb]))]
                ins[0].uses.append(("v", MSUB[nb].i))
                if masked and mask_kind(causal, mb, nb) == "cmp":
                    ins += masked_select(causal, mb, nb, 8 * hf + e, tb[e], tb[e])
            fmas.append(sm.add(ins, deps))
        for e in range(8):
            exps.append(sm.add(V("v_exp_f32", tb[e], tb[e], trans=True), [(fmas[e], 1)]))
        unp = {}
        for q in range(4):
            op = sm.add(V(PK_OP, PB[kk][nb][q], tb[2 * q], tb[2 * q + 1]),
                        [(exps[2 * q], TRANS_FWD), (exps[2 * q + 1], TRANS_FWD)], nb_gap=kk_release[kk])
            last_read[(g, 2 * q)] = last_read[(g, 2 * q + 1)] = op
            if MX:
                # the sums take the weights as rounded for PV (the pair back
                # to fp32 in the temporaries), so a tile's dominant weight
                # cancels in O / l
                unp[2 * q] = sm.add(V("v_lshlrev_b32", tb[2 * q], 16, PB[kk][nb][q]), [(op, 1)])
                unp[2 * q + 1] = sm.add(V("v_and_b32", tb[2 * q + 1], MASKHI, PB[kk][nb][q]), [(op, 1)])
        for e in range(8):
            acc = PSUM[nb][e % 2]
            init = first_sum_init and kk == 0 and e < 2
            deps = [(exps[e], TRANS_FWD), (last_read[(g, e)], 1)] + ([(unp[e], 1)] if MX else [])
            if (nb, e % 2) in last_sum:
                deps.append((last_sum[(nb, e % 2)], 1))
            op = sm.add(V("v_add_f32", acc, 0 if init else acc, tb[e]), deps)
            last_sum[(nb, e % 2)] = op
            last_read[(g, e)] = op
    return sm


class Block:
    def __init__(self):
        self.out = []

    def emit(self, x):
        if isinstance(x, list):
            for y in x:
                self.out.append(y)
        else:
            self.out.append(x)


def schedule_iteration(blk, mfmas, reads, pre_reads, side, sm_ops, budget=30, end_ops=(), fixed=None,
                       read_gaps=None):
    """Emit one iteration: `mfmas` a list of (Ins, frag index or None); `reads`
    dict frag -> list of Ins, issued at gap 2(f - LOOK) (f >= LOOK) or before
    the first MFMA (f < LOOK, unless in `pre_reads`, already in flight); `side` dict
    gap -> list of Ins (gap -1: before the first MFMA); `sm_ops` the VALU
    program, issued greedily under a per-gap cycle budget."""
    nm = len(mfmas)
    gap_reads = {}
    for f, lst in reads.items():
        if f in pre_reads:
            continue
        gap = 2 * (f - LOOK) if f >= LOOK else -1
        if read_gaps and f in read_gaps:
            gap = read_gaps[f]
        gap_reads.setdefault(min(gap, nm - 1), []).extend(lst)
    # LDS op bookkeeping for lgkmcnt: list of frag ids per emitted LDS op
    lds_log = list(pre_reads_log_for(pre_reads, reads))
    pending = list(sm_ops)
    idx_of = {}

    def emitted_index():
        return len(blk.out)

    def ready(op, gap):
        if op.nb_gap > gap:
            return False
        for d, dist in op.deps:
            if not d.done:
                return False
            if emitted_index() - d.emitted_at < dist:
                return False
        return True

    def emit_op(op):
        op.emitted_at = len(blk.out) + len(op.ins) - 1
        for x in op.ins:
            blk.out.append(x)
        op.done = True

    def fill(gap, limit):
        spent = 0
        while True:
            found = None
            for op in pending[:40]:
                if ready(op, gap):
                    found = op
                    break
            if found is None or spent + found.cost > limit and spent > 0:
                break
            pending.remove(found)
            emit_op(found)
            spent += found.cost
        return spent

    def do_gap(gap):
        # side ops first: they include the address updates the gap's reads use
        spent = 0
        for x in side.get(gap, []):
            blk.out.append(x)
            spent += x.cost
        for x in gap_reads.get(gap, []):
            blk.out.append(x)
            spent += x.cost
            if x.mem == "lgkm":
                lds_log.append(x.frag)
        if fixed:
            for x in fixed.get(gap, []):
                blk.out.append(x)
                spent += x.cost
        fill(gap, max(budget - spent, 0))

    do_gap(-1)
    for mi, (ins, frag) in enumerate(mfmas):
        if frag is not None and (mi == 0 or mfmas[mi - 1][1] != frag):
            # wait for this fragment's reads: count LDS ops issued after its last one
            last = max(j for j, f in enumerate(lds_log) if f == frag)
            after = len(lds_log) - 1 - last
            assert after <= 15
            blk.out.append(WAIT(lgkm=after))
        blk.out.append(ins)
        do_gap(mi)
    # leftover VALU after the MFMA stream: in order, with nops for the deps
    gap = nm
    while pending:
        op = None
        for cand in pending[:40]:
            if ready(cand, gap + 1000):
                op = cand
                break
        if op is None:
            blk.out.append(NOP(0))
            continue
        pending.remove(op)
        emit_op(op)
    if fixed:
        for x in fixed.get("tail", []):
            blk.out.append(x)
    for x in end_ops:
        blk.out.append(x)
    check_item_order(None, blk.out, ref=[x for op in sm_ops for x in op.ins])


# ---------------------------------------------------------------------------
# slot scheduler: a single wave issues one instruction per 4-cycle slot, so an
# MFMA every 32 cycles leaves 7 slots between two MFMAs (measured on gfx950:
# 6 FMAs between MFMAs cost nothing, 8 cost 8 cycles, 10 cost 16; SALU the
# same). Instructions are placed into those slots within their windows.
# ---------------------------------------------------------------------------


class Item:
    """An instruction bundle placed into the gap after MFMA `gap` (gap -1:
    before the first MFMA) with lo <= gap <= hi (hi None: any, or the tail);
    deps: (item, d) -- at least d wait states (instructions) between the end
    of item and this bundle (0: just after it)."""

    __slots__ = ("ins", "lo", "hi", "deps", "seq", "at", "size")
    _n = 0

    def __init__(self, ins, lo=-1, hi=None, deps=()):
        self.ins = ins if isinstance(ins, list) else [ins]
        self.lo, self.hi = lo, hi
        self.deps = list(deps)
        Item._n += 1
        self.seq = Item._n
        self.at = None
        self.size = sum(x.ws if x.kind == "nop" else LDS_SLOTS if x.kind == "lds" else 1 for x in self.ins)


def slot_schedule(mfmas, items, pre_log, cap=7, tail=()):
    """Emit `mfmas` [(Ins, frag)] with `items` in the gaps. LDS reads carry
    their fragment in Ins.frag; before an MFMA whose fragment's reads are not
    known complete, an s_waitcnt lgkmcnt covers it (and the next fragment, if
    its reads are out). pre_log: fragments of the LDS ops already in flight."""
    out = []
    log = list(pre_log)     # fragment per LDS op, in issue order
    done = 0                # ops [0, done) of log are known complete
    pending = sorted(items, key=lambda it: it.seq)
    # an item's deadline also bounds the items it depends on
    changed = True
    while changed:
        changed = False
        for it in pending:
            if it.hi is None:
                continue
            for d, _ in it.deps:
                if d.hi is None or d.hi > it.hi:
                    d.hi = it.hi
                    changed = True
    nm = len(mfmas)

    def ready(it, g):
        if it.lo > g:
            return False
        for d, dist in it.deps:
            if d.at is None or len(out) - d.at - 1 < dist:
                return False
        return True

    def place(it):
        for x in it.ins:
            out.append(x)
            if x.kind == "lds":
                log.append(x.frag)
        it.at = len(out) - 1
        pending.remove(it)

    def last_op(f):
        idx = [j for j, fr in enumerate(log) if fr == f]
        return idx[-1] if idx else None

    for g in range(-1, nm):
        used = 0
        cap_g = cap if not isinstance(cap, list) else cap[max(g, 0)]
        # LDS and vector-memory bundles lead the gap: issued behind VALU work
        # (a transcendental in particular) they hold up the next MFMA
        # (measured on gfx950: +2.3 cycles per MFMA for an LDS read at the end
        # of the gap, +3 for an LDS DMA, nothing at its start)
        for mem_only in (True, False):
            while True:
                cands = [it for it in pending if ready(it, g) and
                         (not mem_only or it.ins[0].kind in ("lds", "vmem"))]
                if not cands:
                    break
                forced = [it for it in cands if it.hi is not None and it.hi <= g]
                pick = min(forced or cands, key=lambda it: (it.hi if it.hi is not None else 10 ** 6, it.seq))
                if not forced and used + pick.size > cap_g:
                    break
                place(pick)
                used += pick.size
        late = [it for it in pending if it.hi is not None and it.hi <= g]
        assert not late, f"gap {g}: items past their deadline: {[x.ins[0].text for x in late]}"
        if g + 1 < nm:
            ins, f = mfmas[g + 1]
            if f is not None:
                lf = last_op(f)
                assert lf is not None, f"fragment {f} read before its MFMA {g + 1}"
                if lf >= done:
                    # cover the next fragment too if its reads are out: a wait
                    # per two fragments
                    ln = last_op(f + 1)
                    upto = ln if ln is not None else lf
                    n_after = min(len(log) - 1 - upto, 15)
                    out.append(WAIT(lgkm=n_after))
                    done = len(log) - n_after
            out.append(ins)
    # the tail: the rest in order of readiness, nops where a distance is not met
    while pending:
        cands = [it for it in pending if ready(it, 10 ** 6)]
        if cands:
            place(min(cands, key=lambda it: (it.hi if it.hi is not None else 10 ** 6, it.seq)))
        else:
            out.append(NOP(0))
    out.extend(tail)
    check_item_order(items, out)
    return out


def check_item_order(items, out, ref=None):
    """The scheduled order keeps the items' dataflow: every register a
    placed instruction reads comes from the same writer as in the items'
    creation order (or the reference order `ref`), and each register's last
    writer is the same. (Items that touch a register without a dependency
    between them would race.)"""
    if ref is None:
        ref = [x for it in sorted(items, key=lambda it: it.seq) for x in it.ins]
    ids = {id(x) for x in ref}
    assert len(ids) == len(ref), "an instruction placed twice"

    def flow(seq):
        last, reads = {}, {}
        for x in seq:
            if id(x) not in ids:
                continue
            for k in x.uses:
                reads[(id(x), k)] = last.get(k)
            for k in x.defs:
                last[k] = id(x)
        return reads, last
    r0, l0 = flow(ref)
    r1, l1 = flow(out)
    bad = [k for k in r0 if r0[k] != r1.get(k)] + [k for k in l0 if l0[k] != l1.get(k)]
    if bad:
        txt = {id(x): x.text for x in ref}
        k = bad[0]
        where = txt.get(k[0], k) if isinstance(k, tuple) else k
        raise CheckError(f"schedule changes the dataflow of {len(bad)} reads, first: {where} {k}")


def _conflict(a, b):
    da, ua, db, ub = set(a.defs), set(a.uses), set(b.defs), set(b.uses)
    return bool(da & ub or ua & db or da & db)


def pre_reads_log_for(pre_reads, reads):
    log = []
    for f in sorted(pre_reads):
        for x in reads[f]:
            if x.mem == "lgkm":
                log.append(f)
    return log


# ---------------------------------------------------------------------------
# kernel body
# ---------------------------------------------------------------------------


class Gen:
    def __init__(self, causal):
        self.causal = causal
        self.tag = ("M" if MX else "H" if F16 else "") + ("C" if causal else "F")
        self.prog = []
        self.nlab = 0

    def L(self, name):
        return f"L_pfw64{self.tag}_{name}"

    def emit(self, x):
        if isinstance(x, list):
            self.prog.extend(x)
        else:
            self.prog.append(x)

    # ------------------------------------------------------------ iteration parts
    # Ring slots. Iteration i (u = i mod 4) reads K tile i + 1 (QK), V tile
    # i - 1 (PV) and V tile i (the next PV's first fragments), and loads K
    # tile i + 4 and V tile i + 2; tile t lives in slot t mod 4 of its ring.
    # Every iteration but the idle one has its u fixed where it is generated,
    # so the slots are instruction offsets on addresses fixed for the kernel.
    @staticmethod
    def slots(u):
        return dict(krd=(u + 1) % 4, vpv=(u + 3) % 4, vpre=u, kld=u, vld=(u + 2) % 4)

    def load_groups(self, u):
        """The 8 LDS-DMA loads of iteration i (u = i mod 4): K tile i+4, then V
        tile i+2, this wave's 16 rows of each as 4 x 1 KB. M0 is set once per
        tile (the instruction offset steps the LDS and global addresses by
        1 KB together); RK and RV move on to tiles i+5 and i+3 after their last
        load. 8 groups, one load each."""
        sl = self.slots(u)
        if MX:
            groups = [([m0, NOP(0)] if m0 is not None else []) + [ld] for m0, ld in self.mx_loads(u)]
            for r, step, j in self.mx_steps():
                groups[j] += [x for b in rsrc_step(r, step) for x in b]
            return groups
        groups = []
        for r, base in ((RK, SLOT * sl["kld"]), (RV, LDS_V + SLOT * sl["vld"])):
            for j in range(4):
                pre = [S("s_add_u32", M0, WOFF, base), NOP(0)] if j == 0 else []
                groups.append(pre + [BLOAD_LDS(INV[f"loff{j}"], r, 1024 * j)])
        groups[4] += [x for b in rsrc_step(RK) for x in b]
        groups[7] += [x for b in rsrc_step(RV) for x in b]
        return groups

    def barrier(self, vm):
        return [WAIT(vm=vm), BAR()]

    def mx_loads(self, u):
        """MX: the 7 LDS-DMA loads of iteration i (u = i mod 4) as (M0 write or
        None, load): K tile i+4's codes (this wave's 16 rows of 128 bytes as
        2 x 1 KB), its 64 scale words (every wave loads all of them, to the
        same place), then V tile i+2 as in the bf16 walk."""
        sl = self.slots(u)
        kb = SLOT * sl["kld"]
        vb = LDS_V + SLOT * sl["vld"]
        return [(S("s_add_u32", M0, WOFFK, kb), BLOAD_LDS(INV["kl0"], RK)),
                (None, BLOAD_LDS(INV["kl1"], RK, 1024)),
                (S("s_add_u32", M0, LDSB, kb + 8192), BLOAD_LDS_DW(INV["sl"], RKS)),
                (S("s_add_u32", M0, WOFF, vb), BLOAD_LDS(INV["loff0"], RV))] + [
                (None, BLOAD_LDS(INV[f"loff{j}"], RV, 1024 * j)) for j in range(1, 4)]

    @staticmethod
    def mx_steps():
        """MX: (resource, step, index of its last load) of the ring loads."""
        return [(RK, KTILE, 1), (RKS, 256, 2), (RV, SLOT, 6)]

    @staticmethod
    def caps(mf, cap):
        """Issue slots per gap: the gap after a 16-pass MX QK MFMA (64 cycles)
        holds twice the gap after an 8-pass one."""
        if not MX:
            return cap
        return [2 * cap if "scale" in ins.text else cap for ins, _ in mf]

    @staticmethod
    def pre_lo(nf, j):
        """First gap for the prefetch of the next iteration's fragment j (slot
        j): a gap after the MFMAs of this iteration's last fragment in that slot, and
        no more than LOOK fragments ahead."""
        lo = -1
        for jj in range(j + 1):          # not before the fragments ahead of it (reads stay in order)
            prev = [f for f in range(nf) if f % NSLOT == jj % NSLOT]
            lo = max(lo, 2 * prev[-1] + 2 if prev else -1, 2 * (nf + jj - LOOK))
        return lo

    def prefetch_items(self, nf, nm, u):
        """[(fragment, first gap, reads)] of the prefetch; one placed after the
        last MFMA (which may read its slot) starts with a wait state."""
        out = []
        for j, (f, lst) in enumerate(sorted(self.v_prefetch(nf, u).items())):
            lo = self.pre_lo(nf, j)
            out.append((f, lo, ([NOP(0)] if nm and lo >= nm else []) + lst))
        return out

    @staticmethod
    def pre_log():
        """Fragments of the LDS reads the previous iteration's prefetch left in
        flight, in issue order."""
        return ([0, 0] if MX else []) + [f for f in range(LOOK) for _ in range(2)]

    def mfma_lists(self, pv, qk_par, u):
        """MFMA list [(Ins, frag)] and frag reads {frag: [Ins]} of iteration
        i = u (mod 4) with PV(i - 1) and/or QK(i + 1) into SACC[qk_par]."""
        sl = self.slots(u)
        mf, reads = [], {}
        f = 0
        if pv:
            for kk in range(4):
                for ob in range(4):
                    slot = f % NSLOT
                    reads[f] = v_frag_reads(slot, kk, ob, sl["vpv"])
                    for nb in range(2):
                        mf.append((MFMA(OACC[ob][nb], FRAG[slot].sl(0, 4), PB[kk][nb], OACC[ob][nb]), f))
                    f += 1
        if qk_par is not None and MX:
            for s2 in range(2):
                for mb in range(2):
                    slot = f % NSLOT
                    reads[f] = k_frag_reads_mx(slot, s2, mb, sl["krd"])
                    for nb in range(2):
                        dst = SACC[qk_par][mb][nb]
                        mf.append((MFMA_SCALE(dst, FRAG[slot], QA_MX[nb][s2], None if s2 == 0 else dst, KSW, QSC,
                                              2 * mb + s2, 2 * nb + s2), f))
                    f += 1
        elif qk_par is not None:
            for ks in range(8):
                for mb in range(2):
                    slot = f % NSLOT
                    reads[f] = k_frag_reads(slot, ks, mb, mb == 0, sl["krd"])
                    for nb in range(2):
                        dst = SACC[qk_par][mb][nb]
                        mf.append((MFMA(dst, FRAG[slot], QA[nb][ks], None if ks == 0 else dst), f))
                    f += 1
        for fr, lst in reads.items():
            for x in lst:
                x.frag = fr
        return mf, reads, f

    # the V(i) fragments 0..LOOK-1 read at the end of an iteration for the next PV
    def v_prefetch(self, nf, u):
        """(MX: first the scale words of K tile i + 2, whose QK is the next
        iteration's, counted with its first fragment.)"""
        reads = {}
        for j in range(LOOK):
            lst = v_frag_reads(j % NSLOT, j // 4, j % 4, self.slots(u)["vpre"])
            if MX and j == 0:
                lst = ksw_reads((u + 2) % 4) + lst
            for x in lst:
                x.frag = nf + j
            reads[nf + j] = lst
        return reads

    def mfma_iteration(self, name, u, pv, qk_par, sm, prefetch, side_extra=None, budget=30, end_ops=(), fixed=None):
        mf, reads, nf = self.mfma_lists(pv, qk_par, u)
        pre = set(range(LOOK)) if pv else set()
        assert not (MX and pv)
        read_gaps = None
        if prefetch:
            if MX:
                pre_it = self.prefetch_items(nf, len(mf), u)
                reads.update({f: lst for f, _, lst in pre_it})
                read_gaps = {f: lo for f, lo, _ in pre_it}
            else:
                reads.update(self.v_prefetch(nf, u))
        side = {}
        if MX and qk_par is not None:
            # the scale bytes of this iteration's QK (no prefetch before it)
            side[-1] = ksw_reads(self.slots(u)["krd"]) + [WAIT(lgkm=0), ksw_perm()]
        nm = len(mf)
        # loads spread over the stream
        loads = self.load_groups(u)
        for j, grp in enumerate(loads):
            gap = (j * nm) // len(loads) + 1 if nm else -1
            side.setdefault(min(gap, nm - 1) if nm else -1, []).extend(grp)
        if side_extra:
            for g, lst in side_extra.items():
                side.setdefault(g, []).extend(lst)
        blk = Block()
        schedule_iteration(blk, mf, reads, pre, side, sm.ops if sm else [], budget=budget, end_ops=end_ops,
                           fixed=fixed, read_gaps=read_gaps)
        return blk.out

    # ------------------------------------------------------------ softmax programs
    def first_softmax(self, masked):
        """Softmax of a wave's first tile (parity 0): the row max first."""
        sm = Softmax()
        p = 0
        settle = []
        for nb in range(2):
            # temporaries in TMP[2]: its first exponentials wait for the max
            acc = [TMP[2][nb * 4 + 0], TMP[2][nb * 4 + 1]]
            ops = []
            if not masked:
                for mb in range(2):
                    src = SACC[p][mb][nb]
                    prev = sm.add(V("v_max3_f32", acc[mb], src[0], src[1], src[2]))
                    r = 3
                    while r < 16:
                        hi = src[r + 1] if r + 1 < 16 else src[r]
                        prev = sm.add(V("v_max3_f32", acc[mb], acc[mb], src[r], hi), [(prev, 1)])
                        r += 2
                    ops.append(prev)
            else:
                for mb in range(2):
                    src = SACC[p][mb][nb]
                    prev = sm.add(V("v_mov_b32", acc[mb], NINF))
                    kind = mask_kind(self.causal, mb, nb)
                    for r in range(16 if kind != "all" else 0):
                        if kind == "none":
                            prev = sm.add(V("v_max_f32", acc[mb], acc[mb], src[r]), [(prev, 1)])
                            continue
                        # one temporary per (nb, mb) chain: the chains are
                        # independent and may interleave; within a chain the
                        # select waits for the previous max
                        tmpr = TMP[0][2 * nb + mb]
                        op = sm.add(masked_select(self.causal, mb, nb, r, tmpr, src[r]), [(prev, 1)])
                        prev = sm.add(V("v_max_f32", acc[mb], acc[mb], tmpr), [(op, 1)])
                    ops.append(prev)
            m = TMP[2][nb * 4 + 2]
            x = TMP[2][nb * 4 + 3]
            o1 = sm.add(V("v_max_f32", m, acc[0], acc[1]), [(ops[0], 1), (ops[1], 1)])
            o2 = sm.add(V("v_mov_b32", x, m), [(o1, 1)])
            o3 = sm.add([NOP(PERM_WS - 1), V("v_permlane32_swap_b32", m, x, perm=True)], [(o2, 1)])
            o4 = sm.add([NOP(PERM_WS - 1), V("v_max_f32", m, m, x)], [(o3, 1)])
            # MRUN = m == -inf ? -inf : m * c; MSUB = finite ? MRUN : 0
            o5 = sm.add(V("v_mul_f32", MRUN[nb], SCALE, m), [(o4, 1)])
            o6 = sm.add([V("v_cmp_neq_f32", VCC, NINF, m), NOP(1), V("v_cndmask_b32", MRUN[nb], NINF, MRUN[nb], VCC)],
                        [(o5, 1)])
            o7 = sm.add([V("v_cmp_neq_f32", VCC, NINF, MRUN[nb]), NOP(1),
                         V("v_cndmask_b32", MSUB[nb], 0, MRUN[nb], VCC)], [(o6, 1)])
            settle.append((o7, 1))
        softmax_exp_program(sm, p, masked, self.causal, kk_release=[-1] * 4, msub_deps=settle)
        return sm

    def tail_first(self):
        """Tile sums -> LRUN (first tile: l = sum)."""
        return NOPS(DOT_FWD) + [V("v_add_f32", LRUN[0], PSUM[0][0], PSUM[0][1]),
                                V("v_add_f32", LRUN[1], PSUM[1][0], PSUM[1][1])]

    def tail_stale(self, redo_label, ret_label):
        """Tile sums; redo when some lane's sum is above the bound or not
        finite; else l += sum."""
        return NOPS(DOT_FWD) + [
                V("v_add_f32", PSUM[0][0], PSUM[0][0], PSUM[0][1]),
                V("v_add_f32", PSUM[1][0], PSUM[1][0], PSUM[1][1]),
                V("v_cmp_nle_f32", CMPA, PSUM[0][0], BOUND),
                V("v_cmp_nle_f32", CMPB, PSUM[1][0], BOUND),
                NOP(4),
                S("s_or_b64", CMPA, CMPA, CMPB),
                CBR("s_cbranch_scc1", redo_label),
                V("v_add_f32", LRUN[0], LRUN[0], PSUM[0][0]),
                V("v_add_f32", LRUN[1], LRUN[1], PSUM[1][0]),
                LABEL(ret_label)]

    def redo_block(self, label, ret_kind, p, masked):
        """Rare path: a tile sum passed the bound. New max of S^T[p], O and l
        rescaled, exponentials again (straight-line); back to the copy of the
        iteration (u = ITER mod 4, u = p or p + 2) it came from."""
        # temporaries in TMP and PB: the next tile's first V^T fragments are in
        # flight into the fragment slots
        R = TMP[1]
        out = [LABEL(label)] + NOPS(MFMA_WS + 4)
        for nb in range(2):
            acc = [R[nb * 4 + 0], R[nb * 4 + 1]]
            for mb in range(2):
                src = SACC[p][mb][nb]
                out.append(V("v_mov_b32", acc[mb], NINF))
                kind = mask_kind(self.causal, mb, nb) if masked else "none"
                for r in range(16 if kind != "all" else 0):
                    if kind == "cmp":
                        out += masked_select(self.causal, mb, nb, r, TMP[0][0], src[r])
                        out.append(V("v_max_f32", acc[mb], acc[mb], TMP[0][0]))
                    else:
                        out.append(V("v_max_f32", acc[mb], acc[mb], src[r]))
            m, x = R[nb * 4 + 2], R[nb * 4 + 3]
            out += [V("v_max_f32", m, acc[0], acc[1]), V("v_mov_b32", x, m)] + NOPS(PERM_WS) + [
                V("v_permlane32_swap_b32", m, x, perm=True)] + NOPS(PERM_WS) + [
                V("v_max_f32", m, m, x),
                V("v_mul_f32", acc[0], SCALE, m),
                V("v_cmp_neq_f32", VCC, NINF, m), NOP(1),
                V("v_cndmask_b32", acc[0], NINF, acc[0], VCC),                                  # tile max (scaled)
                V("v_max_f32", m, MRUN[nb], acc[0]),                                            # m_new
                V("v_sub_f32", x, MRUN[nb], m), V("v_exp_f32", x, x, trans=True), NOP(1),
                V("v_cmp_neq_f32", VCC, NINF, m), NOP(1), V("v_cndmask_b32", x, "1.0", x, VCC)]
            # alpha in x (R[nb*4+3]), m_new in m (R[nb*4+2])
        # O *= alpha, 16 accumulators at a time through PB
        for nb in range(2):
            al = R[nb * 4 + 3]
            for ob in range(4):
                src = OACC[ob][nb]
                tmp = [v(128 + 16 * (ob % 2) + r) for r in range(16)]
                out += [ACCR(tmp[r], src[r]) for r in range(16)]
                out += [V("v_mul_f32", tmp[r], al, tmp[r]) for r in range(16)]
                out += [ACCW(src[r], tmp[r]) for r in range(16)]
            out += [V("v_mul_f32", LRUN[nb], al, LRUN[nb]),
                    V("v_mov_b32", MRUN[nb], R[nb * 4 + 2]),
                    V("v_cmp_neq_f32", VCC, NINF, MRUN[nb]), NOP(1), V("v_cndmask_b32", MSUB[nb], 0, MRUN[nb], VCC)]
        # exponentials again (program order, nops where a result is read early)
        sm = Softmax()
        softmax_exp_program(sm, p, masked, self.causal, kk_release=[-1] * 4)
        emitted = []
        for op in sm.ops:
            for d, dist in op.deps:
                have = len(emitted) - d.emitted_at
                if have < dist:
                    emitted += NOPS(dist - have)
            op.emitted_at = len(emitted) + len(op.ins) - 1
            emitted += op.ins
        out += emitted + NOPS(DOT_FWD)
        out += [V("v_add_f32", PSUM[0][0], PSUM[0][0], PSUM[0][1]),
                V("v_add_f32", PSUM[1][0], PSUM[1][0], PSUM[1][1]),
                V("v_add_f32", LRUN[0], LRUN[0], PSUM[0][0]),
                V("v_add_f32", LRUN[1], LRUN[1], PSUM[1][0]),
                S("s_and_b32", T[0], ITER, 3), S("s_cmp_eq_u32", T[0], p),
                CBR("s_cbranch_scc1", self.L(f"{ret_kind}{p}")), BR(self.L(f"{ret_kind}{p + 2}"))]
        return out

    def stale_softmax(self, p, masked, kk_release):
        sm = Softmax()
        softmax_exp_program(sm, p, masked, self.causal, kk_release)
        return sm

    def slot_iter(self, kind, u, pv, qk_par, sm, prefetch, side=None, end_ops=()):
        """An iteration i = u (mod 4) other than the steady one, placed by
        slot_schedule: PV(i-1) if pv, QK(i+1) into SACC[qk_par] if qk_par is
        not None, the VALU program sm (its ops in program order, a VOp
        distance d kept as d instructions between), the V(i) prefetch, the 8
        loads and the resource steps; side: {gap: [Ins]} placed in order from
        that gap on; end_ops after the stream."""
        mf, reads, nf = self.mfma_lists(pv, qk_par, u)
        nm = len(mf)
        items = []

        def add(ins, lo=-1, hi=None, deps=()):
            it = Item(ins, lo, hi, deps)
            items.append(it)
            return it
        sl = self.slots(u)
        ksw_item = None
        if MX and qk_par is not None:
            # the scale bytes of this iteration's QK (no prefetch before it)
            assert not pv
            ksw_item = add(ksw_reads(sl["krd"]) + [WAIT(lgkm=0), ksw_perm()] + NOPS(VALU_TO_MFMA), -1, -1)
        if MX:
            prev, lasts = None, []
            for j, (m0, ld) in enumerate(self.mx_loads(u)):
                at = (j * nm) // NLD_IT
                deps = [(prev, 0)] if prev else []
                if m0 is not None:
                    m = add(m0, at - 1 if nm else -1, at if nm else None, deps)
                    deps = deps + [(m, M0_WS)]
                prev = add(ld, at + 1 if nm else -1, None, deps)
                lasts.append(prev)
            for r, step, j in self.mx_steps():
                dep = lasts[j]
                for b in rsrc_step(r, step):
                    dep = add(b, -1, None, [(dep, 0)])
        if not MX:
            prev, last = None, {}
        for j in range(8 if not MX else 0):
            r = RK if j < 4 else RV
            at = (j * nm) // 8
            deps = [(prev, 0)] if prev else []
            if j % 4 == 0:
                base = SLOT * sl["kld"] if j < 4 else LDS_V + SLOT * sl["vld"]
                m = add(S("s_add_u32", M0, WOFF, base), at - 1 if nm else -1, at if nm else None, deps)
                deps = deps + [(m, M0_WS)]
            prev = add(BLOAD_LDS(INV[f"loff{j % 4}"], r, 1024 * (j % 4)), at + 1 if nm else -1, None, deps)
            last[r.i] = prev
        for r in (RK, RV) if not MX else ():
            dep = last[r.i]
            for b in rsrc_step(r):
                dep = add(b, -1, None, [(dep, 0)])
        fitem, xitem = {}, None
        for f in range(nf):
            if pv and f < LOOK:
                continue                       # read by the iteration before
            lo = max(2 * (f - NSLOT) + 1, 2 * (f - LOOK), -1)
            hi = max(2 * f - 5, -1) if nm else None
            deps = []
            lds = [x for x in reads[f] if x.kind == "lds"]
            xor = [x for x in reads[f] if x.kind != "lds"]
            if xor:                            # KX for this ks, after the last read of the old one
                xitem = add(xor, max(lo - 2, -1), max(2 * f - 6, -1) if nm else None,
                            [(fitem[f - 1], 0)] if f - 1 in fitem else [])
            if not MX and ("v", KX.i) in lds[0].uses:
                deps.append((xitem, 0))
            fitem[f] = add(lds, lo, hi, deps)
        if prefetch:
            for f, lo, lst in self.prefetch_items(nf, nm, u):
                add(lst, lo if nm else -1, None, [(ksw_item, 0)] if ksw_item else [])
        # side ops (gap -1's before the VALU program, which may read them)
        first_side = None
        for g, lst in sorted((side or {}).items()):
            dep = None
            for x in lst:
                dep = add(x, g if nm else -1, None, [(dep, 0)] if dep else [])
            if g == -1:
                first_side = dep
        if sm is not None:
            conv = {}
            for op in sm.ops:
                deps = [(conv[id(d)], dist) for d, dist in op.deps] + ([(first_side, 0)] if first_side else [])
                conv[id(op)] = add(op.ins, op.nb_gap if nm else -1, None, deps)
        pre_log = self.pre_log() if pv else []
        return slot_schedule(mf, items, pre_log, cap=self.caps(mf, OTHER_CAP[kind]), tail=list(end_ops))

    # ------------------------------------------------------------ iteration variants
    def it_fill(self):
        """i = -1: QK(0) into SACC[0]; O zeroed under it."""
        sm = Softmax()
        for ob in range(4):
            for nb in range(2):
                for r in range(16):
                    sm.add(ACCW(OACC[ob][nb][r], 0))
        return self.slot_iter("fill", 3, False, 0, sm, False)

    def it_first(self):
        """i = 0 (walk of >= 2 tiles): softmax(0) with the row max, QK(1)."""
        sm = self.first_softmax(False)
        return self.mfma_iteration("first", 0, False, 1, sm, True, budget=48, end_ops=self.tail_first())

    def it_first_last(self):
        """i = 0 of a one-tile walk: masked softmax(0), no MFMAs."""
        sm = self.first_softmax(True)
        side = {}
        if not self.causal:
            side[-1] = [V("v_sub_u32", DREM, KVEND, INV["h8"])]   # keys >= S of tile 0
        side.setdefault(-1, []).extend(x for b in self.q_loads() for x in b)
        return self.mfma_iteration("first_last", 0, False, None, sm, True, side_extra=side, budget=10 ** 6,
                                   end_ops=self.tail_first())

    def it_steady(self, u):
        """1 <= i <= wt-2 (u = i mod 4): PV(i-1), QK(i+1) into SACC[1-p],
        softmax(i) of SACC[p] (p = u % 2) and the loads of K tile i+4 and V
        tile i+2, placed by slot_schedule."""
        if MX:
            return self.it_steady_mx(u)
        p = u % 2
        sl = self.slots(u)
        mf, reads, nf = self.mfma_lists(True, 1 - p, u)
        items = []

        def add(ins, lo=-1, hi=None, deps=()):
            it = Item(ins, lo, hi, deps)
            items.append(it)
            return it

        # The iteration's barrier, behind its first MFMA (which reads a V(i-1)
        # fragment read in the previous iteration): it orders every wave's
        # reads of iteration i-1 before this iteration's loads into the slots
        # they read, and (after vmcnt(8): the loads of i-2 and older have
        # landed) the V(i) prefetch after the tile's arrival. The reads of
        # this iteration before the prefetch are of tiles that landed by the
        # previous barrier (K(i+1) and V(i-1) were loaded in iteration i-3).
        bar = add([WAIT(vm=8), BAR()], 0, 0)
        # loads: one per 8 gaps, K then V (the barrier's vmcnt assumes this
        # order); M0 once per tile, written in an earlier gap than its first
        # load (the MFMA between gives the wait state, and the load can lead
        # its gap) and after the last load that reads the old value
        prev = bar
        last = {}
        for j in range(8):
            r = RK if j < 4 else RV
            deps = [(prev, 0)] if prev else []
            if j % 4 == 0:
                base = SLOT * sl["kld"] if j < 4 else LDS_V + SLOT * sl["vld"]
                m = add(S("s_add_u32", M0, WOFF, base), 8 * j - 1, 8 * j, deps)
                deps = deps + [(m, M0_WS)]
            prev = add(BLOAD_LDS(INV[f"loff{j % 4}"], r, 1024 * (j % 4)), 1 + 8 * j, 61, deps)
            last[r.i] = prev
        # the resources move on to tiles i+5 (K) and i+3 (V) after their last load
        for r in (RK, RV):
            dep = last[r.i]
            for b in rsrc_step(r):
                dep = add(b, -1, None, [(dep, 0)])
        # fragment reads: slot f % NSLOT is free after the MFMAs of fragment f - NSLOT
        fitem = {}
        xitem = None
        for f in range(LOOK, nf):
            # no earlier than LOOK fragments ahead (the LDS counter tracks 15 ops)
            lo = max(2 * (f - NSLOT) + 1, 2 * (f - LOOK))
            deps = []
            lds = [x for x in reads[f] if x.kind == "lds"]
            if f >= 16:                       # K fragment (ks, mb) = ((f-16)//2, (f-16)%2)
                ks, mb = (f - 16) // 2, (f - 16) % 2
                xor = [x for x in reads[f] if x.kind != "lds"]
                if xor:                        # KX for this ks, after the last read of the old one
                    xitem = add(xor, lo - 2, 2 * f - 6, [(fitem[f - 1], 0)] if f - 1 >= 16 else [])
                if ks > 0:
                    deps.append((xitem, 0))
            fitem[f] = add(lds, lo, 2 * f - 5, deps)
        # prefetch of V(i) fragments 0..LOOK-1 into the next iteration's slots
        pre_next = self.v_prefetch(nf, u)
        for f, lst in sorted(pre_next.items()):
            add(lst, max(2 * (f - NSLOT) + 1, 2 * (f - LOOK)), None, [(bar, 0)])
        # softmax of tile i: element e (group e / 8 = (kk, nb)), fp32 row sums
        rel = [8 * kk + 7 for kk in range(4)]
        tmp = [v(160 + j) for j in range(24)]
        fma, exp, adds, cvt = {}, {}, {}, {}
        for e in range(64):
            # element e around gap pos: the 64 elements over gaps 0..SPAN, so
            # the tile sums and the redo check fit before the last MFMA
            pos = (e * STEADY_SPAN) // 63
            g = e // 8
            kk, nb = g // 2, g % 2
            srcr = SACC[p][kk // 2][nb][8 * (kk % 2) + e % 8]
            t = tmp[e % 24]
            x = V("v_fma_f32", t, srcr, SCALE, "-" + str(MSUB[nb]))
            x.uses.append(("v", MSUB[nb].i))
            deps = []
            if e >= 24:
                deps += [(adds[e - 24], 0), (cvt[(e - 24) // 2], 0)]
            fma[e] = add(x, max(0, pos - 3), pos + 1, deps)
            exp[e] = add(V("v_exp_f32", t, t, trans=True), pos, pos + 2, [(fma[e], 0)])
            if e % 2 == 1:
                i = e // 2
                lo = max(pos + 1, rel[kk])
                cvt[i] = add(V(PK_OP, PB[kk][nb][(e % 8) // 2], tmp[(e - 1) % 24], t),
                             lo, min(lo + 6, 62), [(exp[e - 1], TRANS_FWD), (exp[e], TRANS_FWD)])
            acc = PSUM[nb][e % 2]
            init = kk == 0 and e % 8 < 2
            deps = [(exp[e], TRANS_FWD)]
            if not init:
                prev_same = max(j for j in adds if (j // 8) % 2 == nb and j % 2 == e % 2)
                deps.append((adds[prev_same], 0))
            adds[e] = add(V("v_add_f32", acc, 0 if init else acc, t), pos + 1, pos + 4, deps)
        # tile sums (nb = 0 is complete before the stream ends)
        last0 = [adds[e] for e in range(64) if (e // 8) % 2 == 0]
        last1 = [adds[e] for e in range(64) if (e // 8) % 2 == 1]
        s0 = add(V("v_add_f32", PSUM[0][0], PSUM[0][0], PSUM[0][1]), 0, None, [(a_, 0) for a_ in last0])
        c0 = add(V("v_cmp_nle_f32", CMPA, PSUM[0][0], BOUND), 0, None, [(s0, 0)])
        s1 = add(V("v_add_f32", PSUM[1][0], PSUM[1][0], PSUM[1][1]), 0, None, [(a_, 0) for a_ in last1])
        c1 = add(V("v_cmp_nle_f32", CMPB, PSUM[1][0], BOUND), 0, None, [(s1, 0)])
        # the redo check before the last MFMA (QK(i+1) does not read the
        # sums; PV(i-1) is complete, so the redo path may rescale O); the redo
        # path adds its own sums to l and comes back to the label
        add([S("s_or_b64", CMPA, CMPA, CMPB), CBR("s_cbranch_scc1", self.L(f"redo_s{p}")),
             V("v_add_f32", LRUN[0], LRUN[0], PSUM[0][0]), V("v_add_f32", LRUN[1], LRUN[1], PSUM[1][0]),
             LABEL(self.L(f"ret_s{u}"))], 0, len(mf) - 2, [(c0, VALU_SGPR_VMEM), (c1, VALU_SGPR_VMEM)])
        pre_log = self.pre_log()
        return slot_schedule(mf, items, pre_log, cap=self.caps(mf, GAP_CAP))

    def it_steady_mx(self, u):
        """MX steady iteration: 32 PV MFMAs (8 passes), then 8 QK MFMAs (16
        passes) whose gaps hold twice the slots; the softmax spreads over gaps
        0..STEADY_SPAN; the scale bytes of QK(i+1) are assembled from the
        words the previous iteration's prefetch read."""
        p = u % 2
        mf, reads, nf = self.mfma_lists(True, 1 - p, u)
        nm = len(mf)
        nqk = sum(1 for ins, _ in mf if "scale" in ins.text)
        items = []

        def add(ins, lo=-1, hi=None, deps=()):
            it = Item(ins, lo, hi, deps)
            items.append(it)
            return it

        # the barrier as in the bf16 walk (after vmcnt(NLD_IT): the loads of
        # i-2 and older have landed)
        bar = add([WAIT(vm=NLD_IT), BAR()], 0, 0)
        # KSW for QK(i+1), before its first MFMA (VALU -> MFMA wait states)
        perm = add(ksw_perm(), 0, nm - nqk - 2)
        # loads spread over gaps 1..nm-3, K codes, K scales, then V (the
        # barrier's vmcnt assumes this order); M0 written in the gap before
        prev, lasts = bar, []
        lds_loads = self.mx_loads(u)
        for j, (m0, ld) in enumerate(lds_loads):
            at = (j * (nm - 4)) // len(lds_loads)
            deps = [(prev, 0)]
            if m0 is not None:
                m = add(m0, max(at - 1, 0), at, deps)
                deps = deps + [(m, M0_WS)]
            prev = add(ld, at + 1, nm - 3, deps)
            lasts.append(prev)
        for r, step, j in self.mx_steps():
            dep = lasts[j]
            for b in rsrc_step(r, step):
                dep = add(b, -1, None, [(dep, 0)])
        # fragment reads (one AGPR ring for V^T and K fragments)
        for f in range(LOOK, nf):
            add(reads[f], max(2 * (f - NSLOT) + 1, 2 * (f - LOOK)), 2 * f - 5)
        # prefetch of V(i) fragments 0..LOOK-1 and K(i+2)'s scale words
        for j, (f, lo, lst) in enumerate(self.prefetch_items(nf, nm, u)):
            add(lst, lo, None, [(bar, 0)] + ([(perm, 0)] if j == 0 else []))
        # softmax of tile i (as the bf16 steady iteration, over 0..STEADY_SPAN)
        rel = [8 * kk + 7 for kk in range(4)]
        tmp = [v(160 + j) for j in range(24)]
        fma, exp, adds, cvt = {}, {}, {}, {}
        for e in range(64):
            pos = (e * STEADY_SPAN) // 63
            g = e // 8
            kk, nb = g // 2, g % 2
            srcr = SACC[p][kk // 2][nb][8 * (kk % 2) + e % 8]
            t = tmp[e % 24]
            x = V("v_fma_f32", t, srcr, SCALE, "-" + str(MSUB[nb]))
            x.uses.append(("v", MSUB[nb].i))
            deps = []
            if e >= 24:
                deps += [(adds[e - 24], 0), (cvt[(e - 24) // 2], 0)]
            fma[e] = add(x, max(0, pos - 3), pos + 1, deps)
            exp[e] = add(V("v_exp_f32", t, t, trans=True), pos, pos + 2, [(fma[e], 0)])
            if e % 2 == 0:
                continue
            # the pair packed for PV, back to fp32 as rounded, into the sums
            # (so a tile's dominant weight cancels in O / l)
            i = e // 2
            lo = max(pos + 1, rel[kk])
            w = PB[kk][nb][(e % 8) // 2]
            def dl(x):       # a deadline; past the MFMA stream: the tail
                return x if x <= nm - 2 else None
            cvt[i] = add(V("v_cvt_pk_bf16_f32", w, tmp[(e - 1) % 24], t),
                         lo, dl(lo + 6), [(exp[e - 1], TRANS_FWD), (exp[e], TRANS_FWD)])
            unp = [add(V("v_lshlrev_b32", tmp[(e - 1) % 24], 16, w), lo, dl(lo + 8), [(cvt[i], 0)]),
                   add(V("v_and_b32", t, MASKHI, w), lo, dl(lo + 8), [(cvt[i], 0)])]
            for ee, un in ((e - 1, unp[0]), (e, unp[1])):
                acc = PSUM[nb][ee % 2]
                init = kk == 0 and ee % 8 < 2
                deps = [(un, 0)]
                if not init:
                    prev_same = max(j for j in adds if (j // 8) % 2 == nb and j % 2 == ee % 2)
                    deps.append((adds[prev_same], 0))
                adds[ee] = add(V("v_add_f32", acc, 0 if init else acc, tmp[ee % 24]), lo, dl(lo + 10), deps)
        last0 = [adds[e] for e in range(64) if (e // 8) % 2 == 0]
        last1 = [adds[e] for e in range(64) if (e // 8) % 2 == 1]
        s0 = add(V("v_add_f32", PSUM[0][0], PSUM[0][0], PSUM[0][1]), 0, None, [(a_, 0) for a_ in last0])
        c0 = add(V("v_cmp_nle_f32", CMPA, PSUM[0][0], BOUND), 0, None, [(s0, 0)])
        s1 = add(V("v_add_f32", PSUM[1][0], PSUM[1][0], PSUM[1][1]), 0, None, [(a_, 0) for a_ in last1])
        c1 = add(V("v_cmp_nle_f32", CMPB, PSUM[1][0], BOUND), 0, None, [(s1, 0)])
        add([S("s_or_b64", CMPA, CMPA, CMPB), CBR("s_cbranch_scc1", self.L(f"redo_s{p}")),
             V("v_add_f32", LRUN[0], LRUN[0], PSUM[0][0]), V("v_add_f32", LRUN[1], LRUN[1], PSUM[1][0]),
             LABEL(self.L(f"ret_s{u}"))], 0, None, [(c0, VALU_SGPR_VMEM), (c1, VALU_SGPR_VMEM)])
        return slot_schedule(mf, items, self.pre_log(), cap=self.caps(mf, GAP_CAP))

    def it_last(self, u):
        """i = wt-1 >= 1 (u = i mod 4): PV(i-1), masked softmax(i) of SACC[u % 2]."""
        p = u % 2
        rel = [8 * kk + 8 for kk in range(4)]
        sm = self.stale_softmax(p, True, rel)
        side = {}
        if not self.causal:
            side[-1] = [S("s_lshl_b32", T[4], ITER, 6), S("s_sub_i32", T[4], KVEND, T[4]),
                        V("v_sub_u32", DREM, T[4], INV["h8"])]
        # the next tile's Q, into QA (the last QK was in the previous
        # iteration): one load every other gap
        for j, b in enumerate(self.q_loads()):
            side.setdefault(2 * j, []).extend(b)
        return self.slot_iter("last", u, True, None, sm, True, side=side,
                                   end_ops=self.tail_stale(self.L(f"redo_l{p}"), self.L(f"ret_l{u}")))

    def it_drain(self, u):
        """i = wt (u = i mod 4): PV(wt-1)."""
        return self.slot_iter("drain", u, True, None, None, False, end_ops=[WAIT(lgkm=0)])

    def it_idle(self):
        """An iteration with no tile of this wave's walk: its share of the loads
        only, slots and resources from ITER (MX: the resources step on from the
        iteration before, as in every other iteration)."""
        if MX:
            t1, t2 = T[1], T[2]
            out = [S("s_and_b32", t1, ITER, 3), S("s_lshl_b32", t1, t1, 14), S("s_add_u32", SKLD, t1, WOFFK),
                   S("s_add_u32", T[5], t1, LDSB), S("s_add_u32", T[5], T[5], 8192),
                   S("s_add_i32", t2, ITER, 2), S("s_and_b32", t2, t2, 3), S("s_lshl_b32", t2, t2, 14),
                   S("s_add_u32", SVLD, t2, WOFF), S("s_add_u32", SVLD, SVLD, LDS_V)]
            dst = {0: SKLD, 2: T[5], 3: SVLD}
            for j, (m0, ld) in enumerate(self.mx_loads(0)):
                if m0 is not None:
                    out += [S("s_mov_b32", M0, dst[j]), NOP(0)]
                out.append(ld)
            for r, step, _ in self.mx_steps():
                out += [x for b in rsrc_step(r, step) for x in b]
            return out
        t1, t2, t3 = T[1], T[2], T[3]
        out = [S("s_and_b32", t1, ITER, 3), S("s_lshl_b32", t1, t1, 14), S("s_add_u32", SKLD, t1, WOFF),
               S("s_add_i32", t2, ITER, 2), S("s_and_b32", t2, t2, 3), S("s_lshl_b32", t2, t2, 14),
               S("s_add_u32", SVLD, t2, WOFF), S("s_add_u32", SVLD, SVLD, LDS_V),
               S("s_add_i32", t3, ITER, 4), S("s_lshl_b32", t3, t3, 14)] + rsrc_at(RK, KH, t3, KVB) + [
               S("s_add_i32", t3, ITER, 2), S("s_lshl_b32", t3, t3, 14)] + rsrc_at(RV, VH, t3, KVB)
        for r, base in ((RK, SKLD), (RV, SVLD)):
            for j in range(4):
                out += ([S("s_mov_b32", M0, base), NOP(0)] if j == 0 else []) + [BLOAD_LDS(INV[f"loff{j}"], r, 1024 * j)]
        for r in (RK, RV):
            out += [x for b in rsrc_step(r) for x in b]
        return out

    # ------------------------------------------------------------ output
    # the output registers of a finished tile: the next tile's setup reuses
    # RO and QW0 while this tile's O is still being written out
    INVL = [SCR[0], SCR[1]]

    def output_lse(self):
        """1 / l of the wave's rows into INVL, the LSE stores; then RO and QW0
        copied to ORO, OQW for output_o."""
        out = []
        INVL = self.INVL
        LT = [SCR[2], SCR[3]]
        X = SCR[4]
        out += NOPS(MFMA_WS + 4)
        for nb in range(2 if MX else 0):
            # MX: no LSE output
            out += [V("v_mov_b32", X, LRUN[nb])] + NOPS(PERM_WS) + [
                V("v_permlane32_swap_b32", LRUN[nb], X, perm=True)] + NOPS(PERM_WS) + [
                V("v_add_f32", LT[nb], LRUN[nb], X),
                V("v_rcp_f32", INVL[nb], LT[nb], trans=True), NOP(1),
                V("v_cmp_lt_f32", VCC, 0, LT[nb]), NOP(1), V("v_cndmask_b32", INVL[nb], 0, INVL[nb], VCC)]
        for nb in range(2 if not MX else 0):
            out += [V("v_mov_b32", X, LRUN[nb])] + NOPS(PERM_WS) + [
                V("v_permlane32_swap_b32", LRUN[nb], X, perm=True)] + NOPS(PERM_WS) + [
                V("v_add_f32", LT[nb], LRUN[nb], X),
                V("v_rcp_f32", INVL[nb], LT[nb], trans=True), NOP(1),
                V("v_cmp_lt_f32", VCC, 0, LT[nb]), NOP(1), V("v_cndmask_b32", INVL[nb], 0, INVL[nb], VCC)]
            # LSE = (m + log2 l) ln 2, -inf for an empty row; lanes h = 1 store out of range
            lg = SCR[5]
            out += [V("v_log_f32", lg, LT[nb], trans=True), NOP(1),
                    V("v_add_f32", lg, MRUN[nb], lg), V("v_mul_f32", lg, LN2, lg),
                    V("v_cndmask_b32", lg, NINF, lg, VCC),
                    S("s_lshl_b32", T[0], QW0, 2), S("s_add_u32", T[0], T[0], 128 * nb),
                    V("v_add_u32", SCR[6], T[0], INV["lsel"]),
                    BSTORE("buffer_store_dword", lg, SCR[6], RL)]
            out += NOPS(STORE_DATA)
        out += [S("s_mov_b32", OQW, QW0)] + [S("s_mov_b32", ORO[j], RO[j]) for j in range(4)]
        return out

    def output_o_any(self, tag):
        """output_o; MX: bf16 or fp16 by OUTF16."""
        if not MX:
            return self.output_o(f16=F16)[0]
        L = lambda n: self.L(f"{n}_{tag}")
        return ([S("s_bitcmp1_b32", OUTF16, 0), CBR("s_cbranch_scc1", L("o16"))] + self.output_o()[0] +
                [BR(L("odone")), LABEL(L("o16"))] + self.output_o(f16=True)[0] + [LABEL(L("odone"))])

    def output_o(self, bundles=(), f16=False):
        """O / l through the wave's LDS staging area to global memory
        (16 buffer_store_dwordx4), from ORO, OQW and INVL; `bundles` (the next
        tile's prologue loads) go one per 4-row block. Returns the program and
        the number of vector-memory operations after the last of the first
        N_EARLY bundles."""
        out = []
        bundles = list(bundles)
        early_end = None
        INVL = self.INVL
        # staging write addresses, chunk c: base + 128 l32 + 8 h + (16 c ^ 16 (l32 & 7))
        stg = T[1]
        out += [S("s_lshl_b32", stg, WAVE, 13), S("s_add_u32", stg, stg, LDSB), S("s_add_u32", stg, stg, LDS_STG)]
        WA = [TMP[2][c] for c in range(8)]
        for c in range(8):
            out += [V("v_xor_b32", WA[c], 16 * c, INV["wx"]), V("v_add3_u32", WA[c], WA[c], INV["wbase"], stg)]
        RDA = SCR[7]
        out += [V("v_add_u32", RDA, stg, INV["rdl"])]
        # global row offsets: (qw0 + 8k) * 256 + lane part; pass p adds 128 bytes
        out += [S("s_lshl_b32", T[2], OQW, 8)]
        VO = [TMP[1][k] for k in range(8)]
        for k in range(8):
            out += [S("s_add_u32", T[3], T[2], 2048 * k) if k else S("s_mov_b32", T[3], T[2]),
                    V("v_add_u32", VO[k], T[3], INV["stl"])]
        for ps in range(2):
            dst = [v(128 + 4 * k, 4) for k in range(8)] if ps == 0 else \
                  [TMP[0].sl(0, 4), TMP[0].sl(4, 4)] + [FRAG[k].sl(0, 4) for k in range(4)] + [
                   SCR.sl(8, 4), SCR.sl(12, 4)]
            for j in range(2):
                ob = 2 * ps + j
                for nb in range(2):
                    for aa in range(4):
                        blk = 16 * ps + 8 * j + 4 * nb + aa
                        if blk < len(bundles):
                            out += bundles[blk]
                            if blk == self.N_EARLY - 1:
                                early_end = len(out)
                        t = [SCR[8 + e] for e in range(4)] if ps == 0 else [v(128 + e + 8 * (aa % 2)) for e in range(4)]
                        o = OACC[ob][nb]
                        out += [ACCR(t[e], o[4 * aa + e]) for e in range(4)]
                        out += [V("v_mul_f32", t[e], INVL[nb], t[e]) for e in range(4)]
                        cvt = "v_cvt_pk_f16_f32" if f16 else "v_cvt_pk_bf16_f32"
                        out += [V(cvt, t[0], t[0], t[1]), V(cvt, t[1], t[2], t[3])]
                        c = 4 * j + aa
                        out += [DSW("ds_write_b64", WA[c], Reg(t[0].f, t[0].i, 2), 4096 * nb)]
            out += [WAIT(lgkm=0)]
            for k in range(8):
                out.append(DSR("ds_read_b128", dst[k], RDA, 1024 * k))
            out += [WAIT(lgkm=0)]
            for k in range(8):
                out.append(BSTORE("buffer_store_dwordx4", dst[k], VO[k], ORO, 128 * ps))
            out += NOPS(STORE_DATA)
        assert len(bundles) <= 32
        n_after = None if early_end is None else sum(1 for x in out[early_end:] if x.kind == "vmem")
        return out, n_after

    # ------------------------------------------------------------ query tile
    def setup_loads(self):
        """Registers of the query tile (BH, QT) and its prologue loads: K(0),
        Q, K(1), K(2), V(0) (32 vector-memory operations)."""
        if MX:
            return self.setup_loads_mx()
        L = self.L
        out = []
        t = T
        # kv head of bh: (bh / Hq) * Hkv + (bh % Hq) / (Hq / Hkv)
        out += div_magic(t[0], BH, MHQ, SHHQ)
        out += [S("s_mul_i32", t[1], t[0], HQ), S("s_sub_u32", t[1], BH, t[1])]
        out += div_magic(t[2], t[1], MRATIO, SHRATIO)
        out += [S("s_mul_i32", t[0], t[0], HKV), S("s_add_u32", t[0], t[0], t[2])]
        out += [S("s_lshl_b32", t[3], SEQ, 8)]                     # bytes per head (S * 256)
        out += [S("s_mul_i32", t[4], t[0], t[3]), S("s_mul_hi_u32", t[5], t[0], t[3]),
                S("s_add_u32", KH[0], KP[0], t[4]), S("s_addc_u32", KH[1], KP[1], t[5]),
                S("s_add_u32", VH[0], VP[0], t[4]), S("s_addc_u32", VH[1], VP[1], t[5])]
        out += [S("s_mul_i32", t[4], BH, t[3]), S("s_mul_hi_u32", t[5], BH, t[3]),
                S("s_add_u32", RQ[0], QP[0], t[4]), S("s_addc_u32", RQ[1], QP[1], t[5]),
                S("s_and_b32", RQ[1], RQ[1], 0xFFFF), S("s_mov_b32", RQ[2], t[3]), S("s_mov_b32", RQ[3], RSRC3),
                S("s_add_u32", RO[0], OP[0], t[4]), S("s_addc_u32", RO[1], OP[1], t[5]),
                S("s_and_b32", RO[1], RO[1], 0xFFFF), S("s_mov_b32", RO[2], t[3]), S("s_mov_b32", RO[3], RSRC3)]
        out += [S("s_lshl_b32", t[6], SEQ, 2), S("s_mul_i32", t[4], BH, t[6]), S("s_mul_hi_u32", t[5], BH, t[6]),
                S("s_add_u32", RL[0], LP[0], t[4]), S("s_addc_u32", RL[1], LP[1], t[5]),
                S("s_and_b32", RL[1], RL[1], 0xFFFF),
                S("s_or_b32", t[7], LP[0], LP[1]), S("s_cmp_eq_u32", t[7], 0),
                S("s_cselect_b32", RL[2], 0, t[6]), S("s_mov_b32", RL[3], RSRC3)]
        # q0, kv_end, tiles, this wave's first row and walk length
        out += [S("s_lshl_b32", Q0, QT, 8), S("s_sub_i32", Q0, Q0, QSHIFT)]
        if self.causal:
            out += [S("s_add_i32", KVEND, Q0, 256), S("s_min_i32", KVEND, KVEND, SEQ)]
        else:
            out += [S("s_mov_b32", KVEND, SEQ)]
        out += [S("s_add_i32", NT, KVEND, 63), S("s_ashr_i32", NT, NT, 6), S("s_lshl_b32", KVB, KVEND, 8),
                S("s_lshl_b32", t[0], WAVE, 6), S("s_add_i32", QW0, Q0, t[0])]
        if self.causal:
            out += [S("s_ashr_i32", t[0], QW0, 6), S("s_add_i32", t[0], t[0], 1), S("s_min_i32", t[0], t[0], NT),
                    S("s_cmp_ge_i32", QW0, 0), S("s_cselect_b32", WT, t[0], 0)]
        else:
            out += [S("s_cmp_ge_i32", QW0, 0), S("s_cselect_b32", WT, NT, 0)]
        # Q offsets of the lane's two rows
        out += [S("s_lshl_b32", t[0], QW0, 8), V("v_add_u32", QOFF[0], t[0], INV["qlane"]),
                V("v_add_u32", QOFF[1], 0x2000, QOFF[0])]
        return out

    def setup_loads_mx(self):
        """MX: the registers of query tile (BH, QT) (no GQA: the K and V head
        is BH): K codes and Q codes 128 bytes per row, V and O 256, K scale
        words 4 (RKS's base; its size is set with K(0)'s loads)."""
        t = T
        out = [S("s_lshl_b32", t[3], SEQ, 8), S("s_lshl_b32", t[6], SEQ, 7)]
        out += [S("s_mul_i32", t[4], BH, t[6]), S("s_mul_hi_u32", t[5], BH, t[6]),
                S("s_add_u32", KH[0], KP[0], t[4]), S("s_addc_u32", KH[1], KP[1], t[5]),
                S("s_add_u32", RQ[0], QP[0], t[4]), S("s_addc_u32", RQ[1], QP[1], t[5]),
                S("s_and_b32", RQ[1], RQ[1], 0xFFFF), S("s_mov_b32", RQ[2], t[6]), S("s_mov_b32", RQ[3], RSRC3)]
        out += [S("s_mul_i32", t[4], BH, t[3]), S("s_mul_hi_u32", t[5], BH, t[3]),
                S("s_add_u32", VH[0], VP[0], t[4]), S("s_addc_u32", VH[1], VP[1], t[5]),
                S("s_add_u32", RO[0], OP[0], t[4]), S("s_addc_u32", RO[1], OP[1], t[5]),
                S("s_and_b32", RO[1], RO[1], 0xFFFF), S("s_mov_b32", RO[2], t[3]), S("s_mov_b32", RO[3], RSRC3)]
        out += [S("s_lshl_b32", t[6], SEQ, 2), S("s_mul_i32", t[4], BH, t[6]), S("s_mul_hi_u32", t[5], BH, t[6]),
                S("s_add_u32", RKS[0], KSP[0], t[4]), S("s_addc_u32", RKS[1], KSP[1], t[5]),
                S("s_and_b32", RKS[1], RKS[1], 0xFFFF), S("s_mov_b32", RKS[3], RSRC3)]
        # q0, kv_end, tiles, this wave's first row and walk length (as bf16)
        out += [S("s_lshl_b32", Q0, QT, 8), S("s_sub_i32", Q0, Q0, QSHIFT)]
        if self.causal:
            out += [S("s_add_i32", KVEND, Q0, 256), S("s_min_i32", KVEND, KVEND, SEQ)]
        else:
            out += [S("s_mov_b32", KVEND, SEQ)]
        out += [S("s_add_i32", NT, KVEND, 63), S("s_ashr_i32", NT, NT, 6), S("s_lshl_b32", KVB, KVEND, 8),
                S("s_lshl_b32", t[0], WAVE, 6), S("s_add_i32", QW0, Q0, t[0])]
        if self.causal:
            out += [S("s_ashr_i32", t[0], QW0, 6), S("s_add_i32", t[0], t[0], 1), S("s_min_i32", t[0], t[0], NT),
                    S("s_cmp_ge_i32", QW0, 0), S("s_cselect_b32", WT, t[0], 0)]
        else:
            out += [S("s_cmp_ge_i32", QW0, 0), S("s_cselect_b32", WT, NT, 0)]
        return out + self.q_offsets_mx(QW0)

    def q_offsets_mx(self, qw):
        """MX: QOFF (codes) and QSO (scale words) of the lane's rows qw + l32
        and qw + 32 + l32 of head BH. The scale rows are clamped into [0, S)
        (a global load has no range check; the codes of rows outside read as
        zeros, so their products are zero)."""
        t = T
        return [S("s_lshl_b32", t[0], qw, 7), V("v_add_u32", QOFF[0], t[0], INV["qlane"]),
                V("v_add_u32", QOFF[1], 0x1000, QOFF[0]),
                V("v_lshrrev_b32", QSO[0], 7, INV["qlane"]), V("v_add_u32", QSO[0], qw, QSO[0]),
                V("v_add_u32", QSO[1], 32, QSO[0]), S("s_sub_i32", t[1], SEQ, 1),
                V("v_med3_i32", QSO[0], QSO[0], 0, t[1]), V("v_med3_i32", QSO[1], QSO[1], 0, t[1]),
                S("s_mul_i32", t[2], BH, SEQ),
                V("v_add_u32", QSO[0], t[2], QSO[0]), V("v_add_u32", QSO[1], t[2], QSO[1]),
                V("v_lshlrev_b32", QSO[0], 2, QSO[0]), V("v_lshlrev_b32", QSO[1], 2, QSO[1])]

    def prologue_loads_mx(self, with_q=True):
        """MX prologue bundles, each ending in one load: K(0) (codes, scale
        words), Q (unless the previous walk loaded it), K(1), K(2), V(0); RK,
        RKS and RV end at the first iteration's tiles (K 3, V 1)."""
        def flat(bl):
            return [x for b in bl for x in b]

        def bundles(lds, pre):
            return [(pre if j == 0 else []) + ([m0, NOP(0)] if m0 is not None else []) + [ld]
                    for j, (m0, ld) in enumerate(lds)]
        k0 = [S("s_mov_b32", RK[0], KH[0]), S("s_and_b32", RK[1], KH[1], 0xFFFF), S("s_lshl_b32", RK[2], KVEND, 7),
              S("s_max_i32", RK[2], RK[2], 0), S("s_mov_b32", RK[3], RSRC3),
              S("s_lshl_b32", RKS[2], KVEND, 2), S("s_max_i32", RKS[2], RKS[2], 0)]
        step = flat(rsrc_step(RK, KTILE)) + flat(rsrc_step(RKS, 256))
        b = bundles(self.mx_loads(0)[:3], k0)
        if with_q:
            b += self.q_loads()
            assert len(b) == self.N_EARLY_MX
        for tl in (1, 2):
            b += bundles(self.mx_loads(tl)[:3], step)
        b += bundles(self.mx_loads(2)[3:], step + rsrc_base(RV, VH, KVB))
        b[-1] += flat(rsrc_step(RV))
        return b

    N_EARLY_MX = 13

    # the prologue loads of K(0) and Q are the first N_EARLY bundles
    N_EARLY = 20

    def prologue_loads(self, with_q=True):
        """The query tile's prologue loads as bundles, each ending in one
        load: K(0), Q (unless the previous walk loaded it), K(1), K(2), V(0);
        the last leaves RK, RV at the first iteration's tiles (K 3, V 1)."""
        if MX:
            return self.prologue_loads_mx(with_q)

        def flat(bl):
            return [x for b in bl for x in b]

        def tile(r, dst, pre):
            return [(pre + [S("s_add_u32", M0, WOFF, dst), NOP(0)] if j == 0 else []) +
                    [BLOAD_LDS(INV[f"loff{j}"], r, 1024 * j)] for j in range(4)]
        b = tile(RK, 0, rsrc_base(RK, KH, KVB))
        if with_q:
            b += self.q_loads()
            assert len(b) == self.N_EARLY
        for tl in (1, 2):
            b += tile(RK, tl * SLOT, flat(rsrc_step(RK)))
        b += tile(RV, LDS_V, flat(rsrc_step(RK)) + rsrc_base(RV, VH, KVB))
        b[-1] += flat(rsrc_step(RV))
        return b

    def q_loads(self):
        """The 16 loads of this wave's 64 Q rows into QA (from RQ, QOFF); MX:
        8 loads of codes into QA_MX, then the rows' 2 scale words."""
        if MX:
            return [[BLOAD("buffer_load_dwordx4", QA_MX[nb][s2].sl(4 * j, 4), QOFF[nb], RQ, 64 * s2 + 32 * j)]
                    for nb in range(2) for s2 in range(2) for j in range(2)] + [
                    [GLOAD("global_load_dword", QSW[nb], QSO[nb], QSP)] for nb in range(2)]
        return [[BLOAD("buffer_load_dwordx4", QA[nb][ks], QOFF[nb], RQ, 32 * ks)] for nb in range(2) for ks in range(8)]

    def q_address(self):
        """RQ and QOFF of query tile (BH, QT) for this wave's rows (MX: and QSO)."""
        t = T
        if MX:
            return [S("s_lshl_b32", t[3], SEQ, 7), S("s_mul_i32", t[4], BH, t[3]), S("s_mul_hi_u32", t[5], BH, t[3]),
                    S("s_add_u32", RQ[0], QP[0], t[4]), S("s_addc_u32", RQ[1], QP[1], t[5]),
                    S("s_and_b32", RQ[1], RQ[1], 0xFFFF), S("s_mov_b32", RQ[2], t[3]), S("s_mov_b32", RQ[3], RSRC3),
                    S("s_lshl_b32", t[3], QT, 8), S("s_sub_i32", t[3], t[3], QSHIFT), S("s_lshl_b32", t[4], WAVE, 6),
                    S("s_add_i32", t[3], t[3], t[4])] + self.q_offsets_mx(t[3])
        return [S("s_lshl_b32", t[3], SEQ, 8), S("s_mul_i32", t[4], BH, t[3]), S("s_mul_hi_u32", t[5], BH, t[3]),
                S("s_add_u32", RQ[0], QP[0], t[4]), S("s_addc_u32", RQ[1], QP[1], t[5]),
                S("s_and_b32", RQ[1], RQ[1], 0xFFFF), S("s_mov_b32", RQ[2], t[3]), S("s_mov_b32", RQ[3], RSRC3),
                S("s_lshl_b32", t[0], QT, 8), S("s_sub_i32", t[0], t[0], QSHIFT), S("s_lshl_b32", t[1], WAVE, 6),
                S("s_add_i32", t[0], t[0], t[1]), S("s_lshl_b32", t[0], t[0], 8),
                V("v_add_u32", QOFF[0], t[0], INV["qlane"]), V("v_add_u32", QOFF[1], 0x2000, QOFF[0])]

    def next_tile(self):
        """At the start of a walk (its prologue loads issued): the next query
        tile into (BH, QT) -- pass 1 of this work item, or pass 0 of the next
        one, decoded here -- and its Q address into RQ, QOFF, so the walk's
        last iteration can load its Q. NXT: bit 0 a next tile exists, bit 1
        it is pass 1. Without one, RQ is empty."""
        L = lambda n: self.L(f"nt_{n}")
        out = [S("s_cmp_eq_u32", PASS, 0), CBR("s_cbranch_scc0", L("item")), S("s_cmp_lt_i32", QT1, 0),
               CBR("s_cbranch_scc1", L("item")), S("s_mov_b32", BH, BH1), S("s_mov_b32", QT, QT1),
               S("s_mov_b32", NXT, 3), BR(L("q"))]
        out += [LABEL(L("item")), S("s_add_u32", ITEMV, ITEMV, GRID), S("s_cmp_ge_u32", ITEMV, NWORK),
                CBR("s_cbranch_scc1", L("none"))]
        out += self.decode("d1") + [S("s_mov_b32", BH, BH0), S("s_mov_b32", QT, QT0), S("s_mov_b32", NXT, 1),
                                    BR(L("q"))]
        out += [LABEL(L("none")), S("s_mov_b32", NXT, 0), S("s_mov_b32", RQ[2], 0), BR(L("done"))]
        out += [LABEL(L("q"))] + self.q_address() + [LABEL(L("done"))]
        return out

    def walk(self):
        """The key walk of the query tile, from iteration -1 (the prologue's
        K(0) and Q have landed, and the barrier after them has passed)."""
        L = self.L
        out = [S("s_mov_b32", ITER, -1)]
        if MX:
            # the tile's Q scale bytes (its Q landed before the walk's barrier);
            # for a negative softmax scale (flag bit 1, the kernel then takes
            # |scale|) the Q codes' signs flip: softmax(c Q K^T) with c < 0 is
            # softmax(|c| (-Q) K^T)
            t = TMP[0]
            flip = []
            for j in range(32):
                flip += [ACCR(t[j % 8], a(128 + j)), V("v_xor_b32", t[j % 8], 0x80808080, t[j % 8]),
                         ACCW(a(128 + j), t[j % 8])]
            out = [V("v_perm_b32", QSC, QSW[1], QSW[0], INV["psel"]), S("s_bitcmp1_b32", OUTF16, 1),
                   CBR("s_cbranch_scc0", L("pos"))] + flip + NOPS(VALU_TO_MFMA) + [LABEL(L("pos"))] + out
        out += [S("s_cmp_ge_i32", WT, 1), CBR("s_cbranch_scc0", L("idle_m1"))]
        out += self.it_fill()
        out += [BR(L("it0")), LABEL(L("idle_m1"))] + self.it_idle()
        out += [LABEL(L("it0")), S("s_mov_b32", ITER, 0)] + self.barrier(NLD_IT)
        out += [S("s_cmp_ge_i32", WT, 2), CBR("s_cbranch_scc1", L("first")),
                S("s_cmp_eq_u32", WT, 1), CBR("s_cbranch_scc1", L("first_last"))]
        out += self.it_idle() + [BR(L("it1"))]
        out += [LABEL(L("first"))] + self.it_first() + [BR(L("it1"))]
        # a one-tile walk (wt = 1) goes on to its drain at i = 1
        out += [LABEL(L("first_last"))] + self.it_first_last() + [S("s_mov_b32", ITER, 1), BR(L("drain1"))]
        # i = 1: steady while i < wt - 1, then last (i = wt - 1), drain (i = wt);
        # a copy per i mod 4 of each, chained in walk order
        out += [LABEL(L("it1")), S("s_mov_b32", ITER, 1), S("s_sub_i32", LIM, WT, 1),
                S("s_cmp_lt_i32", ITER, LIM), CBR("s_cbranch_scc1", L("steady1")),
                S("s_cmp_eq_u32", ITER, LIM), CBR("s_cbranch_scc1", L("last1")),
                S("s_cmp_eq_u32", ITER, WT), CBR("s_cbranch_scc1", L("drain1")),
                BR(L("idle_chk"))]
        for u in (1, 2, 3, 0):
            out += [LABEL(L(f"steady{u}"))] + self.it_steady(u)
            out += [S("s_add_i32", ITER, ITER, 1), S("s_cmp_lt_i32", ITER, LIM)]
            if u == 0:
                out += [CBR("s_cbranch_scc1", L("steady1")), BR(L("last1"))]
            else:
                out += [CBR("s_cbranch_scc0", L(f"last{(u + 1) % 4}"))]
        for u in range(4):
            out += [LABEL(L(f"last{u}"))] + self.barrier(NLD_IT) + self.it_last(u)
            out += [S("s_add_i32", ITER, ITER, 1), BR(L(f"drain{(u + 1) % 4}"))]
        for u in range(4):
            # the last iteration's 8 ring loads and 16 Q loads may be in flight
            out += [LABEL(L(f"drain{u}"))] + self.barrier(NLD_IT + NLD_Q) + self.it_drain(u)
            out += [S("s_add_i32", ITER, ITER, 1), BR(L("idle_chk"))]
        out += [LABEL(L("idle_chk")), S("s_cmp_le_i32", ITER, NT), CBR("s_cbranch_scc0", L("walk_end"))]
        out += self.barrier(NLD_IT) + self.it_idle() + [S("s_add_i32", ITER, ITER, 1), BR(L("idle_chk"))]
        out += [LABEL(L("walk_end"))] + [WAIT(vm=0, lgkm=0), BAR()]
        return out

    def decode(self, tag):
        """Work item ITEMV -> (BH0, QT0) and (BH1, QT1) (QT1 = -1: no second
        tile): work = xcd_remap(ITEMV), then prefill_work's pairing."""
        L = lambda n: self.L(f"{n}_{tag}")
        t = T
        out = [S("s_and_b32", t[0], ITEMV, 7), S("s_lshr_b32", t[1], ITEMV, 3), S("s_add_u32", t[2], XQ, 1),
               S("s_mul_i32", t[3], t[0], t[2]), S("s_sub_u32", t[4], t[0], XR), S("s_mul_i32", t[4], t[4], XQ),
               S("s_mul_i32", t[5], XR, t[2]), S("s_add_u32", t[4], t[4], t[5]), S("s_cmp_lt_u32", t[0], XR),
               S("s_cselect_b32", t[3], t[3], t[4]), S("s_add_u32", WORK, t[3], t[1])]
        out += [S("s_cmp_eq_u32", PAIRED, 0), CBR("s_cbranch_scc1", L("unpaired")),
                S("s_cmp_lt_u32", WORK, NFULL), CBR("s_cbranch_scc0", L("pair_tail"))]
        out += div_magic(t[0], WORK, MHALF, SHHALF)
        out += [S("s_mul_i32", t[1], t[0], HALF), S("s_sub_u32", t[1], WORK, t[1]),
                S("s_mov_b32", BH0, t[0]), S("s_mov_b32", BH1, t[0]), S("s_sub_u32", QT0, NQT, 1),
                S("s_sub_u32", QT0, QT0, t[1]), S("s_mov_b32", QT1, t[1]), BR(L("decoded"))]
        out += [LABEL(L("pair_tail")), S("s_sub_u32", t[0], WORK, NFULL), S("s_lshl_b32", BH0, t[0], 1),
                S("s_mov_b32", QT0, HALF), S("s_add_u32", BH1, BH0, 1), S("s_mov_b32", QT1, HALF),
                S("s_cmp_lt_u32", BH1, NBH), CBR("s_cbranch_scc1", L("decoded")), S("s_mov_b32", QT1, -1),
                BR(L("decoded"))]
        out += [LABEL(L("unpaired"))] + div_magic(t[0], WORK, MNQT, SHNQT)
        out += [S("s_mul_i32", t[1], t[0], NQT), S("s_sub_u32", t[1], WORK, t[1]), S("s_mov_b32", BH0, t[0]),
                S("s_sub_u32", QT0, NQT, 1), S("s_sub_u32", QT0, QT0, t[1]), S("s_mov_b32", QT1, -1)]
        out += [LABEL(L("decoded"))]
        return out

    def select(self):
        """(BH, QT) of pass PASS of the work item."""
        return [S("s_cmp_eq_u32", PASS, 0), S("s_cselect_b32", BH, BH0, BH1), S("s_cselect_b32", QT, QT0, QT1)]

    def redo_blocks(self):
        out = []
        for p in (0, 1):
            out += self.redo_block(self.L(f"redo_s{p}"), "ret_s", p, False)
            out += self.redo_block(self.L(f"redo_l{p}"), "ret_l", p, True)
        return out

    def kernel(self):
        L = self.L
        out = [SLOAD("s_load_dwordx16", s(0, 16), INS_["ka"], 0), SLOAD("s_load_dwordx16", s(16, 16), INS_["ka"], 64),
               S("s_mov_b32", ITEMV, INS_["wg"]), S("s_mov_b32", GRID, INS_["ng"]), S("s_mov_b32", WAVE, INS_["wv"]),
               S("s_mov_b32", LDSB, INS_["lb"]), S("s_mov_b32", BOUND, BOUND_F),
               S("s_lshl_b32", WOFF, INS_["wv"], 12), S("s_add_u32", WOFF, WOFF, INS_["lb"]),
               V("v_mov_b32", NINF, 0xFF800000),
               # LDS read bases, fixed for the kernel (the ring slot is the
               # instruction offset; the base is 1 KB aligned, so the XORs on
               # bits 5-7 commute with it)
               V("v_add_u32", KA, INS_["lb"], INV["kofs"]),
               V("v_add_u32", VA[0][0], INS_["lb"], INV["vofs1"]), V("v_add_u32", VA[0][1], INS_["lb"], INV["vofs2"]),
               V("v_add_u32", VA[0][0], LDS_V, VA[0][0]), V("v_add_u32", VA[0][1], LDS_V, VA[0][1])] + [
               V("v_xor_b32", VA[ob][j], 64 * ob, VA[0][j]) for ob in range(1, 4) for j in range(2)] + [
               WAIT(lgkm=0)]
        if MX:
            # after the argument loads (WOFFK takes HKV's slot): this wave's K
            # code rows of a slot, the K read bases of chunk pairs 1..3
            out += [S("s_lshl_b32", WOFFK, INS_["wv"], 11), S("s_add_u32", WOFFK, WOFFK, INS_["lb"]),
                    S("s_mov_b32", MASKHI, 0xFFFF0000)] + [
                V("v_xor_b32", KXM[cp], 32 * cp, KA) for cp in range(1, 4)]
        t = T
        # A tile's walk, then its LSE; the next tile's setup and prologue
        # loads go out before this tile's O is written, so the loads land
        # while the output runs.
        out += [S("s_cmp_ge_u32", ITEMV, NWORK), CBR("s_cbranch_scc1", L("end"))]
        loads = [x for b in self.prologue_loads() for x in b]
        out += self.decode("d0") + [S("s_mov_b32", PASS, 0)] + self.select() + self.setup_loads() + loads
        out += self.barrier(NLD_PRO) + [BR(L("walk"))]
        out += [LABEL(L("walk"))] + self.next_tile() + self.walk()
        out += [S("s_mov_b32", OQW, -1), S("s_cmp_ge_i32", WT, 1), CBR("s_cbranch_scc0", L("lse_done"))]
        out += self.output_lse() + [LABEL(L("lse_done"))]
        # the next tile (BH, QT) was chosen at the walk's start
        out += [S("s_bitcmp1_b32", NXT, 0), CBR("s_cbranch_scc0", L("final")), S("s_lshr_b32", PASS, NXT, 1)]
        out += self.setup_loads()
        out += [S("s_cmp_lt_i32", OQW, 0), CBR("s_cbranch_scc1", L("no_out"))]
        # this wave had rows, so its last iteration loaded the next Q: K(0),
        # K(1), K(2), V(0), then the output's 16 stores; the barrier waits for
        # K(0) (the 12 loads and 16 stores after it may be in flight)
        out += [x for b in self.prologue_loads(False) for x in b] + self.output_o_any("a")
        out += self.barrier(NLD_PRO + 16) + [BR(L("walk"))]
        out += [LABEL(L("no_out"))] + loads + self.barrier(NLD_PRO) + [BR(L("walk"))]
        out += [LABEL(L("final")), S("s_cmp_lt_i32", OQW, 0), CBR("s_cbranch_scc1", L("end"))]
        out += self.output_o_any("b") + [BR(L("end"))]
        out += self.redo_blocks()
        out += [LABEL(L("end")), WAIT(vm=0, lgkm=0)]
        self.prog = out
        return out


_SCC_KEEP = ("s_mov", "s_cselect", "s_mul_i32", "s_mul_hi", "s_nop", "s_waitcnt", "s_barrier", "s_branch",
             "s_cbranch", "s_load", "s_memtime", "s_movk")


def check_scc(prog, name):
    """Each SCC reader's nearest SCC writer before it in program order is its
    producer: s_addc_u32 r[i] after s_add_u32 r[i-1]; a select or conditional
    branch after a compare (s_cmp, s_bitcmp) or s_or_b64 / s_and_b64."""
    writer = None
    for k, x in enumerate(prog):
        if x.kind != "salu" and not (x.kind == "br" and x.cond):
            continue
        op = x.text.split()[0]
        reads = op in ("s_addc_u32", "s_subb_u32") or op.startswith(("s_cselect", "s_cbranch_scc"))
        if reads:
            assert writer is not None, f"{name}: {x.text} with no SCC writer before it"
            wop, wtxt = writer.text.split()[0], writer.text
            if op in ("s_addc_u32", "s_subb_u32"):
                lo = x.defs[0][1] - 1
                ok = wop == {"s_addc_u32": "s_add_u32", "s_subb_u32": "s_sub_u32"}[op] and writer.defs[0] == ("s", lo)
            else:
                ok = wop.startswith(("s_cmp", "s_bitcmp")) or wop in ("s_or_b64", "s_and_b64")
            assert ok, f"{name}: {x.text!r} reads SCC of {wtxt!r} (instruction {k})"
        if not op.startswith(_SCC_KEEP) and x.kind == "salu":
            writer = x


def to_macro(name, prog):
    lines = []
    for ins in prog:
        t = ins.text
        if ins.kind != "label":
            t = "  " + t
        t = t.replace("%[", "\x00").replace("%", "%%").replace("\x00", "%[")
        lines.append(f'  "{t}\\n"')
    return f"#define {name} \\\n" + " \\\n".join(lines) + "\n"


def clobbers():
    regs = [f'"v{i}"' for i in range(N_VGPR_OWN) if i not in CLOB_SKIP_V] + [f'"a{i}"' for i in range(256)]
    regs += [f'"s{i}"' for i in range(N_SGPR_OWN) if i not in (32, 33)]
    regs += ['"vcc"', '"scc"', '"memory"']
    return ", ".join(regs)


def stats(prog):
    from collections import Counter
    c = Counter(i.kind for i in prog)
    return dict(c)


def main(argv):
    """gen_prefill_w64.py [--mx] OUT.inc: the bf16 bodies (CA_PFW64_*) or, with
    --mx, the MXFP8 ones (CA_PFW64MX_*)."""
    mx = "--mx" in argv[1:]
    args = [x for x in argv[1:] if x != "--mx"]
    out_path = args[0] if args else None
    configure(mx)
    pre = "CA_PFW64MX_" if mx else "CA_PFW64_"
    text = ["// Generated by gen_prefill_w64.py: the 64-row prefill kernel bodies. Do not edit.",
            "#pragma once", ""]
    # the 16-bit file holds bf16 (CA_PFW64_BODY_*) and fp16 (CA_PFW64_F16_BODY_*)
    for f16 in ((False, True) if not mx else (False,)):
        configure_f16(f16)
        for causal in (True, False):
            g = Gen(causal)
            prog = g.kernel()
            check(prog, g.tag)
            check_scc(prog, g.tag)
            name = pre + ("F16_" if f16 else "") + "BODY_" + ("CAUSAL" if causal else "FULL")
            text.append(to_macro(name, prog))
            print(f"variant {g.tag}: {len(prog)} lines {stats(prog)}", file=sys.stderr)
    configure_f16(False)
    text.append(f"#define {pre}CLOBBERS " + clobbers())
    text.append(f"#define {pre}IN_V {len(IN_V)}")
    src = "\n".join(text) + "\n"
    if out_path:
        with open(out_path, "w") as f:
            f.write(src)
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv))

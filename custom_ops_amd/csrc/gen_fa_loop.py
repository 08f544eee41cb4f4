#!/usr/bin/env python3
"""Generate the gfx950 tile loop of the 64-rows-per-wave attention kernel.

    python custom_ops_amd/csrc/gen_fa_loop.py   # rewrites fa_loop.inc

The loop is emitted as GCN assembly text (one C++ string per element type) that
``fa_fwd.hip`` places in a single inline-asm statement. Writing it out
instruction by instruction fixes two things the compiler does not do for this
loop: a software pipeline across KV tiles inside one wave, and an exact
interleave of matrix-core (MFMA) and vector-ALU work.

Work per wave: 64 query rows as two halves h = 0, 1 of 32 rows; KV tiles of 64
keys. For tile n (S[n % 2] holds its scores u = q·k + mask/scale):

  X(n): MFMA  S[(n+1) % 2] = K(n+1)·Qᵀ          (32 MFMAs, K from LDS)
        VALU  P(n) = exp2(u·c2 - m·c2) -> bf16/fp16, in place in S[n % 2]
  Y(n): MFMA  Oᵀ += Vᵀ(n)·Pᵀ(n)                 (32 MFMAs, V read transposed)
        VALU  row sums of P(n); mask(n+1)/scale added to S[(n+1) % 2];
              row max of tile n+1; lazy rescale decision

so every MFMA of one phase runs under the VALU work of the other tile. Q and O
live in AGPRs (MFMA operands and accumulators); the scores, operand windows and
addresses in VGPRs. K, V and the mask tile arrive by LDS DMA (two stages each),
one workgroup barrier per tile.

Register map (physical, fixed by this generator; fa_fwd.hip binds its operands
to the same registers):
  v[0:63]    S0      (half h: v[32h .. 32h+31], block b: +16b)
  v[64:127]  S1
  v[128:143] K operand window, 4 slots
  v[144:159] V operand window, 4 slots
  v[160:175] mask window: fp16, 2 slots of 8 (two 16-byte LDS reads each);
             bf16, 2 slots of 4 (v160..167) and the mask selectors (v168..175)
  v[176:179] K DMA offsets    v[180:183] V DMA offsets   v[184:191] mask DMA offsets
  v[192:199] K LDS read addresses (per 16-d step)        v[200:203] V read addresses
  v[204:207] mask LDS read addresses
  v208/209 running max (u units) of half 0/1   v210/211 max·c2   v212/213 row sums
  v[214:223] temporaries, v224 -inf, v225..v228 c2, 1/scale, slack, -inf (inputs)
  a[0:63]    Q (half h: a[32h + 4kd .. +3])     a[64:191] O (half h: a[64 + 64h + 16db ..])
  s[80:83] K descriptor, s[84:87] V descriptor, s[88:91] mask descriptor,
  s92 tile counter, s[94:97] ballots
"""
from __future__ import annotations

import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "fa_loop.inc")
BAL_BUDGET = 28        # 64-row bf16 loop: VALU cycles per MFMA in the cost-balanced tile body

D = 128
KD = D // 16          # 16-d steps of QK
DB = D // 32          # 32-d blocks of O
KSTAGE = 16384        # bytes per K (or V) stage: 64 keys x 128 d x 2
MSTAGE = 32768        # bytes per mask stage: 256 rows x 64 keys x 2
# LDS layout: [K stage 0|1][V stage 0|1][mask stage 0|1] = 128 KiB. The region
# bases are folded into the address registers on the C side (ds_read immediate
# offsets are 16-bit), so the offsets below are relative to each region.
K_LDS = V_LDS = M_LDS = 0
LDS_BYTES = 4 * KSTAGE + 2 * MSTAGE

# Register map, set by configure(nh) for one of the two kernels:
#   nh = 2: 4 waves of 64 rows (one wave per SIMD; 512 registers per wave)
#   nh = 1: 8 waves of 32 rows (two waves per SIMD; 256 registers per wave)
# Window bases stay multiples of 4 (MFMA operand tuples).
def configure(nh):
    g = globals()
    g["NH"] = nh
    g["WAVES"] = 8 if nh == 1 else 4
    g["SBUF"] = 32 * nh                  # registers per score buffer
    r = 2 * SBUF
    g["KWIN"] = r; r += 16               # K operand window, 4 slots
    g["VWIN"] = r; r += 16               # V operand window, 4 slots
    g["MWIN"] = r; r += 32 if nh == 2 else 8   # mask window, slots of 4
    g["MSEL"] = r; r += 8                # bf16 mask selectors A_0, A_1
    g["NKL"] = 16 // WAVES               # K (and V) DMA loads per wave per tile
    g["NML"] = 4 * nh                    # mask DMA loads per wave per tile
    g["K_OFF"] = r; r += NKL
    g["V_OFF"] = r; r += NKL
    g["M_OFF"] = r; r += NML
    g["K_RD"] = r; r += 8
    g["V_RD"] = r; r += 4
    g["M_RD"] = r; r += 4
    g["MRUN"] = r; r += nh               # running max (u units) per half
    g["MLOG"] = r; r += nh               # running max · c2
    g["LSUM"] = r; r += nh               # this lane's partial row sums
    # temporaries: widen temp, 16·g, per half: row max, swap temp, threshold;
    # then alpha and a second widen temp
    g["T"] = r; r += 4 + 3 * nh
    g["FIN"] = r; r += 4                 # inputs: c2, 1/scale, slack, -inf
    g["NEGINF"] = FIN + 3                # -inf in a VGPR (v_cndmask reads one of SGPR/VCC)
    g["NVGPR"] = r
    g["QA"] = 0                          # a[0 : 32·nh]   Q
    g["OA"] = 32 * nh                    # a[32·nh : 96·nh] O
    g["NAGPR"] = 96 * nh
    g["WT0"], g["W16G"] = T + 0, T + 1
    g["TMX"], g["TSW"], g["TTH"] = T + 2, T + 2 + nh, T + 2 + 2 * nh   # + h
    g["TAL"], g["WT1"] = T + 2 + 3 * nh, T + 3 + 3 * nh
    # bf16 mask chunks in flight: the mask window plus (idle during PV) K window
    g["MSLOTS"] = [MWIN, MWIN + 4, KWIN, KWIN + 4, KWIN + 8, KWIN + 12][:6 if nh == 2 else 4]
    if nh == 2:     # the balanced body: one slot per chunk (the K window is busy)
        g["MSLOTS"] = [MWIN + 4 * i for i in range(8)]
    g["NSLOT"] = len(MSLOTS)


def S(p, h, b, i):
    """Score register: buffer p, half h, 32-key block b, element i."""
    return 2 * 0 + SBUF * p + 32 * h + 16 * b + i


# required wait states (instructions issued) between producer and consumer,
# as LLVM's hazard recognizer inserts them for gfx950, plus one of margin
W_MFMA_VALU = 13      # 32x32x16 MFMA result -> VALU read/write
W_VALU_MFMA = 3       # VALU write -> MFMA source
W_MFMA_CHAIN = 3      # MFMA result -> the next MFMA accumulating into it
W_TRANS = 2           # v_exp result -> VALU read
W_VCC = 3             # VALU write of VCC -> lane-mask read
W_PERM = 3            # VALU write -> v_permlane32_swap source
W_DOT = 4             # v_dot2 result -> another VALU's read (the same dot's accumulator: none)


class Stream:
    """An instruction list with the wave's issue position and per-VGPR hazard
    bookkeeping: ``need(regs, kind)`` pads with s_nop until the producer of each
    register is far enough back."""

    def __init__(self):
        self.lines = []
        self.pos = 0
        self.ready = {}     # reg -> (position it was written, min distance for VALU readers)

    def emit(self, text, n=1):
        self.lines.append(text)
        self.pos += n

    def nop(self, k):
        while k > 0:
            c = min(k, 8)
            self.emit(f"s_nop {c - 1}", c)
            k -= c

    def wait_for(self, regs, dist_key):
        need = 0
        for r in regs:
            if r in self.ready:
                at, d = self.ready[r]
                dd = d.get(dist_key, 0)
                need = max(need, at + dd - self.pos)
        self.nop(need)

    def wrote(self, regs, **dists):
        for r in regs:
            self.ready[r] = (self.pos, dists)


def vrange(lo, n):
    return list(range(lo, lo + n))


def vreg(r, n=1):
    return f"v{r}" if n == 1 else f"v[{r}:{r + n - 1}]"


def areg(r, n=1):
    return f"a{r}" if n == 1 else f"a[{r}:{r + n - 1}]"


class Load:
    """One LDS read: its text, destination registers and window slot. A slot is
    reused only after every consumer of the previous load in it has issued."""

    def __init__(self, text, dst, slot=None, pre=False):
        # the slot is the destination's first register: loads into the same
        # registers (whichever window they belong to) are ordered by it
        self.text, self.dst, self.slot = text, dst, dst[0]
        self.consumers = 0
        self.used = 0
        self.index = None       # position in the issue order
        # pre: issued (and waited for) before this phase; it only holds its
        # registers until its consumers here have issued
        self.pre = pre


class Phase:
    """Interleave MFMA items with VALU items (and scalar/DMA groups) into one
    stream: after every MFMA, its share of VALU work. All LDS reads of the
    phase issue in first-use order through one queue (at most MAXQ in flight,
    slots recycled); before an instruction that needs a read, s_waitcnt
    lgkmcnt(k) with k = reads issued after it (LDS reads complete in order).

    item = dict(text=..., needs=[Load], src=[regs read], dst=[regs written],
                kind='mfma'|'valu'|'trans'|'perm'|'vcc_write'|'vcc_read'|'raw'|'other')
    """
    MAXQ = 12

    def __init__(self, st, maxq=None):
        self.st = st
        if maxq:
            assert maxq <= 15, "lgkmcnt tracks at most 15 LDS reads"
            self.MAXQ = maxq

    def run(self, mfmas, valus, others=(), valu_lead=0, exact=False, others_span=None):
        """exact: every VALU item carries the MFMA slot it follows (min_mfma,
        -1 = before the first MFMA) and goes exactly there; others_span: the
        scalar/DMA items spread over the first that many MFMAs only."""
        st = self.st
        prog = []
        valus, others = list(valus), list(others)
        nm = len(mfmas)
        per = (len(valus) - valu_lead + nm - 1) // nm if nm else 0
        if exact:
            per, valu_lead = len(valus), len(valus)
        span = min(nm, others_span or nm)
        oper = (len(others) + span - 1) // span if nm else 0
        oi = 0
        vi = 0

        def take_valu(limit_idx, mi):
            # VALU items leave in list order; an item with min_mfma > mi waits
            nonlocal vi
            while vi < limit_idx and valus[vi].get("min_mfma", -1) <= mi:
                prog.append(valus[vi])
                vi += 1

        take_valu(valu_lead, -1)
        for mi, m in enumerate(mfmas):
            deps = m.get("deps", ())
            if deps:   # every VALU item tagged with one of deps goes before this MFMA
                last = max((j for j in range(len(valus)) if valus[j].get("tag") in deps), default=-1)
                take_valu(last + 1, mi - 1)
                assert vi > last, "an MFMA's VALU dependency is held back by min_mfma"
            prog.append(m)
            mine = others[oi:oi + oper]    # one before this slot's VALU share, the rest after
            oi += oper
            prog += mine[:1]
            take_valu(min(len(valus), vi + per), mi)
            prog += mine[1:]
        take_valu(len(valus), nm)
        prog += valus[vi:] + others[oi:]
        # loads in first-use order
        order, seen = [], set()
        for it in prog:
            for ld in it.get("needs", []):
                ld.consumers += 1
                if id(ld) not in seen:
                    seen.add(id(ld))
                    order.append(ld)
        # a load may issue once every earlier load whose destination overlaps
        # its own has been read by all of its consumers
        last_writer = {}
        prev = {}
        for ld in order:
            prev[id(ld)] = {id(last_writer[r]): last_writer[r] for r in ld.dst if r in last_writer}.values()
            for r in ld.dst:
                last_writer[r] = ld
        for ld in order:
            if ld.pre:
                ld.index = -1
        order = [ld for ld in order if not ld.pre]
        issued = 0
        complete = -1           # loads [0..complete] known landed

        def try_issue():
            nonlocal issued
            while issued < len(order) and issued - 1 - complete < self.MAXQ:
                ld = order[issued]
                if any(pv.used < pv.consumers for pv in prev[id(ld)]):
                    return
                ld.index = issued
                st.emit(ld.text)
                issued += 1

        for it in prog:
            try_issue()
            needs = it.get("needs", [])
            if needs:
                last = max(ld.index if ld.index is not None else 10 ** 9 for ld in needs)
                assert last < 10 ** 9, "a needed LDS read could not be issued (slot deadlock)"
                if last > complete:
                    st.emit(f"s_waitcnt lgkmcnt({issued - 1 - last})")
                    complete = last
            emit_item(st, it)
            for ld in needs:
                ld.used += 1
        try_issue()
        assert issued == len(order)


def emit_item(st, v):
    kind = v.get("kind", "valu")
    if kind == "dma":                 # SALU write of M0 -> LDS DMA: one wait state
        if st.lines and st.lines[-1].startswith("s_add_u32 m0"):
            st.emit("s_nop 0")
    if kind in ("other", "m0", "dma"):
        for line, n in v["lines"]:
            st.emit(line, n)
        return
    if kind == "raw":
        # a block that may branch over its body counts, as wait states, only
        # the instructions up to its branch (the body may not execute)
        start, cut = st.pos, None
        for line in v["lines"]:
            st.emit(line)
            if cut is None and line.startswith("s_cbranch"):
                cut = st.pos
        if cut is not None:
            st.pos = cut
        return
    reads = v.get("src", [])
    if kind == "mfma":
        st.wait_for(reads, "mfma")
        st.emit(v["text"])
        st.wrote(v.get("dst", []), valu=W_MFMA_VALU, mfma=W_MFMA_CHAIN)
        return
    if kind == "dot":               # dst is also the accumulator it reads
        acc = v["dst"]
        st.wait_for([r for r in reads if r not in acc], "valu")
        st.wait_for(acc, "dotacc")
        st.emit(v["text"])
        st.wrote(acc, valu=W_DOT, dotacc=0, mfma=W_VALU_MFMA, perm=W_PERM)
        return
    if kind == "vcc_read":
        st.wait_for(["vcc"], "vcc")
    if kind == "perm":
        st.wait_for(reads, "perm")
    st.wait_for(reads, "valu")
    st.emit(v["text"])
    w = v.get("dst", [])
    if kind == "trans":
        st.wrote(w, valu=W_TRANS, mfma=W_VALU_MFMA, perm=W_PERM)
    elif kind == "vcc_write":
        st.wrote(["vcc"], vcc=W_VCC)
    else:
        st.wrote(w, valu=0, mfma=W_VALU_MFMA, perm=W_PERM)


def interleave(a, b):
    """Merge two ordered lists, alternating by their relative lengths."""
    out, i, j = [], 0, 0
    while i < len(a) or j < len(b):
        if j >= len(b) or (i < len(a) and i * len(b) <= j * len(a)):
            out.append(a[i]); i += 1
        else:
            out.append(b[j]); j += 1
    return out


def valu(text, reads=(), writes=(), kind="valu", needs=()):
    return {"text": text, "src": list(reads), "dst": list(writes), "kind": kind,
            "needs": list(needs)}


def other(group):
    return {"kind": "other", "lines": group}


# ── instruction groups ───────────────────────────────────────────────────────
def mfma_op(bf16):
    return "v_mfma_f32_32x32x16_bf16" if bf16 else "v_mfma_f32_32x32x16_f16"


def qk_mfmas(bf16, kstage_off, s_next):
    """32 MFMAs of S_next = K·Qᵀ for both halves; each K operand (kd, kb) is
    read once and feeds both halves. Chains S_next[h][kb] start from 0."""
    out = []
    slot = 0
    for kd in range(KD):
        for kb in range(2):
            w = KWIN + 4 * (slot % 4)
            off = kstage_off + kb * 32 * D * 2
            ld = Load(f"ds_read_b128 {vreg(w, 4)}, {vreg(K_RD + kd)} offset:{off}", vrange(w, 4),
                      ("k", slot % 4))
            slot += 1
            for h in range(NH):
                dst = S(s_next, h, kb, 0)
                src_c = "0" if kd == 0 else vreg(dst, 16)
                out.append({"kind": "mfma", "needs": [ld],
                            "text": f"{mfma_op(bf16)} {vreg(dst, 16)}, {vreg(w, 4)}, "
                                    f"{areg(QA + 32 * h + 4 * kd, 4)}, {src_c}",
                            "dst": vrange(dst, 16),
                            "src": vrange(w, 4) + (vrange(dst, 16) if kd else [])})
    return out


def pv_mfmas(bf16, vstage_off, s_cur):
    """32 MFMAs of Oᵀ += Vᵀ·Pᵀ for both halves; each transposed V operand
    (key step j, d block db) is read once (two 8-byte transposing reads)."""
    out = []
    slot = 0
    for j in range(4):
        for db in range(DB):
            w = VWIN + 4 * (slot % 4)
            off = vstage_off + ((j // 2) * 32 + (j % 2) * 8) * D * 2
            l0 = Load(f"ds_read_b64_tr_b16 {vreg(w, 2)}, {vreg(V_RD + db)} offset:{off}",
                      vrange(w, 2), ("v", slot % 4, 0))
            l1 = Load(f"ds_read_b64_tr_b16 {vreg(w + 2, 2)}, {vreg(V_RD + db)} offset:{off + 4 * D * 2}",
                      vrange(w + 2, 2), ("v", slot % 4, 1))
            slot += 1
            for h in range(NH):
                pr = S(s_cur, h, 0, 0) + 4 * j      # P of key step j (bf16/fp16 pairs)
                o = OA + 64 * h + 16 * db
                out.append({"kind": "mfma", "needs": [l0, l1], "deps": (f"cvt{j}",),
                            "text": f"{mfma_op(bf16)} {areg(o, 16)}, {vreg(w, 4)}, {vreg(pr, 4)}, "
                                    f"{areg(o, 16)}",
                            "dst": [], "src": vrange(w, 4) + vrange(pr, 4)})
    return out


def exp_only_valus(s_cur, fp32_sum=False):
    """exp2(u·c2 - m·c2) in place, fp32 (converted to P in Y by cvt_valus);
    fp32_sum: the row sums taken from these fp32 values (v_dot2 over the
    packed P would wait on the matrix core, busy with this wave's MFMAs)."""
    out = []
    for grp in range(4):
        for h in range(NH):
            base = S(s_cur, h, 0, 0)
            regs = [base + 8 * grp + e for e in range(8)]
            for r in regs:
                out.append(valu(f"v_fma_f32 v{r}, v{r}, %[c2], -v{MLOG + h}", [r, MLOG + h], [r]))
            for r in regs:
                out.append(valu(f"v_exp_f32 v{r}, v{r}", [r], [r], kind="trans"))
            if fp32_sum:
                for r in regs:
                    out.append(valu(f"v_add_f32 v{LSUM + h}, v{LSUM + h}, v{r}", [r, LSUM + h], [LSUM + h]))
    return out


def cvt_valus(bf16, s_cur):
    """Round the exponentials to P pairs in place; key step j of half h lands in
    S(s_cur, h, 0, 0) + 4j .. +3 (tagged cvt{j} for the PV MFMAs of step j)."""
    cvt = "v_cvt_pk_bf16_f32" if bf16 else "v_cvt_pk_f16_f32"
    out = []
    for grp in range(4):
        for h in range(NH):
            base = S(s_cur, h, 0, 0)
            for k in range(4):
                a, b = base + 8 * grp + 2 * k, base + 8 * grp + 2 * k + 1
                dst = base + 4 * grp + k
                it = valu(f"{cvt} v{dst}, v{a}, v{b}", [a, b], [dst])
                it["tag"] = f"cvt{grp}"
                out.append(it)
    return out


def exp_valus(bf16, s_cur, fp32_sum=False):
    """P = exp2(u·c2 - m·c2) rounded to the element type, in place: the P pairs
    of key step j of half h land in S(s_cur, h, 0, 0) + 4j .. +3."""
    cvt = "v_cvt_pk_bf16_f32" if bf16 else "v_cvt_pk_f16_f32"
    out = []
    for grp in range(4):                          # one P operand (8 scores) per half
        for h in range(NH):
            base = S(s_cur, h, 0, 0)
            regs = [base + 8 * grp + e for e in range(8)]
            for r in regs:
                out.append(valu(f"v_fma_f32 v{r}, v{r}, %[c2], -v{MLOG + h}", [r, MLOG + h], [r]))
            for r in regs:
                out.append(valu(f"v_exp_f32 v{r}, v{r}", [r], [r], kind="trans"))
            if fp32_sum:
                # the row sum from the fp32 P, before rounding; v_dot2 over the
                # packed P would run on the matrix core's datapath, which the
                # other wave of the SIMD keeps busy
                for r in regs:
                    out.append(valu(f"v_add_f32 v{LSUM + h}, v{LSUM + h}, v{r}", [r, LSUM + h], [LSUM + h]))
            for k in range(4):
                a, b = regs[2 * k], regs[2 * k + 1]
                dst = base + 4 * grp + k
                out.append(valu(f"{cvt} v{dst}, v{a}, v{b}", [a, b], [dst]))
    return out


def mask_add_valus(bf16, s_next, mstage_off):
    """u += mask·(1/scale) for the next tile, both halves. The 16 mask values of
    (half h, block b) are two 16-byte LDS reads into a window slot of 8."""
    out = []
    for idx, (h, b) in enumerate([(h, b) for h in range(NH) for b in range(2)]):
        w = MWIN + 8 * (idx % 2)
        off = mstage_off + h * 4096
        lds = [Load(f"ds_read_b128 {vreg(w + 4 * i, 4)}, {vreg(M_RD + 2 * b + i)} offset:{off}",
                    vrange(w + 4 * i, 4), ("m", idx % 2, i)) for i in range(2)]
        for i in range(2):
            for wd in range(4):
                src = w + 4 * i + wd
                lo = S(s_next, h, b, 8 * i + 2 * wd)
                hi = lo + 1
                nd = [lds[i]]
                if bf16:
                    out.append(valu(f"v_lshlrev_b32 v{WT0}, 16, v{src}", [src], [WT0], needs=nd))
                    out.append(valu(f"v_and_b32 v{WT1}, 0xffff0000, v{src}", [src], [WT1], needs=nd))
                    out.append(valu(f"v_fma_f32 v{lo}, v{WT0}, %[inv_scale], v{lo}", [WT0, lo], [lo]))
                    out.append(valu(f"v_fma_f32 v{hi}, v{WT1}, %[inv_scale], v{hi}", [WT1, hi], [hi]))
                else:
                    out.append(valu(f"v_fma_mix_f32 v{lo}, v{src}, %[inv_scale], v{lo} op_sel_hi:[1,0,0]",
                                    [src, lo], [lo], needs=nd))
                    out.append(valu(f"v_fma_mix_f32 v{hi}, v{src}, %[inv_scale], v{hi} op_sel:[1,0,0] "
                                    f"op_sel_hi:[1,0,0]", [src, hi], [hi], needs=nd))
    return out


def mask_mfma_items(s_next, mstage_off):
    """bf16: u += mask·(1/scale) on the matrix core. The mask chunk of 16 keys
    (half h, block b, chunk c: keys 32b + 16c + 8g .. +7 of this lane's row) is
    the B operand as it sits in LDS; the A operand A_c (v[MSEL + 4c ..]) holds
    bf16(1/scale) where its row's key (π-permuted, as in the score tile) is key
    16c + k of its k index, else 0, so the MFMA adds mask·(1/scale) to exactly
    the matching score. -inf is first clamped to -max_bf16 (v_pk_min_u16; 0 ×
    -inf would be NaN); -max·(1/scale) overflows fp32 back to -inf because
    bf16(1/scale) > 1.0078 (checked on the host). Returns (mfmas, valus)."""
    mf, va = [], []
    slots = MSLOTS
    for idx, (h, b, c) in enumerate([(h, b, c) for h in range(NH) for b in range(2) for c in range(2)]):
        w = slots[idx % len(slots)]
        off = mstage_off + h * 4096
        ld = Load(f"ds_read_b128 {vreg(w, 4)}, {vreg(M_RD + 2 * b + c)} offset:{off}", vrange(w, 4),
                  ("mm", idx % len(slots)))
        tag = f"clamp{idx}"
        for r in range(4):
            it = valu(f"v_pk_min_u16 v{w + r}, v{w + r}, %[mclamp]", [w + r], [w + r], needs=[ld])
            it["tag"] = tag
            va.append(it)
        dst = S(s_next, h, b, 0)
        mf.append({"kind": "mfma", "needs": [ld], "deps": (tag,),   # the slot stays held until here
                   "text": f"v_mfma_f32_32x32x16_bf16 {vreg(dst, 16)}, {vreg(MSEL + 4 * c, 4)}, "
                           f"{vreg(w, 4)}, {vreg(dst, 16)}",
                   "dst": vrange(dst, 16), "src": vrange(w, 4) + vrange(dst, 16)})
    return mf, va


def tail_item(label, s_next, left=1):
    """Keys at or past Sk in the tile being scored -> -inf. Taken only when that
    tile is the last one (s92 == 1) and Sk % 64 != 0 (%[lim] = valid keys < 64).
    Lane (row, half g) owns keys 32b + 16g + i of block b."""
    lines = [f"s_cmp_eq_u32 s92, {left}", f"s_cbranch_scc0 {label}_skip",
             "s_cmp_eq_u32 %[lim], 64", f"s_cbranch_scc1 {label}_skip",
             f"v_sub_u32 v{WT1}, %[lim], v{W16G}"]
    for b in range(2):
        for i in range(16):
            lines += [f"v_cmp_lt_i32 vcc, {32 * b + i}, v{WT1}", "s_nop 2"]
            for h in range(NH):
                r = S(s_next, h, b, i)
                lines.append(f"v_cndmask_b32 v{r}, v{NEGINF}, v{r}, vcc")
    lines += ["s_nop 1", f"{label}_skip:"]
    return {"kind": "raw", "lines": lines}


def max_valus(s_next):
    """Row max of the next tile per half into v(TMX+h) (both 32-lane halves of
    a row combined), then the rescale test: lanes whose max exceeds the running
    max by more than the slack set their bit in s[94:95]."""
    out = []
    for h in range(NH):
        mx = TMX + h
        regs = [S(s_next, h, b, i) for b in range(2) for i in range(16)]
        out.append(valu(f"v_max3_f32 v{mx}, v{regs[0]}, v{regs[1]}, v{regs[2]}", regs[:3], [mx]))
        k = 3
        while k < 32:
            pair = regs[k:k + 2]
            if len(pair) == 2:
                out.append(valu(f"v_max3_f32 v{mx}, v{mx}, v{pair[0]}, v{pair[1]}", [mx] + pair, [mx]))
            else:
                out.append(valu(f"v_max_f32 v{mx}, v{mx}, v{pair[0]}", [mx] + pair, [mx]))
            k += 2
    for h in range(NH):
        mx, tmp = TMX + h, TSW + h
        out.append(valu(f"v_mov_b32 v{tmp}, v{mx}", [mx], [tmp]))
        out.append(valu(f"v_permlane32_swap_b32 v{mx}, v{tmp}", [mx, tmp], [mx, tmp], kind="perm"))
    for h in range(NH):
        mx, tmp, th = TMX + h, TSW + h, TTH + h
        out.append(valu(f"v_max_f32 v{mx}, v{mx}, v{tmp}", [mx, tmp], [mx]))
        out.append(valu(f"v_add_f32 v{th}, %[slack], v{MRUN + h}", [MRUN + h], [th]))
    for h in range(NH):
        mx, th = TMX + h, TTH + h
        out.append(valu(f"v_cmp_gt_f32 vcc, v{mx}, v{th}", [mx, th], [], kind="vcc_write"))
        out.append({"kind": "raw", "lines": [
            "s_nop 2", "s_mov_b64 s[94:95], vcc" if h == 0 else "s_or_b64 s[94:95], s[94:95], vcc"]})
    return out


def rescale_lines(label):
    """Taken when some row's max grew past the slack (rare): per lane alpha =
    exp2((m_old - m_new)·c2) (1 for lanes keeping their max), O and l scaled,
    running max and max·c2 updated. Waits for every PV MFMA first."""
    lines = ["s_cmp_eq_u64 s[94:95], 0", f"s_cbranch_scc1 {label}_skip", "s_nop 7", "s_nop 7"]
    al, tmp = TAL, WT1
    for h in range(NH):
        mx, th = TMX + h, TTH + h
        lines += [
            f"v_cmp_gt_f32 vcc, v{mx}, v{th}",
            f"v_sub_f32 v{al}, v{MRUN + h}, v{mx}",
            f"v_mul_f32 v{al}, %[c2], v{al}",
            f"v_exp_f32 v{al}, v{al}",
            "s_nop 2",
            f"v_cndmask_b32 v{al}, 1.0, v{al}, vcc",
            f"v_cndmask_b32 v{MRUN + h}, v{MRUN + h}, v{mx}, vcc",
            f"v_mul_f32 v{LSUM + h}, v{LSUM + h}, v{al}",
            f"v_mul_f32 v{MLOG + h}, %[c2], v{MRUN + h}",
            f"v_cmp_eq_f32 vcc, %[neginf], v{MRUN + h}",
            "s_nop 2",
            f"v_cndmask_b32_e64 v{MLOG + h}, v{MLOG + h}, 0, vcc",
        ]
        for r in range(64):
            a = OA + 64 * h + r
            lines += [f"v_accvgpr_read_b32 v{tmp}, a{a}", "s_nop 1",
                      f"v_mul_f32 v{tmp}, v{tmp}, v{al}", "s_nop 1",
                      f"v_accvgpr_write_b32 a{a}, v{tmp}"]
    lines += ["s_nop 7", f"{label}_skip:"]
    return lines


def dma_items(stage_k, stage_v, stage_m, do_k, do_v, do_m):
    """LDS DMA of one tile as single-instruction items: per 16-byte-per-lane
    load, the M0 write (LDS destination: lane i lands at M0 + 16·i) and then the
    load, kept at least one instruction apart by emit_item. Each descriptor then
    moves on by one tile: base up, remaining size down, saturating at 0, so a
    load for a tile past the end is out of range (reads nothing, writes no LDS)."""
    items = []

    def one(sl, lds, off, v):
        items.append({"kind": "m0", "lines": [(f"s_add_u32 m0, %[{lds}], {off}", 1)]})
        items.append({"kind": "dma", "lines": [(f"buffer_load_dwordx4 v{v}, s[{sl}:{sl + 3}], 0 offen lds", 1)]})

    def adv(sl, step):
        items.append({"kind": "other", "lines": [
            (f"s_add_u32 s{sl}, s{sl}, {step}", 1), (f"s_addc_u32 s{sl + 1}, s{sl + 1}, 0", 1),
            (f"s_sub_u32 s{sl + 2}, s{sl + 2}, {step}", 1), (f"s_cselect_b32 s{sl + 2}, 0, s{sl + 2}", 1)]})
    if do_k:
        for i in range(NKL):
            one(80, "lds_k", stage_k * KSTAGE + i * WAVES * 1024, K_OFF + i)
        adv(80, "%[kstep]")
    if do_v:
        for i in range(NKL):
            one(84, "lds_v", stage_v * KSTAGE + i * WAVES * 1024, V_OFF + i)
        adv(84, "%[vstep]")
    if do_m:
        for i in range(NML):
            one(88, "lds_m", stage_m * MSTAGE + i * 1024, M_OFF + i)
        adv(88, "128")
    return items


def emit_groups(st, items):
    for it in items:
        emit_item(st, it)


# issue cost (cycles, one wave) of a VALU item when planning slots
def valu_cost(it):
    if it.get("kind") == "raw":
        return 0
    if it.get("kind") == "trans":
        return 8
    if it.get("kind") == "perm":
        return 10
    return 5


def plan_slots(nm, queues, budget):
    """Assign each VALU item the MFMA slot it follows (-1: before the first).
    queues: ordered lists of items, each item optionally with 'earliest' (slot)
    and 'deadline' (the MFMA index it must precede). Slot by slot, the item whose
    queue has the nearest deadline goes first while the slot's cost budget
    lasts; an item past its deadline's last slot goes anyway. Returns the
    items in issue order, each with min_mfma set."""
    qs = [list(q) for q in queues]
    out = []
    for slot in range(-1, nm):
        used = 0
        while True:
            best, key = None, None
            for qi, q in enumerate(qs):
                if not q or q[0].get("earliest", -1) > slot:
                    continue
                # urgency: cost left up to the queue's next deadline per slot left
                k_dl = next((k for k, it in enumerate(q) if "deadline" in it), None)
                dl = q[k_dl]["deadline"] if k_dl is not None else nm
                todo = sum(valu_cost(it) for it in q[:(k_dl + 1) if k_dl is not None else len(q)])
                urg = todo / max(1, dl - slot)
                forced = k_dl is not None and dl - 1 <= slot
                k = (0 if forced else 1, -urg, qi)
                if key is None or k < key:
                    best, key = qi, k
            if best is None:
                break
            it = qs[best][0]
            c = valu_cost(it)
            if used + c > budget and key[0] == 1 and slot < nm - 1:
                break
            qs[best].pop(0)
            it["min_mfma"] = slot
            used += c
            out.append(it)
    for q in qs:
        for it in q:
            it["min_mfma"] = nm - 1
            out.append(it)
    return out


def gen(bf16: bool, nh: int = 2) -> str:
    configure(nh)
    st = Stream()
    L = f"fa_w{32 * NH}_%="
    # entry: Q -> AGPRs, O = 0, running state, 16·g of this lane
    for r in range(32 * NH):
        st.emit(f"v_accvgpr_write_b32 a{QA + r}, v{r}")
    for r in range(64 * NH):
        st.emit(f"v_accvgpr_write_b32 a{OA + r}, 0")
    for h in range(NH):
        st.emit(f"v_mov_b32 v{MRUN + h}, %[neginf]")
        st.emit(f"v_mov_b32 v{MLOG + h}, 0")
        st.emit(f"v_mov_b32 v{LSUM + h}, 0")
    st.emit(f"v_mbcnt_lo_u32_b32 v{W16G}, -1, 0")
    st.emit(f"v_mbcnt_hi_u32_b32 v{W16G}, -1, v{W16G}")
    st.emit(f"v_lshrrev_b32 v{W16G}, 5, v{W16G}")
    st.emit(f"v_lshlrev_b32 v{W16G}, 4, v{W16G}")
    for base, names in ((80, ("klo", "khi", "kn", "fl")), (84, ("vlo", "vhi", "vn", "fl")),
                        (88, ("mlo", "mhi", "mn", "fl"))):
        for i, nm in enumerate(names):
            st.emit(f"s_mov_b32 s{base + i}, %[{nm}]")
    st.emit("s_mov_b32 s92, %[ntiles]")          # tiles left to score, including the next one
    st.nop(4)
    st.ready.clear()

    # prologue: tile nb's K, mask, V into stage 0; nb+1's K and mask into stage 1
    emit_groups(st, dma_items(0, 0, 0, True, True, True))
    emit_groups(st, dma_items(1, 0, 1, True, False, True))
    st.emit("s_waitcnt vmcnt(0)")
    st.emit("s_barrier")
    Phase(st).run(qk_mfmas(bf16, K_LDS, 0), [])
    if bf16:
        mm, clamps = mask_mfma_items(0, M_LDS)
        Phase(st).run(mm, clamps)
        st.nop(W_MFMA_VALU)
        Phase(st).run([], [tail_item(f"{L}_t0", 0)] + max_valus(0))
    else:
        Phase(st).run([], mask_add_valus(bf16, 0, M_LDS) + [tail_item(f"{L}_t0", 0)] + max_valus(0))
    for line in rescale_lines(f"{L}_r0"):
        st.emit(line)
    st.ready.clear()

    def body(p, last):
        nxt = 1 - p
        lab = f"{L}_b{p}{'L' if last else ''}"
        st.emit("s_waitcnt vmcnt(0) lgkmcnt(0)")
        st.emit("s_barrier")
        if last:
            Phase(st).run([], exp_only_valus(p, fp32_sum=True))
            Phase(st).run(pv_mfmas(bf16, V_LDS + p * KSTAGE, p), cvt_valus(bf16, p))
            return
        # tile n+2's K and mask into stage p (out of range past the last tile),
        # tile n+1's V into stage 1-p: single instructions spread over the tile
        others = dma_items(p, nxt, p, True, True, True)
        # One stream per tile: QK(n+1) then PV(n) (with the bf16 mask MFMAs of
        # n+1 between the first PV MFMAs) on the matrix core; exp(n), cvt(n),
        # clamps, row sums, tail and max of n+1 on the VALU. One load queue,
        # so V and mask reads of PV prefetch under the end of QK.
        qk = qk_mfmas(bf16, K_LDS + nxt * KSTAGE, nxt)
        pv = pv_mfmas(bf16, V_LDS + p * KSTAGE, p)
        ex = exp_only_valus(p, fp32_sum=True)
        if bf16 and NH == 2:
            balanced_body(st, qk, pv, ex, others, nxt, lab)
            return
        if bf16:
            mm, clamps = mask_mfma_items(nxt, M_LDS + nxt * MSTAGE)
            mfy = []
            for i, m in enumerate(pv):
                mfy.append(m)
                if i % 2 == 1 and mm:
                    mfy.append(mm.pop(0))
            mfy += mm
            mf = qk + mfy
            mpos = [i for i, m in enumerate(mf) if "clamp" in m.get("deps", ("",))[0]]
            # chunk k shares its window slot with chunk k-NSLOT
            for it in clamps:
                k = int(it["tag"][5:])
                if k >= NSLOT:
                    it["min_mfma"] = mpos[k - NSLOT]
            late = [tail_item(f"{lab}_t", nxt, left=2)] + max_valus(nxt)
            for it in late:
                it["min_mfma"] = mpos[-1]
            vy = interleave(cvt_valus(bf16, p), clamps) + late
        else:
            mf = qk + pv
            late = mask_add_valus(bf16, nxt, M_LDS + nxt * MSTAGE) + \
                [tail_item(f"{lab}_t", nxt, left=2)] + max_valus(nxt)
            for it in late:     # they read the QK results: after the last QK MFMA
                it["min_mfma"] = len(qk) - 1
            vy = cvt_valus(bf16, p) + late
        Phase(st).run(mf, ex + vy, others, valu_lead=8)
        st.emit("s_sub_u32 s92, s92, 1")
        for line in rescale_lines(f"{lab}_r"):
            st.emit(line)
        st.ready.clear()

    def balanced_body(st, qk, pv, ex, others, nxt, lab):
        """MFMAs: QK(n+1) kd 0-3, the mask of n+1, QK(n+1) kd 4-7, PV(n). VALU,
        placed by cost (plan_slots): the mask clamps first (each before its mask
        MFMA), then exp/row sums/conversion of n group by group (conversion j
        before PV step j), the tail and row max of n+1 once S(n+1) is final.
        The tile's DMA issues under the first half of the MFMAs."""
        p = 1 - nxt
        mm, clamps = mask_mfma_items(nxt, M_LDS + nxt * MSTAGE)
        mf = qk[:16] + mm + qk[16:] + pv
        for idx in range(len(mm)):
            for it in clamps[4 * idx:4 * idx + 4]:
                it["deadline"] = 16 + idx
        cv = cvt_valus(bf16, p)
        chain = []
        per_grp = len(ex) // 4
        for j in range(4):
            chain += ex[per_grp * j:per_grp * (j + 1)]
            grp = [it for it in cv if it.get("tag") == f"cvt{j}"]
            for it in grp:
                it["deadline"] = 40 + 8 * j
            chain += grp
        late = [tail_item(f"{lab}_t", nxt, left=2)] + max_valus(nxt)
        for it in late:
            it["earliest"] = 40
        vy = plan_slots(len(mf), [clamps, chain, late], BAL_BUDGET)
        Phase(st).run(mf, vy, others, exact=True, others_span=36)
        st.emit("s_sub_u32 s92, s92, 1")
        for line in rescale_lines(f"{lab}_r"):
            st.emit(line)
        st.ready.clear()

    st.emit(f"{L}_loop:")
    st.emit("s_cmp_le_u32 s92, 1")
    st.emit(f"s_cbranch_scc1 {L}_last0")
    body(0, False)
    st.emit("s_cmp_le_u32 s92, 1")
    st.emit(f"s_cbranch_scc1 {L}_last1")
    body(1, False)
    st.emit(f"s_branch {L}_loop")
    st.emit(f"{L}_last0:")
    body(0, True)
    st.emit(f"s_branch {L}_end")
    st.emit(f"{L}_last1:")
    body(1, True)
    st.emit(f"{L}_end:")
    # O out of the AGPRs once the last PV MFMA has finished
    st.nop(16)
    for r in range(64 * NH):
        st.emit(f"v_accvgpr_read_b32 v{r}, a{OA + r}")
    st.nop(2)
    return "\n".join(st.lines)


# ── ping-pong form (bf16, 8 waves of 32 rows) ────────────────────────────────
# Waves 0-3 (group A) and 4-7 (group B); wave w and w+4 share a SIMD. Every
# wave runs the same phases, B one phase behind A, with one workgroup barrier
# between phases, so while one wave of a SIMD runs an MFMA phase its partner
# runs a VALU phase:
#   M_t: mask MFMAs(t) and QK(t) into S[t % 2], then PV(t-1) from P in S[(t-1) % 2]
#   V_t: tail/max/rescale test of tile t, P(t) = exp2(...) rounded, row sums;
#        reads (and clamps) mask(t+1) and the first K(t+1) operands for M_{t+1}
# LDS: K and V in 3 stages each, the mask in 2 (160 KiB). In M_s group A issues
# K(s+2) and V(s+1) (all K/V DMA of the tile), every wave its own mask rows
# of tile s+2; that batch is waited for at the end of M_{s+1}.
PP_KST = 16384
PP_MST = 32768
PP_VBASE = 3 * PP_KST
PP_MBASE = 6 * PP_KST
PP_LDS = PP_MBASE + 2 * PP_MST      # 160 KiB
PP_KSLOTS = 6         # K operand window slots
PP_VSLOTS = 6         # V (and mask) window slots
PP_MAXQ = 12          # LDS reads in flight
PP_KPRE = 6           # K operands read in the V phase before
PP_DK = (0, 8, 32, 40)               # key offset of K DMA load i (16 rows on, π-permuted)


def configure_pp():
    g = globals()
    g["NH"] = 1
    g["WAVES"] = 8
    g["SBUF"] = 32
    r = 64
    g["KWIN"] = r; r += 4 * PP_KSLOTS
    g["VWIN"] = r; r += 4 * PP_VSLOTS
    g["MSEL"] = r; r += 8
    g["K_RD"] = r; r += 8
    g["V_RD"] = r; r += 4
    g["M_RD"] = r; r += 4
    g["K_OFF"] = r; r += 2           # DMA source offsets of K loads 0, 1 (2, 3: second descriptor)
    g["V_OFF"] = r; r += 2           # V loads 0, 1 (group A; likewise)
    g["M_OFF"] = r; r += 2           # this wave's mask loads 0, 1 (likewise)
    g["MRUN"] = r; r += 1
    g["MLOG"] = r; r += 1
    g["LSUM"] = r; r += 1
    g["T"] = r; r += 6
    g["NEGINF"] = r; r += 1
    g["NVGPR"] = r
    g["QA"] = 0
    g["OA"] = 32
    g["NAGPR"] = 96
    g["W16G"] = T + 0
    g["TMX"], g["TSW"], g["TTH"] = T + 1, T + 2, T + 3
    g["TAL"], g["WT1"] = T + 4, T + 5


def pp_qk_mfmas(kstage, sbuf):
    """16 MFMAs of S += K·Qᵀ (accumulating onto the mask MFMAs' result); the
    first PP_KPRE K operands were read in the V phase before."""
    out = []
    for kd in range(KD):
        for kb in range(2):
            k = 2 * kd + kb
            w = KWIN + 4 * (k % PP_KSLOTS)
            off = kstage * PP_KST + kb * 32 * D * 2
            ld = Load(f"ds_read_b128 {vreg(w, 4)}, {vreg(K_RD + kd)} offset:{off}", vrange(w, 4),
                      pre=k < PP_KPRE)
            dst = S(sbuf, 0, kb, 0)
            out.append({"kind": "mfma", "needs": [ld],
                        "text": f"v_mfma_f32_32x32x16_bf16 {vreg(dst, 16)}, {vreg(w, 4)}, "
                                f"{areg(QA + 4 * kd, 4)}, {vreg(dst, 16)}",
                        "dst": vrange(dst, 16), "src": vrange(w, 4) + vrange(dst, 16)})
    return out


def pp_k_preread(kstage):
    """The first PP_KPRE K operand reads of the next M phase (same registers and
    offsets as pp_qk_mfmas), held by a no-op consumer at the end of the phase."""
    loads = []
    for k in range(PP_KPRE):
        kd, kb = k // 2, k % 2
        w = KWIN + 4 * (k % PP_KSLOTS)
        off = kstage * PP_KST + kb * 32 * D * 2
        loads.append(Load(f"ds_read_b128 {vreg(w, 4)}, {vreg(K_RD + kd)} offset:{off}", vrange(w, 4)))
    return {"kind": "raw", "lines": [], "needs": loads}


PP_MCHUNKS = [(0, 0), (1, 0), (0, 1), (1, 1)]   # (block b, chunk c), issue order


def pp_mask_preread(mstage):
    """mask(t+1) chunks read into the V window and clamped (-inf -> -max_bf16);
    the M phase's mask MFMAs take them from there."""
    out = []
    for idx, (b, c) in enumerate(PP_MCHUNKS):
        w = VWIN + 4 * idx
        ld = Load(f"ds_read_b128 {vreg(w, 4)}, {vreg(M_RD + 2 * b + c)} offset:{mstage * PP_MST}", vrange(w, 4))
        for r in range(4):
            out.append(valu(f"v_pk_min_u16 v{w + r}, v{w + r}, %[mclamp]", [w + r], [w + r], needs=[ld]))
    return out


def pp_mask_mfmas(sbuf):
    out = []
    for idx, (b, c) in enumerate(PP_MCHUNKS):
        w = VWIN + 4 * idx
        ld = Load("", vrange(w, 4), pre=True)
        dst = S(sbuf, 0, b, 0)
        src_c = "0" if c == 0 else vreg(dst, 16)
        out.append({"kind": "mfma", "needs": [ld],
                    "text": f"v_mfma_f32_32x32x16_bf16 {vreg(dst, 16)}, {vreg(MSEL + 4 * c, 4)}, "
                            f"{vreg(w, 4)}, {src_c}",
                    "dst": vrange(dst, 16), "src": vrange(w, 4) + (vrange(dst, 16) if c else [])})
    return out


def pp_pv_mfmas(vstage, sbuf):
    """16 MFMAs of Oᵀ += Vᵀ·Pᵀ, transposed V operands through the V window."""
    out = []
    k = 0
    for j in range(4):
        for db in range(DB):
            # slots 4, 5 first: 0-3 hold the mask chunks until the mask MFMAs
            w = VWIN + 4 * ((k + 4) % PP_VSLOTS)
            off = vstage * PP_KST + ((j // 2) * 32 + (j % 2) * 8) * D * 2
            l0 = Load(f"ds_read_b64_tr_b16 {vreg(w, 2)}, {vreg(V_RD + db)} offset:{off}", vrange(w, 2))
            l1 = Load(f"ds_read_b64_tr_b16 {vreg(w + 2, 2)}, {vreg(V_RD + db)} offset:{off + 4 * D * 2}",
                      vrange(w + 2, 2))
            nd = [l0, l1]
            k += 1
            pr = S(sbuf, 0, 0, 0) + 4 * j
            o = OA + 16 * db
            out.append({"kind": "mfma", "needs": nd,
                        "text": f"v_mfma_f32_32x32x16_bf16 {areg(o, 16)}, {vreg(w, 4)}, {vreg(pr, 4)}, "
                                f"{areg(o, 16)}",
                        "dst": [], "src": vrange(w, 4) + vrange(pr, 4)})
    return out


def pp_dma_items(t_plus2_kstage, t_plus1_vstage, mstage, group_a, parts="kvm"):
    """One M phase's DMA: group A all K(t+2) loads of the workgroup, group B
    all V(t+1) loads (4 each per wave; B's M phase runs one phase after A's,
    and V(t+1) is first read by A's M(t+2), two phases on), every wave its own
    mask rows of tile t+2; parts selects K, V and mask. Every load has its source offset in a register of its own
    (fixed per lane; the descriptor base moves one tile per batch), and its M0
    write is a separate item, so the phase scheduler puts an MFMA between the
    two instead of a wait state. Returns (items, VMEM count)."""
    items, n = [], 0

    def load(desc, lds, ldsoff, voff):
        nonlocal n
        items.append({"kind": "m0", "lines": [(f"s_add_u32 m0, %[{lds}], {ldsoff}", 1)]})
        items.append({"kind": "dma", "lines": [(f"buffer_load_dwordx4 v{voff}, s[{desc}:{desc + 3}], 0 offen lds", 1)]})
        n += 1

    def adv(sl, step):
        items.append({"kind": "other", "lines": [
            (f"s_add_u32 s{sl}, s{sl}, {step}", 1), (f"s_addc_u32 s{sl + 1}, s{sl + 1}, 0", 1),
            (f"s_sub_u32 s{sl + 2}, s{sl + 2}, {step}", 1), (f"s_cselect_b32 s{sl + 2}, 0, s{sl + 2}", 1)]})

    # loads 2 and 3 of each tensor use its second descriptor (s68 K, s72 V,
    # s76 mask), whose base is 32 keys / 32 rows / 16 mask rows on
    if "k" in parts and group_a:
        for i in range(4):
            load(80 if i < 2 else 68, "lds_k", t_plus2_kstage * PP_KST + i * 4096, K_OFF + i % 2)
        adv(80, "%[kstep]")
        adv(68, "%[kstep]")
    if "v" in parts and not group_a:
        for i in range(4):
            load(84 if i < 2 else 72, "lds_v", PP_VBASE + t_plus1_vstage * PP_KST + i * 4096,
                 V_OFF + i % 2)
        adv(84, "%[vstep]")
        adv(72, "%[vstep]")
    if "m" not in parts:
        return items, n
    for i in range(4):
        load(88 if i < 2 else 76, "lds_m", mstage * PP_MST + i * 1024, M_OFF + i % 2)
    adv(88, "128")
    adv(76, "128")
    return items, n


def gen_pp(bf16: bool = True) -> str:
    """The ping-pong tile loop: common entry and prologue, then one code path
    per wave group."""
    assert bf16
    configure_pp()
    st = Stream()
    L = "fa_pp_%="
    # Q straight into its AGPRs (row offset in v[TAL], one 16-d step per
    # immediate offset); these loads land with the prologue's DMA below, so
    # the workgroup waits once for both
    for kd in range(KD):
        st.emit(f"buffer_load_dwordx4 {areg(QA + 4 * kd, 4)}, v{TAL}, s[92:95], 0 offen offset:{kd * 32}")
    for r in range(64):
        st.emit(f"v_accvgpr_write_b32 a{OA + r}, 0")
    st.emit(f"v_mov_b32 v{MRUN}, %[neginf]")
    st.emit(f"v_mov_b32 v{MLOG}, 0")
    st.emit(f"v_mov_b32 v{LSUM}, 0")
    st.emit(f"v_mov_b32 v{NEGINF}, %[neginf]")
    st.emit(f"v_mbcnt_lo_u32_b32 v{W16G}, -1, 0")
    st.emit(f"v_mbcnt_hi_u32_b32 v{W16G}, -1, v{W16G}")
    st.emit(f"v_lshrrev_b32 v{W16G}, 5, v{W16G}")
    st.emit(f"v_lshlrev_b32 v{W16G}, 4, v{W16G}")
    st.emit("s_mov_b32 s92, %[ntiles]")
    st.emit("s_sub_u32 s92, s92, 1")             # tiles after the first
    st.nop(4)
    st.ready.clear()

    # prologue: K(0), V(0), mask(0) into stage 0, K(1), mask(1) into stage 1
    # (K by group A, V by group B), all landed before the common barrier
    st.emit("s_cmp_eq_u32 %[grp], 0")
    st.emit(f"s_cbranch_scc0 {L}_pb")
    pa = []
    for kst in (0, 1):
        it, _ = pp_dma_items(kst, 0, kst, True, parts="kvm" if kst == 0 else "km")
        pa += it
    emit_groups(st, pa)
    st.emit(f"s_branch {L}_pj")
    st.emit(f"{L}_pb:")
    pb = []
    for kst in (0, 1):
        it, _ = pp_dma_items(0, 0, kst, False, parts="vm" if kst == 0 else "m")
        pb += it
    emit_groups(st, pb)
    st.emit(f"{L}_pj:")
    st.emit("s_waitcnt vmcnt(0)")
    st.emit("s_barrier")
    st.emit("s_cmp_eq_u32 %[grp], 0")
    st.emit(f"s_cbranch_scc0 {L}_gb")
    head = list(st.lines)
    ga = pp_group(True, L + "_a")
    gb = pp_group(False, L + "_b")
    return "\n".join(head + ga + [f"s_branch {L}_end", f"{L}_gb:"] + gb + [f"{L}_end:"] + pp_tail())


def pp_tail():
    st = Stream()
    st.nop(16)
    for r in range(64):
        st.emit(f"v_accvgpr_read_b32 v{r}, a{OA + r}")
    st.nop(2)
    return st.lines


def pp_group(group_a, L):
    """One wave group's phases. Group B runs one phase behind group A: it
    passes one extra barrier first, A one extra at the end."""
    st = Stream()

    if not group_a:
        st.emit("s_barrier")
    # operands of M_0: mask(0) clamped, K(0)'s first operands
    Phase(st, PP_MAXQ).run([], pp_mask_preread(0) + [pp_k_preread(0)])

    def m_phase(t, first, last, prev_batch):
        """M_t; t is the tile index mod 6 (stages and buffers)."""
        mf = [] if last else pp_mask_mfmas(t % 2) + pp_qk_mfmas(t % 3, t % 2)
        if not first:
            mf += pp_pv_mfmas((t - 1) % 3, (t - 1) % 2)
        items, n = ([], 0) if last else pp_dma_items((t + 2) % 3, (t + 1) % 3, t % 2, group_a)
        Phase(st, PP_MAXQ).run(mf, [], items)
        # the batch of the previous M phase has landed (LDS DMA: visible to
        # the other waves after the barrier)
        if prev_batch is not None:
            st.emit(f"s_waitcnt vmcnt({n})")
        if not (last and not group_a):
            st.emit("s_barrier")
        return n

    def v_phase(t, lab, last=False):
        vy = [tail_item(f"{lab}_t", t % 2, left=0)] + max_valus(t % 2)
        vy.append({"kind": "raw", "lines": rescale_lines(f"{lab}_r")})
        vy += exp_valus(True, t % 2, fp32_sum=True)
        vy += pp_mask_preread((t + 1) % 2)
        vy += [pp_k_preread((t + 1) % 3)]
        Phase(st, PP_MAXQ).run([], vy)
        st.emit("s_barrier")

    m_phase(0, True, False, None)
    v_phase(0, f"{L}_v0")
    st.emit("s_cmp_eq_u32 s92, 0")
    st.emit(f"s_cbranch_scc1 {L}_f0")
    st.emit(f"{L}_loop:")
    for r in range(1, 7):
        t = r % 6
        m_phase(t, False, False, True)
        st.emit("s_sub_u32 s92, s92, 1")
        v_phase(t, f"{L}_v{r}")
        st.emit("s_cmp_eq_u32 s92, 0")
        st.emit(f"s_cbranch_scc1 {L}_f{t}")
    st.emit(f"s_branch {L}_loop")
    for t in range(6):
        st.emit(f"{L}_f{t}:")
        m_phase((t + 1) % 6, False, True, True)
        st.emit(f"s_branch {L}_x")
    st.emit(f"{L}_x:")
    st.emit("s_waitcnt vmcnt(0)")
    return st.lines


def operand_macros_pp():
    outs = [f'"={{{vreg(16 * i, 16)}}}"(o[{i}])' for i in range(4)]
    outs += [f'"={{v{MRUN}}}"(mrun[0])', f'"={{v{LSUM}}}"(lsum[0])', f'"+{{v{TAL}}}"(qoff)']
    # buffer descriptors bound to their SGPR quads (the loop advances them)
    outs += [f'"+{{s[{b}:{b + 3}]}}"({n})' for b, n in ((80, "kd0"), (68, "kd1"), (84, "vd0"), (72, "vd1"),
                                                         (88, "md0"), (76, "md1"), (92, "qd"))]
    ins = [f'"{{{vreg(K_OFF, 2)}}}"(koff)', f'"{{{vreg(V_OFF, 2)}}}"(voff)',
           f'"{{{vreg(M_OFF, 2)}}}"(moff)', f'"{{{vreg(K_RD, 8)}}}"(krd)', f'"{{{vreg(V_RD, 4)}}}"(vrd)',
           f'"{{{vreg(M_RD, 4)}}}"(mrd)', f'"{{{vreg(MSEL, 8)}}}"(msel)']
    ins += [f'[{n}] "s"({n})' for n in ("mclamp", "c2", "slack", "neginf", "lim", "lds_k", "lds_v", "lds_m",
                                         "kstep", "vstep", "ntiles", "grp")]
    clob = list(range(KWIN, MSEL)) + [MLOG] + [r for r in range(T, NVGPR) if r != TAL]
    cl = [f'"v{r}"' for r in clob] + [f'"a{r}"' for r in range(NAGPR)]
    cl += [f'"s{r}"' for r in range(96, 100)] + ['"m0"', '"vcc"', '"scc"', '"memory"']
    return ["#define MI355_PP_OUTPUTS_BF16 " + ", ".join(outs),
            "#define MI355_PP_INPUTS_BF16 " + ", ".join(ins),
            "#define MI355_PP_CLOBBERS_BF16 " + ", ".join(cl)]


def operand_macros(prefix, bf16):
    """The asm statement's operand lists for one kernel: outputs and inputs
    bound to the physical registers the loop text uses, plus the clobbers."""
    outs = [f'"={{{vreg(16 * i, 16)}}}"(o[{i}])' for i in range(4 * NH)]
    outs += [f'"={{v{MRUN + h}}}"(mrun[{h}])' for h in range(NH)]
    outs += [f'"={{v{LSUM + h}}}"(lsum[{h}])' for h in range(NH)]
    ins = [f'"{{{vreg(32 * h, 32)}}}"(q[{h}])' for h in range(NH)]
    ins += [f'"{{{vreg(K_OFF, NKL)}}}"(koff)', f'"{{{vreg(V_OFF, NKL)}}}"(voff)',
            f'"{{{vreg(M_OFF, NML)}}}"(moff)', f'"{{{vreg(K_RD, 8)}}}"(krd)',
            f'"{{{vreg(V_RD, 4)}}}"(vrd)', f'"{{{vreg(M_RD, 4)}}}"(mrd)']
    if bf16:
        ins += [f'"{{{vreg(MSEL, 8)}}}"(msel)', '[mclamp] "s"(mclamp)']
    ins += [f'[c2] "{{v{FIN}}}"(c2)', f'[inv_scale] "{{v{FIN + 1}}}"(inv_scale)',
            f'[slack] "{{v{FIN + 2}}}"(slack)', f'[neginf] "{{v{FIN + 3}}}"(neginf)']
    ins += [f'[{n}] "s"({n})' for n in ("lim", "lds_k", "lds_v", "lds_m", "kstep", "vstep", "klo", "khi",
                                         "kn", "vlo", "vhi", "vn", "mlo", "mhi", "mn", "fl", "ntiles")]
    clob = list(range(KWIN, MSEL)) + ([] if bf16 else list(range(MSEL, MSEL + 8)))   # the windows
    clob += [MLOG + h for h in range(NH)] + list(range(T, FIN))
    cl = [f'"v{r}"' for r in clob] + [f'"a{r}"' for r in range(NAGPR)]
    cl += [f'"s{r}"' for r in range(80, 98)] + ['"m0"', '"vcc"', '"scc"', '"memory"']
    dt = "BF16" if bf16 else "F16"
    return [f"#define {prefix}_OUTPUTS_{dt} " + ", ".join(outs),
            f"#define {prefix}_INPUTS_{dt} " + ", ".join(ins),
            f"#define {prefix}_CLOBBERS_{dt} " + ", ".join(cl)]


def render() -> str:
    parts = ["// Generated by gen_fa_loop.py -- do not edit.",
             "// Software-pipelined tile loops (gfx950 assembly) of the 32- and 64-rows-per-wave",
             "// kernels, one string per element type, with the operand bindings they assume.",
             "#pragma once"]
    for nh, prefix in ((2, "MI355_W64"), (1, "MI355_W32")):
        for bf16 in (True, False):
            text = gen(bf16, nh)
            dt = "BF16" if bf16 else "F16"
            parts += operand_macros(prefix, bf16)
            parts.append(f"#define {prefix}_LOOP_{dt} \\")
            for line in text.split("\n"):
                parts.append(f'  "{line}\\n\\t" \\')
            parts.append('  ""')
        parts.append(f"// {prefix}: {NVGPR} VGPRs and {NAGPR} AGPRs of the loop's own")
    text = gen_pp(True)
    parts += operand_macros_pp()
    parts.append("#define MI355_PP_LOOP_BF16 \\")
    for line in text.split("\n"):
        parts.append(f'  "{line}\\n\\t" \\')
    parts.append('  ""')
    parts.append(f"// MI355_PP: {NVGPR} VGPRs and {NAGPR} AGPRs of the loop's own")
    return "\n".join(parts) + "\n"


if __name__ == "__main__":
    txt = render()
    if len(sys.argv) > 2 and sys.argv[1] == "--out":
        with open(sys.argv[2], "w") as f:
            f.write(txt)
        sys.exit(0)
    if len(sys.argv) > 1 and sys.argv[1] == "--check":
        with open(OUT) as f:
            sys.exit(0 if f.read() == txt else 1)
    with open(OUT, "w") as f:
        f.write(txt)
    print(OUT, txt.count("\\n"), "lines")

"""Generates fal_bwd_pipe.inc: the query-tile loop of the head_dim-128 dK/dV kernel
(bwd_kv_pipe_kernel) as a single inline-asm block, software-pipelined inside one wave
at one wave per SIMD.

A workgroup owns 128 keys of one KV head; wave w owns keys kw0 = n0 + 32w .. +31 and
keeps their K and V fragments in registers (B operands).  It walks the items (query
head of the GQA group, 64-row query tile) in order.  For item i:
  A(i):  S = Q K^T + Ls and dP = dO V^T + Dn for the 64 rows x 32 keys (32 MFMAs,
         Q/dO fragments from LDS).  The accumulators start at Ls = -L*log2(e)/c and
         Dn = -D, read from LDS, so c*S is the exponent and dP is already dP - D;
  V(i):  P = exp2(c*S) and dS = P*dP (VALU), packed to fp16/bf16 in place;
  B(i):  dV^T += dO^T P and dK^T += Q^T dS (32 MFMAs, dO^T and Q^T from LDS by
         transposed reads), accumulated over every item in AGPRs.
Iteration i runs B(i-1) with the first row block of V(i) between its MFMAs, then one
barrier, then A(i+1) with the second row block of V(i): the MFMA pipe never waits
for the exponentials.

LDS: a ring of 4 item slots of 32 KB (Q tile 16 KB, dO tile 16 KB, SwizzledTile<128>)
and 4 slots of 512 bytes (64 Ls values, 64 Dn values) at 128 KB.  Item F is copied
into slot F % 4 by buffer->LDS loads two iterations ahead; its Q/dO rows past the end
of the sequence read as zeros and its Ls rows there hold the value whose exponent is
-inf, so they add nothing.  After the last item each wave writes dV (fp16/bf16) and
dK * scale to its own pieces of LDS (OSTR apart) for the C++ epilogue.

Causal attention (keys past a row masked): an item whose rows and this wave's keys
straddle the diagonal gets its scores set to `negc` (c * negc = -inf) before V(i).

Register plan (per lane; one wave per SIMD: 256 VGPRs and 256 AGPRs):
  a[0:63], a[64:127]       dV^T and dK^T accumulators, db*16 + i (+64)
  a[192:223], a[224:255]   Q/dO fragment ring (8 x 4), transposed-read ring (8 x 4)
  v[128:191], v[192:255]   item sets (parity of the item): S rb0, S rb1, dP rb0, dP rb1
                           (16 each); P and dS are packed in place into the first 8
                           registers of each 16-register block
  v[112:119]  Q fragment addresses of the slot of item i+1
  v[120:127]  transposed-read addresses of the slot of item i-1
  v104        Ls/Dn read address of the slot of item i+1, v108..v111 temporaries
  s72 caller's m0, s73 iteration i, s74 query tile of the next item to copy,
  s75 query tile of item i, s[76:79]/s[80:83]/s[84:87] Q, dO, Ls/Dn copy resources,
  s[88:89] compare mask, s90..s93 and s95 temporaries, s94 next item to copy
  v0..v103, a128..a191 and s0..s71 are left to the compiler (K and V arrive in AGPRs).

The output is deterministic text, tracked under csrc/gen/; build.py checks the tracked
file against render() and rewrites it only when asked (--regen).
"""

import os
import sys

NBUF = 4
OSTR = 528              # bytes between the hand-off pieces (kKvOStr in fal_bwd.hip)
SLOT = 32768
DOFF = 16384            # dO tile inside a slot
LDOFF = 131072          # Ls/Dn slots
# Knobs (set by configure(); the values here are the product kernel's)
DEFAULTS = {
    "ADIST": 4,    # Q/dO fragment reads ahead of their MFMA
    "BDIST": 6,    # transposed reads ahead (2 per MFMA)
    # measurement builds only (wrong results): comma-separated subset of
    # nodma, nobar, novalu, nolds, nob (no dV/dK products), noa (no S/dP products)
    "ABL": "",
}
ADIST, BDIST = 4, 6
DEFAULT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gen", "fal_bwd_pipe.inc")

SET = (128, 192)
QA = 112
TA = 120
LA = 104
T0, T1, T2, T3 = 108, 109, 110, 111
AR = 192
BR = 224
SM0, SJ, SQF, SQC = 72, 73, 74, 75
SQ, SD, SL = 76, 80, 84
SM = 88
ST0, ST1, ST2, ST3, ST4 = 90, 91, 92, 93, 95
SF = 94
RSRC_W3 = "0x00020000"
MEASURE, ABL = False, set()

# ---- operands: (name, constraint, C++ expression) ----
OUTS = []
INS = []
for t in range(8):
    INS.append((f"K{t}", "a", f"kreg[{t}]"))
for t in range(8):
    INS.append((f"V{t}", "a", f"vreg[{t}]"))
for t in range(8):
    INS.append((f"qa{t}", "v", f"p_qa[{t}]"))
for hf in range(2):
    for db in range(4):
        INS.append((f"ta{hf}{db}", "v", f"p_ta[{hf}][{db}]"))
for i in range(4):
    INS.append((f"qo{i}", "v", f"p_qo[{i}]"))
for i in range(4):
    INS.append((f"do{i}", "v", f"p_do[{i}]"))
INS += [("la", "v", "p_la"), ("lo4", "v", "p_lo4"), ("lo4b", "v", "p_lo4b"), ("lk", "v", "p_lk"),
        ("olds", "v", "p_olds")]
INS += [(n, "s", f"p_{n}") for n in (
    "qb_lo", "qb_hi", "db_lo", "db_hi", "lb_lo", "lb_hi",
    "qs_lo", "qs_hi", "qw_lo", "qw_hi", "ds_lo", "ds_hi", "dw_lo", "dw_hi", "ldw",
    "qrb", "drb", "nq", "nqt", "qt0", "nitems", "c", "negc", "kw0", "lbase", "ldbase", "scale")]
IDX = {name: i for i, (name, _, _) in enumerate(OUTS + INS)}


def op(name):
    return f"%{IDX[name]}"


def v(n):
    return f"v{n}"


def vr(n, k):
    return f"v[{n}:{n + k - 1}]"


def ar(n, k):
    return f"a[{n}:{n + k - 1}]"


class Emitter:
    def __init__(self, bf16):
        self.lines = []
        self.mf = "v_mfma_f32_32x32x16_bf16" if bf16 else "v_mfma_f32_32x32x16_f16"
        self.cvt = "v_cvt_pk_bf16_f32" if bf16 else "v_cvt_pk_f16_f32"
        self.nlabel = 0
        self.skip_mf = False

    def e(self, s):
        self.lines.append(s)

    def es(self, xs):
        for x in xs:
            self.e(x)

    def label(self, name):
        self.nlabel += 1
        return f"{name}{self.nlabel}_%="

    # -- instruction streams ---------------------------------------------------
    def grad_ops(self, par, rb):
        if "novalu" in ABL:
            return []
        return self._grad_ops(par, rb)

    def _grad_ops(self, par, rb):
        """P = exp2(c*S) and dS = P*dP for row block rb of the item in SET[par], then
        both packed in place (pair k of elements 2k, 2k+1 into register k).  Streamed so
        the quarter-rate exponentials spread between the MFMAs: the multiply by c runs
        two elements ahead, dS one element behind its exponential, and a pair is packed
        once both of its dS products are done."""
        s0 = SET[par] + 16 * rb
        d0 = SET[par] + 32 + 16 * rb
        muls = [f"v_mul_f32 {v(s0 + j)}, {op('c')}, {v(s0 + j)}" for j in range(16)]
        ops = muls[:2]
        for st in range(19):
            if st + 2 < 16:
                ops.append(muls[st + 2])
            if st < 16:
                ops.append(f"v_exp_f32 {v(s0 + st)}, {v(s0 + st)}")
            if 0 <= st - 1 < 16:
                j = st - 1
                ops.append(f"v_mul_f32 {v(d0 + j)}, {v(s0 + j)}, {v(d0 + j)}")
            if st >= 3 and (st - 3) % 2 == 0:
                k = (st - 3) // 2
                if k < 8:
                    ops.append(f"{self.cvt} {v(s0 + k)}, {v(s0 + 2 * k)}, {v(s0 + 2 * k + 1)}")
                    ops.append(f"{self.cvt} {v(d0 + k)}, {v(d0 + 2 * k)}, {v(d0 + 2 * k + 1)}")
        return ops

    def a_prod(self, par):
        """A: S and dP of an item into SET[par] from the slot whose addresses are in QA/LA."""
        reads, mf = [], []
        base = SET[par]
        for blk in range(4):                      # S rb0, S rb1, dP rb0, dP rb1
            for g4 in range(4):
                off = (256 if blk >= 2 else 0) + (blk % 2) * 128 + g4 * 32
                reads.append(f"ds_read_b128 {vr(base + 16 * blk + 4 * g4, 4)}, {v(LA)} offset:{off}")
        k = 0
        for t in range(8):
            for blk in range(4):
                rb = blk % 2
                off = (DOFF if blk >= 2 else 0) + rb * 8192
                slot = AR + 4 * (k % 8)
                reads.append(f"ds_read_b128 {ar(slot, 4)}, {v(QA + t)} offset:{off}")
                acc = vr(base + 16 * blk, 16)
                bop = op(f"K{t}") if blk < 2 else op(f"V{t}")
                mf.append((f"{self.mf} {acc}, {ar(slot, 4)}, {bop}, {acc}", 16 + k))
                k += 1
        return reads, mf

    def b_prod(self, par):
        """B: dV^T += dO^T P and dK^T += Q^T dS of the item packed in SET[par], from the
        slot whose transposed-read addresses are in TA."""
        reads, mf = [], []
        base = SET[par]
        k = 0
        for ks in range(4):
            rb, t2 = ks // 2, ks % 2
            for db in range(4):
                for which in range(2):               # dV, dK
                    slot = BR + 4 * (k % 8)
                    off = (DOFF if which == 0 else 0) + ks * 4096
                    for hf in range(2):
                        reads.append(f"ds_read_b64_tr_b16 {ar(slot + 2 * hf, 2)}, {v(TA + hf * 4 + db)} offset:{off}")
                    acc = ar(which * 64 + db * 16, 16)
                    bop = vr(base + (32 if which else 0) + 16 * rb + 4 * t2, 4)
                    mf.append((f"{self.mf} {acc}, {ar(slot, 4)}, {bop}, {acc}", 2 * k + 1))
                    k += 1
        return reads, mf

    @staticmethod
    def cost(ins):
        """Issue cycles of a VALU instruction (wave64; the exponential is quarter rate)."""
        if ins.startswith("v_exp"):
            return 16
        return 4

    def interleave(self, reads, mf, dist, valu=(), groups=()):
        """MFMAs with their LDS reads issued `dist` reads ahead, and the VALU stream and
        instruction groups spread between them (the VALU by issue cycles).  LDS reads
        complete in order, so the wait before an MFMA leaves the later reads in flight."""
        issued = 0
        valu, groups = list(valu), list(groups)
        total = sum(self.cost(x) for x in valu)
        done = 0.0
        for k, (ins, need) in enumerate(mf):
            target = min(len(reads) - 1, need + dist)
            while issued <= target:
                if "nolds" not in ABL:
                    self.e(reads[issued])
                issued += 1
            if "nolds" not in ABL:
                self.e(f"s_waitcnt lgkmcnt({min(issued - need - 1, 15)})")
            if not self.skip_mf:
                self.e(ins)
            if groups:
                self.es(groups.pop(0))
            goal = total * (k + 1) / len(mf)
            while valu and (done < goal or k == len(mf) - 1):
                x = valu.pop(0)
                done += self.cost(x)
                self.e(x)
        assert not valu and not groups and issued == len(reads)

    def slot_addr(self, delta):
        """s90 = ((i + delta) mod 4) * 32 KB, s91 = ((i + delta) mod 4) * 512"""
        return [f"s_add_u32 s{ST0}, s{SJ}, {delta % NBUF}", f"s_and_b32 s{ST0}, s{ST0}, {NBUF - 1}",
                f"s_lshl_b32 s{ST1}, s{ST0}, 9", f"s_lshl_b32 s{ST0}, s{ST0}, 15"]

    def a_addr_ops(self):
        """QA/LA for the slot of item i+1"""
        return (self.slot_addr(1) + [f"v_add_u32 {v(QA + t)}, s{ST0}, {op(f'qa{t}')}" for t in range(8)] +
                [f"v_add_u32 {v(LA)}, s{ST1}, {op('la')}"])

    def b_addr_ops(self):
        """TA for the slot of item i-1"""
        return self.slot_addr(-1) + [f"v_add_u32 {v(TA + hf * 4 + db)}, s{ST0}, {op(f'ta{hf}{db}')}"
                                     for hf in range(2) for db in range(4)]

    def dma_groups(self):
        """Copy of item s94 (query tile s74) into slot s94 % 4: 4 + 4 Q/dO loads of 1 KB
        per wave, the Ls and Dn rows; then the copy state advances one item."""
        g = [[
            # record counts: the tile's rows inside the sequence (0..64) times the row
            # stride; items past the last one copy nothing (read as zeros)
            f"s_lshl_b32 s{ST2}, s{SQF}, 6", f"s_sub_i32 s{ST2}, {op('nq')}, s{ST2}",
            f"s_max_i32 s{ST2}, s{ST2}, 0", f"s_min_i32 s{ST2}, s{ST2}, 64",
            f"s_cmp_lt_i32 s{SF}, {op('nitems')}",
            f"s_cselect_b32 s{ST2}, s{ST2}, 0", f"s_cselect_b32 s{SL + 2}, 0x200, 0",
            f"s_mul_i32 s{SQ + 2}, s{ST2}, {op('qrb')}", f"s_mul_i32 s{SD + 2}, s{ST2}, {op('drb')}",
            f"s_and_b32 s{ST3}, s{SF}, {NBUF - 1}", f"s_lshl_b32 s{ST2}, s{ST3}, 15",
            f"s_add_u32 s{ST2}, s{ST2}, {op('lbase')}",
            f"s_lshl_b32 s{ST3}, s{ST3}, 9", f"s_add_u32 s{ST3}, s{ST3}, {op('ldbase')}"]]
        for part, rs, vo, base in (("q", SQ, "qo", 0), ("d", SD, "do", DOFF)):
            for i in range(4):
                g.append([f"s_add_u32 m0, s{ST2}, {base + i * 4096}", "s_nop 0"] + ([] if "nodma" in ABL else
                          [f"buffer_load_dwordx4 {op(f'{vo}{i}')}, s[{rs}:{rs + 3}], 0 offen lds"]))
        g.append([f"s_mov_b32 m0, s{ST3}", "s_nop 0"] + ([] if "nodma" in ABL else
                 [f"buffer_load_dword {op('lo4')}, s[{SL}:{SL + 3}], 0 offen lds"]))
        g.append([f"s_add_u32 m0, s{ST3}, 256", "s_nop 0"] + ([] if "nodma" in ABL else
                 [f"buffer_load_dword {op('lo4b')}, s[{SL}:{SL + 3}], 0 offen lds"]))
        g.append([
            f"s_add_u32 s{SQF}, s{SQF}, 1", f"s_cmp_eq_u32 s{SQF}, {op('nqt')}",
            f"s_cselect_b32 s{ST0}, {op('qw_lo')}, {op('qs_lo')}", f"s_cselect_b32 s{ST1}, {op('qw_hi')}, {op('qs_hi')}",
            f"s_cselect_b32 s{ST2}, {op('dw_lo')}, {op('ds_lo')}", f"s_cselect_b32 s{ST3}, {op('dw_hi')}, {op('ds_hi')}",
            f"s_cselect_b32 s{ST4}, {op('ldw')}, 0x200", f"s_cselect_b32 s{SQF}, {op('qt0')}, s{SQF}",
            f"s_add_u32 s{SQ}, s{SQ}, s{ST0}", f"s_addc_u32 s{SQ + 1}, s{SQ + 1}, s{ST1}",
            f"s_add_u32 s{SD}, s{SD}, s{ST2}", f"s_addc_u32 s{SD + 1}, s{SD + 1}, s{ST3}",
            f"s_add_u32 s{SL}, s{SL}, s{ST4}", f"s_addc_u32 s{SL + 1}, s{SL + 1}, 0",
            f"s_add_u32 s{SF}, s{SF}, 1"])
        return g

    def dma(self):
        for grp in self.dma_groups():
            self.es(grp)

    # -- blocks ------------------------------------------------------------------
    def mask_block(self, par):
        """Scores of item i (SET[par]) set to negc where key > row, for each row block
        that straddles this wave's keys (kw0 + 31 > first row of the block)."""
        e = self.e
        e(f"s_lshl_b32 s{ST0}, s{SQC}, 6")
        e(f"s_sub_i32 s{ST0}, {op('kw0')}, s{ST0}")              # kw0 - q0
        done = []
        for rb in range(2):
            skip = self.label(f"nomask{rb}_")
            e(f"s_sub_i32 s{ST1}, s{ST0}, {32 * rb}")
            e(f"s_cmp_gt_i32 s{ST1}, -31")
            e(f"s_cbranch_scc0 {skip}")
            e("s_nop 7")
            e(f"v_mov_b32 {v(T3)}, {op('negc')}")
            # element j: key - row = (kw0 - q0 - 32rb + l32 - 4hh) - (8*(j/4) + j%4)
            e(f"v_add_u32 {v(T0)}, s{ST1}, {op('lk')}")
            for j in range(16):
                cst = 8 * (j // 4) + j % 4
                r = SET[par] + 16 * rb + j
                e(f"v_cmp_lt_i32 vcc, {cst}, {v(T0)}")
                e(f"v_cndmask_b32 {v(r)}, {v(r)}, {v(T3)}, vcc")
            e(f"{skip}:")
            done.append(skip)

    def block(self, par, has_b, has_v, has_a, lbl_next):
        e = self.e
        e("s_nop 7")
        e("s_nop 7")
        if has_b:
            self.es(self.b_addr_ops())
        if has_a:
            self.es(self.a_addr_ops())
        v0 = self.grad_ops(par, 0) if has_v else []
        if has_b:
            reads, mf = self.b_prod(par ^ 1)
            self.skip_mf = "nob" in ABL
            self.interleave(reads, mf, BDIST, v0, self.dma_groups())
            self.skip_mf = False
        else:
            self.dma()
            self.es(v0)
        e("s_waitcnt vmcnt(10)")
        if "nobar" not in ABL:
            e("s_barrier")
        v1 = self.grad_ops(par, 1) if has_v else []
        if has_a:
            reads, mf = self.a_prod(par ^ 1)
            self.skip_mf = "noa" in ABL
            self.interleave(reads, mf, ADIST, v1)
            self.skip_mf = False
        else:
            self.es(v1)
        e(f"s_branch {lbl_next}")

    def program(self):
        e = self.e
        lbl_disp, lbl_next, lbl_out = "disp_%=", "next_%=", "out_%="
        e("s_nop 7")
        e(f"s_mov_b32 s{SM0}, m0")
        for rs, lo, hi in ((SQ, "qb_lo", "qb_hi"), (SD, "db_lo", "db_hi"), (SL, "lb_lo", "lb_hi")):
            e(f"s_mov_b32 s{rs}, {op(lo)}")
            e(f"s_mov_b32 s{rs + 1}, {op(hi)}")
            e(f"s_mov_b32 s{rs + 2}, 0")
            e(f"s_mov_b32 s{rs + 3}, {RSRC_W3}")
        e(f"s_mov_b32 s{SJ}, 0")
        e(f"s_mov_b32 s{SF}, 0")
        e(f"s_mov_b32 s{SQF}, {op('qt0')}")
        e(f"s_mov_b32 s{SQC}, {op('qt0')}")
        for a in range(128):
            e(f"v_accvgpr_write_b32 a{a}, 0")
        self.dma()
        self.dma()
        e("s_waitcnt vmcnt(10)")
        e("s_barrier")
        # A(0) into set 0 from slot 0
        e(f"s_mov_b32 s{ST0}, 0")
        e(f"s_mov_b32 s{ST1}, 0")
        self.es([f"v_add_u32 {v(QA + t)}, s{ST0}, {op(f'qa{t}')}" for t in range(8)])
        e(f"v_add_u32 {v(LA)}, s{ST1}, {op('la')}")
        reads, mf = self.a_prod(0)
        self.interleave(reads, mf, ADIST)

        e(f"{lbl_disp}:")
        e(f"s_and_b32 s{ST0}, s{SJ}, 1")
        e(f"s_cmp_eq_u32 s{ST0}, 0")
        e(f"s_cbranch_scc0 disp1_%=")
        for par in (0, 1):
            if par == 1:
                e("disp1_%=:")
            lm = f"nomask_p{par}_%="
            e(f"s_cmp_lt_i32 s{SJ}, {op('nitems')}")
            e(f"s_cbranch_scc0 {lm}")
            e("s_nop 7")
            e("s_nop 7")
            self.mask_block(par)
            e(f"{lm}:")
            lf, lfl, ll, ld = (f"first_p{par}_%=", f"firstlast_p{par}_%=", f"last_p{par}_%=", f"drain_p{par}_%=")
            e(f"s_cmp_eq_u32 s{SJ}, 0")
            e(f"s_cbranch_scc1 {lf}")
            e(f"s_cmp_eq_u32 s{SJ}, {op('nitems')}")
            e(f"s_cbranch_scc1 {ld}")
            e(f"s_add_u32 s{ST0}, s{SJ}, 1")
            e(f"s_cmp_eq_u32 s{ST0}, {op('nitems')}")
            e(f"s_cbranch_scc1 {ll}")
            self.block(par, True, True, True, lbl_next)
            e(f"{ll}:")
            self.block(par, True, True, False, lbl_next)
            e(f"{lf}:")
            e(f"s_add_u32 s{ST0}, s{SJ}, 1")
            e(f"s_cmp_eq_u32 s{ST0}, {op('nitems')}")
            e(f"s_cbranch_scc1 {lfl}")
            self.block(par, False, True, True, lbl_next)
            e(f"{lfl}:")
            self.block(par, False, True, False, lbl_next)
            e(f"{ld}:")
            self.block(par, True, False, False, lbl_next)
        e(f"{lbl_next}:")
        e(f"s_add_u32 s{SQC}, s{SQC}, 1")
        e(f"s_cmp_eq_u32 s{SQC}, {op('nqt')}")
        e(f"s_cselect_b32 s{SQC}, {op('qt0')}, s{SQC}")
        e(f"s_add_u32 s{SJ}, s{SJ}, 1")
        e(f"s_cmp_le_i32 s{SJ}, {op('nitems')}")
        e(f"s_cbranch_scc1 {lbl_disp}")

        e(f"{lbl_out}:")
        # every wave is done with the ring: dV and dK*scale (fp16/bf16) to this wave's
        # LDS, piece (db, g4) of 4 elements at which*16*OSTR + piece*OSTR + lane*8
        e("s_nop 15")
        e("s_nop 15")
        e("s_waitcnt vmcnt(0) lgkmcnt(0)")
        e("s_barrier")
        for which in range(2):
            for db in range(4):
                for g4 in range(4):
                    a0 = which * 64 + db * 16 + 4 * g4
                    for x in range(4):
                        e(f"v_accvgpr_read_b32 {v(T0 + x)}, a{a0 + x}")
                    if which:
                        for x in range(4):
                            e(f"v_mul_f32 {v(T0 + x)}, {op('scale')}, {v(T0 + x)}")
                    e(f"{self.cvt} {v(T0)}, {v(T0)}, {v(T1)}")
                    e(f"{self.cvt} {v(T1)}, {v(T2)}, {v(T3)}")
                    e(f"ds_write_b64 {op('olds')}, {vr(T0, 2)} offset:{which * 16 * OSTR + (db * 4 + g4) * OSTR}")
        e("s_waitcnt lgkmcnt(0)")
        e(f"s_mov_b32 m0, s{SM0}")
        return self.lines



def configure(knobs=None, measure=False):
    """Set the generator's knobs.  `knobs` maps names of DEFAULTS to values; nothing
    is read from the environment.  Ablations (ABL) give wrong results and are refused
    unless `measure` is true."""
    knobs = dict(knobs or {})
    bad = set(knobs) - set(DEFAULTS)
    if bad:
        raise ValueError(f"unknown generator knobs {sorted(bad)}; known: {sorted(DEFAULTS)}")
    cfg = {**DEFAULTS, **knobs}
    if cfg.get("ABL") and not measure:
        raise ValueError("ablation knobs (ABL) give wrong results; they need a measurement build")
    g = globals()
    for k in DEFAULTS:
        g[k] = type(DEFAULTS[k])(cfg[k]) if k != "ABL" else set(x for x in str(cfg[k]).split(",") if x)
    g["MEASURE"] = bool(measure)

def render(knobs=None, measure=False):
    """The generated text for the given knobs (defaults: the product kernel)."""
    configure(knobs, measure)
    try:
        return _render()
    finally:
        configure()


def _render():
    out = ["// Generated by gen_bwd_pipe.py; do not edit.", "#pragma once", ""]
    for bf16, name in ((False, "FAL_BWDP_ASM_F16"), (True, "FAL_BWDP_ASM_BF16")):
        lines = Emitter(bf16).program()
        out.append(f"#define {name} \\")
        for ln in lines:
            out.append(f'  "{ln}\\n" \\')
        out.append("")
    ins = ", ".join(f'"{c}"({x})' for _, c, x in INS)
    clob = ", ".join([f'"v{i}"' for i in range(104, 256)] + [f'"a{i}"' for i in range(0, 128)] +
                     [f'"a{i}"' for i in range(AR, 256)] + [f'"s{i}"' for i in range(72, 100)] +
                     ['"vcc"', '"scc"', '"memory"'])
    out.append("#define FAL_BWDP_OUTS")
    out.append(f"#define FAL_BWDP_INS {ins}")
    out.append(f"#define FAL_BWDP_CLOBBERS {clob}")
    out.append("")
    return "\n".join(out)


def main(path=None):
    """Write the default text to `path` (the tracked file when None)."""
    path = path or DEFAULT_PATH
    with open(path, "w") as f:
        f.write(render())
    return path


if __name__ == "__main__":
    print(main(sys.argv[1] if len(sys.argv) > 1 else None))

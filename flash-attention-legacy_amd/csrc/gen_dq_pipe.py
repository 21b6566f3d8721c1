"""Generates fal_dq_pipe.inc: the key-tile loop of the head_dim-128 dQ kernel
(bwd_dq_kernel with PIPE) as a single inline-asm block, software-pipelined inside one
wave at one wave per SIMD.

A wave owns 32 query rows of one query head; their Q and dO fragments stay in
registers (B operands), with the row's log2-domain LSE (as -L2) and D in one VGPR
each.  K/V tiles of 64 keys stream through LDS.  For tile j:
  A(j):  S^T = K Q^T and dP^T = V dO^T (32 MFMAs, K/V fragments from LDS);
  G(j):  P^T = exp2(c*S^T - L2), dS^T = P^T (dP^T - D) (VALU), dS^T packed to
         fp16/bf16 in place; keys past the row (causal) or past the end are masked;
  Q(j):  dQ^T += K^T dS^T (16 MFMAs, K^T from LDS by transposed reads).
Iteration j runs Q(j-1) with about a third of G(j) (by issue cycles) between its
MFMAs, then one barrier, then A(j+1) with the rest of G(j).  dQ^T stays in AGPRs; after
the last tile each wave writes it to LDS for the C++ epilogue (scale, store).

LDS: a ring of 4 slots of 32 KB (K tile 16 KB, V tile 16 KB, SwizzledTile<128>); tile
t is copied into slot t % 4 by buffer->LDS loads two iterations ahead; one barrier per
iteration publishes tile j+1 and frees the slot of tile j-1.  Waves own different
tile ranges (causal: each wave stops at its diagonal tile; waves whose rows are past
the end have none); every wave runs every iteration's copy and barrier.

Register plan (per lane; one wave per SIMD):
  a[0:63]                 dQ^T accumulators, db*16 + i
  a[192:223], a[224:255]  K/V fragment ring (8 x 4), K^T transposed-read ring (8 x 4)
  v[128:191], v[192:255]  tile sets (parity): S^T kb0, S^T kb1, dP^T kb0, dP^T kb1
                          (16 each); dS^T is packed in place into the first 8
                          registers of each dP^T block
  v[112:119]  K/V fragment addresses of the slot of tile j+1
  v[120:127]  K^T transposed-read addresses of the slot of tile j-1
  v[92:107]   -D (start of the dP^T accumulators), v108..v111 temporaries
  s[84:85] compare mask, s86 caller's m0, s87 rows left from the next tile to copy,
  s[88:91]/s[92:95] K/V copy resources, s96 tile j, s97 next tile to copy,
  s98/s99 temporaries
  v0..v91, a64..a191 and s0..s83 are left to the compiler (Q and dO arrive in AGPRs).

The output is deterministic text, tracked under csrc/gen/; build.py checks the tracked
file against render() and rewrites it only when asked (--regen).
"""

import os
import sys

NBUF = 4
OSTR = 1040             # bytes between the hand-off blocks (kDqOStr in fal_bwd.hip)
VOFF = 16384
# Knobs (set by configure(); the values here are the product kernel's)
DEFAULTS = {
    "ADIST": 4,    # K/V fragment reads ahead of their MFMA
    "QDIST": 6,    # transposed reads ahead (2 per MFMA)
}
ADIST, QDIST = 4, 6
MEASURE = False
DEFAULT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gen", "fal_dq_pipe.inc")

SET = (128, 192)
DN = 92             # v[92:107]: -D in every register (the dP^T accumulators' start)
KC = 112
VC = 120
T0, T1, T2, T3 = 108, 109, 110, 111
AR = 192
BR = 224
SM, SM0, SR = 84, 86, 87
SK, SV = 88, 92
SJ, SD, ST, ST2 = 96, 97, 98, 99
NEG_INF = "0xff800000"

OUTS = []
INS = []
for t in range(8):
    INS.append((f"Q{t}", "a", f"qreg[{t}]"))
for t in range(8):
    INS.append((f"O{t}", "a", f"doreg[{t}]"))
for i in range(4):
    INS.append((f"kvo{i}", "v", f"kvo[{i}]"))
for i in range(4):
    INS.append((f"vvo{i}", "v", f"vvo[{i}]"))
for t in range(8):
    INS.append((f"ka{t}", "v", f"p_ka[{t}]"))
for hf in range(2):
    for db in range(4):
        INS.append((f"ta{hf}{db}", "v", f"p_ta[{hf}][{db}]"))
INS += [("row", "v", "p_row"), ("hh4", "v", "p_hh4"), ("olds", "v", "p_olds"), ("nl", "v", "p_nl"),
        ("dl", "v", "p_dl")]
for i in range(4):
    INS.append((f"kr{i}", "s", f"pk_rs[{i}]"))
for i in range(4):
    INS.append((f"vr{i}", "s", f"pv_rs[{i}]"))
INS += [("c", "s", "p_c"), ("negc", "s", "p_negc"), ("jend", "s", "p_jend"), ("jl", "s", "p_jl"),
        ("wrow", "s", "p_wrow"), ("nk", "s", "p_nk"), ("ktb", "s", "p_ktb"), ("vtb", "s", "p_vtb"),
        ("krb", "s", "p_krb"), ("vrb", "s", "p_vrb"), ("rows", "s", "p_rows"), ("lbase", "s", "p_lbase")]
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

    def e(self, s):
        self.lines.append(s)

    def es(self, xs):
        for x in xs:
            self.e(x)

    # -- instruction streams ---------------------------------------------------
    def grad_ops(self, par, kb):
        """Block kb (32 keys) of tile j in SET[par]: exponent c*S - L2 (FMA), exp2,
        dS = P*(dP - D) (the dP^T accumulator started at -D), dS packed in place (pair k
        into register k).  Streamed so the exponentials spread between the MFMAs: the FMA runs two elements ahead,
        dS one element behind its exponential, a pair is packed after its second dS."""
        s0 = SET[par] + 16 * kb
        d0 = SET[par] + 32 + 16 * kb
        fmas = [f"v_fma_f32 {v(s0 + j)}, {v(s0 + j)}, {op('c')}, {op('nl')}" for j in range(16)]
        ops = fmas[:2]
        for st in range(19):
            if st + 2 < 16:
                ops.append(fmas[st + 2])
            if st < 16:
                ops.append(f"v_exp_f32 {v(s0 + st)}, {v(s0 + st)}")
            if 0 <= st - 1 < 16:
                j = st - 1
                ops.append(f"v_mul_f32 {v(d0 + j)}, {v(s0 + j)}, {v(d0 + j)}")
            if st >= 3 and (st - 3) % 2 == 0 and (st - 3) // 2 < 8:
                k = (st - 3) // 2
                ops.append(f"{self.cvt} {v(d0 + k)}, {v(d0 + 2 * k)}, {v(d0 + 2 * k + 1)}")
        return ops

    def slot(self, dst, delta):
        """dst = ((j + delta) mod NBUF) * 32 KB"""
        return [f"s_add_u32 {dst}, s{SJ}, {delta % NBUF}", f"s_and_b32 {dst}, {dst}, {NBUF - 1}",
                f"s_lshl_b32 {dst}, {dst}, 15"]

    def kcur_ops(self, sreg):
        return [f"v_add_u32 {v(KC + t)}, {sreg}, {op(f'ka{t}')}" for t in range(8)]

    def tcur_ops(self, sreg):
        return [f"v_add_u32 {v(VC + hf * 4 + db)}, {sreg}, {op(f'ta{hf}{db}')}" for hf in range(2) for db in range(4)]

    def dma_groups(self):
        """Copy of tile s97 into its slot (8 buffer->LDS loads), then the copy resources
        advance one tile (rows past the copy range read as zeros)."""
        groups = [[f"s_and_b32 s{ST}, s{SD}, {NBUF - 1}", f"s_lshl_b32 s{ST}, s{ST}, 15",
                   f"s_add_u32 s{ST}, s{ST}, {op('lbase')}",
                   f"s_max_i32 s{SK + 2}, s{SR}, 0", f"s_min_i32 s{SK + 2}, s{SK + 2}, 64",
                   f"s_mul_i32 s{SV + 2}, s{SK + 2}, {op('vrb')}", f"s_mul_i32 s{SK + 2}, s{SK + 2}, {op('krb')}"]]
        for part, rs, vo in (("k", SK, "kvo"), ("v", SV, "vvo")):
            for i in range(4):
                off = i * 4096 + (VOFF if part == "v" else 0)
                groups.append([f"s_add_u32 m0, s{ST}, {off}", "s_nop 0",
                               f"buffer_load_dwordx4 {op(f'{vo}{i}')}, s[{rs}:{rs + 3}], 0 offen lds"])
        groups.append([
            f"s_add_u32 s{SK}, s{SK}, {op('ktb')}", f"s_addc_u32 s{SK + 1}, s{SK + 1}, 0",
            f"s_add_u32 s{SV}, s{SV}, {op('vtb')}", f"s_addc_u32 s{SV + 1}, s{SV + 1}, 0",
            f"s_sub_i32 s{SR}, s{SR}, 64",
            f"s_add_u32 s{SD}, s{SD}, 1"])
        return groups

    def dma(self):
        for g in self.dma_groups():
            self.es(g)

    def a_prod(self, par):
        """S^T = K Q^T and dP^T = V dO^T of the tile whose fragment addresses are in KC,
        into SET[par]."""
        reads, mf = [], []
        k = 0
        for t in range(8):
            for kb in range(2):
                for which in range(2):          # S (K, Q), dP (V, dO)
                    slot = AR + 4 * (k % 8)
                    reads.append(f"ds_read_b128 {ar(slot, 4)}, {v(KC + t)} offset:{(VOFF if which else 0) + kb * 8192}")
                    acc = vr(SET[par] + 32 * which + 16 * kb, 16)
                    c = acc if t else (vr(DN, 16) if which else "0")
                    bop = op(f"O{t}") if which else op(f"Q{t}")
                    mf.append((f"{self.mf} {acc}, {ar(slot, 4)}, {bop}, {c}", k))
                    k += 1
        return reads, mf

    def q_prod(self, par):
        """dQ^T += K^T dS^T of the tile whose dS^T is packed in SET[par], K^T addresses in VC."""
        reads, mf = [], []
        k = 0
        for ks in range(4):
            kb, t2 = ks // 2, ks % 2
            for db in range(4):
                slot = BR + 4 * (k % 8)
                for hf in range(2):
                    reads.append(f"ds_read_b64_tr_b16 {ar(slot + 2 * hf, 2)}, {v(VC + hf * 4 + db)} offset:{ks * 4096}")
                acc = ar(db * 16, 16)
                bop = vr(SET[par] + 32 + 16 * kb + 4 * t2, 4)
                mf.append((f"{self.mf} {acc}, {ar(slot, 4)}, {bop}, {acc}", 2 * k + 1))
                k += 1
        return reads, mf

    @staticmethod
    def cost(ins):
        if ins.startswith("v_exp"):
            return 16
        return 4

    def interleave(self, reads, mf, dist, valu=(), groups=()):
        """MFMAs with their LDS reads issued `dist` reads ahead, the VALU stream and the
        instruction groups spread between them (the VALU by issue cycles)."""
        issued = 0
        valu, groups = list(valu), list(groups)
        total = sum(self.cost(x) for x in valu)
        done = 0.0
        for k, (ins, need) in enumerate(mf):
            target = min(len(reads) - 1, need + dist)
            while issued <= target:
                self.e(reads[issued])
                issued += 1
            self.e(f"s_waitcnt lgkmcnt({min(issued - need - 1, 15)})")
            self.e(ins)
            if groups:
                self.es(groups.pop(0))
            goal = total * (k + 1) / len(mf)
            while valu and (done < goal or k == len(mf) - 1):
                x = valu.pop(0)
                done += self.cost(x)
                self.e(x)
        assert not valu and not groups and issued == len(reads)

    # -- blocks ----------------------------------------------------------------
    def mask_block(self, par, lbl):
        """Raw scores of tile j in SET[par] set to negc (c * negc = -inf) where
        key > row (causal) or key >= nk.  Skipped when no key of the tile can be masked
        for this wave."""
        e = self.e
        e(f"s_lshl_b32 s{ST}, s{SJ}, 6")                  # n0 = j * 64
        e(f"s_add_u32 s{ST2}, s{ST}, 63")
        e(f"s_cmp_gt_i32 s{ST2}, {op('wrow')}")
        e(f"s_cselect_b32 s{SM}, 1, 0")
        e(f"s_cmp_ge_i32 s{ST2}, {op('nk')}")
        e(f"s_cselect_b32 s{SM + 1}, 1, 0")
        e(f"s_or_b32 s{SM}, s{SM}, s{SM + 1}")
        e(f"s_cmp_eq_u32 s{SM}, 0")
        e(f"s_cbranch_scc1 {lbl}")
        e("s_nop 7")
        e("s_nop 7")
        e(f"v_mov_b32 {v(T3)}, {op('negc')}")
        e(f"s_sub_u32 s{ST2}, {op('nk')}, s{ST}")
        e(f"s_sub_u32 s{ST2}, s{ST2}, 1")                 # last valid key of the tile, local
        # thr = min(row - n0, nk - 1 - n0) - hh*4: key kb*32 + c_i (+ hh*4) is kept iff
        # c_i + kb*32 <= thr
        e(f"v_subrev_u32 {v(T0)}, s{ST}, {op('row')}")
        e(f"v_min_i32 {v(T0)}, s{ST2}, {v(T0)}")
        e(f"v_sub_u32 {v(T0)}, {v(T0)}, {op('hh4')}")
        for kb in range(2):
            e(f"v_subrev_u32 {v(T1)}, {kb * 32}, {v(T0)}")
            for i in range(16):
                ci = (i // 4) * 8 + i % 4
                r = SET[par] + kb * 16 + i
                e(f"v_cmp_le_i32 vcc, {ci}, {v(T1)}")
                e(f"v_cndmask_b32 {v(r)}, {v(T3)}, {v(r)}, vcc")
        e(f"{lbl}:")

    def a_simple(self, par):
        """A of tile j (slot in s98) into SET[par], not interleaved (first tile)."""
        self.es(self.kcur_ops(f"s{ST}"))
        reads, mf = self.a_prod(par)
        self.interleave(reads, mf, ADIST)

    def iteration(self, par, has_q, has_a, L):
        """Iteration j with G(j) (scores in SET[par])."""
        e = self.e
        e("s_nop 7")
        e("s_nop 7")
        self.mask_block(par, L("nomask"))
        if has_q:
            self.es(self.slot(f"s{ST}", -1))
            self.es(self.tcur_ops(f"s{ST}"))
        if has_a:
            self.es(self.slot(f"s{ST2}", 1))
            self.es(self.kcur_ops(f"s{ST2}"))
        # the gradient stream of the whole tile, split by issue cycles: about a third
        # beside the 16 dQ products, the rest beside the 32 S/dP products
        gall = self.grad_ops(par, 0) + self.grad_ops(par, 1)
        tot = sum(self.cost(x) for x in gall)
        cut, acc = 0, 0
        if has_q:
            while cut < len(gall) and acc + self.cost(gall[cut]) <= tot / 3:
                acc += self.cost(gall[cut])
                cut += 1
        else:
            cut = len(gall) // 2
        g0, g1 = gall[:cut], gall[cut:]
        if has_q:
            reads, mf = self.q_prod(par ^ 1)
            self.interleave(reads, mf, QDIST, g0, self.dma_groups())
        else:
            self.dma()
            self.es(g0)
        e("s_waitcnt vmcnt(8)")
        e("s_barrier")
        if has_a:
            reads, mf = self.a_prod(par ^ 1)
            self.interleave(reads, mf, ADIST, g1)
        else:
            self.es(g1)
        e(f"s_branch {L('next', shared=True)}")

    def program(self):
        e = self.e
        labels = {}
        counter = [0]

        def L(name, shared=False):
            if shared:
                if name not in labels:
                    labels[name] = f"{name}_%="
                return labels[name]
            counter[0] += 1
            return f"{name}{counter[0]}_%="

        e("s_nop 7")
        e(f"s_mov_b32 s{SM0}, m0")
        for i in range(4):
            e(f"s_mov_b32 s{SK + i}, {op(f'kr{i}')}")
            e(f"s_mov_b32 s{SV + i}, {op(f'vr{i}')}")
        e(f"s_mov_b32 s{SJ}, 0")
        e(f"s_mov_b32 s{SR}, {op('rows')}")
        e(f"s_mov_b32 s{SD}, 0")
        e(f"v_sub_f32 {v(DN)}, 0, {op('dl')}")
        for r in range(DN + 1, DN + 16):
            e(f"v_mov_b32 {v(r)}, {v(DN)}")
        for a in range(64):
            e(f"v_accvgpr_write_b32 a{a}, 0")
        self.dma()
        self.dma()
        e("s_waitcnt vmcnt(8)")
        e("s_barrier")
        # A of the first tile (if this wave has any tile)
        e(f"s_cmp_gt_i32 s{SJ}, {op('jl')}")
        e(f"s_cbranch_scc1 {L('disp', shared=True)}")
        e(f"s_mov_b32 s{ST}, 0")
        self.a_simple(0)

        e(f"{L('disp', shared=True)}:")
        e(f"s_and_b32 s{ST}, s{SJ}, 1")
        e(f"s_cmp_eq_u32 s{ST}, 0")
        e(f"s_cbranch_scc0 {L('disp1', shared=True)}")
        for par in (0, 1):
            if par == 1:
                e(f"{L('disp1', shared=True)}:")
            e(f"s_cmp_gt_i32 s{SJ}, {op('jl')}")
            e(f"s_cbranch_scc1 {L(f'nograd{par}', shared=True)}")
            e(f"s_cmp_eq_u32 s{SJ}, 0")
            e(f"s_cbranch_scc1 {L(f'first{par}', shared=True)}")
            e(f"s_cmp_eq_u32 s{SJ}, {op('jl')}")
            e(f"s_cbranch_scc1 {L(f'last{par}', shared=True)}")
            self.iteration(par, True, True, L)
            e(f"{L(f'last{par}', shared=True)}:")
            self.iteration(par, True, False, L)
            e(f"{L(f'first{par}', shared=True)}:")
            e(f"s_cmp_eq_u32 s{SJ}, {op('jl')}")
            e(f"s_cbranch_scc1 {L(f'firstlast{par}', shared=True)}")
            self.iteration(par, False, True, L)
            e(f"{L(f'firstlast{par}', shared=True)}:")
            self.iteration(par, False, False, L)
            # no gradient: dQ of the wave's last tile (j = jl + 1), or nothing
            e(f"{L(f'nograd{par}', shared=True)}:")
            e(f"s_add_u32 s{ST}, {op('jl')}, 1")
            e(f"s_cmp_eq_u32 s{SJ}, s{ST}")
            e(f"s_cbranch_scc0 {L(f'idle{par}', shared=True)}")
            e(f"s_cmp_gt_i32 s{SJ}, 0")
            e(f"s_cbranch_scc0 {L(f'idle{par}', shared=True)}")
            self.es(self.slot(f"s{ST}", -1))
            self.es(self.tcur_ops(f"s{ST}"))
            reads, mf = self.q_prod(par ^ 1)
            self.interleave(reads, mf, QDIST, (), self.dma_groups())
            e("s_waitcnt vmcnt(8)")
            e("s_barrier")
            e(f"s_branch {L('next', shared=True)}")
            e(f"{L(f'idle{par}', shared=True)}:")
            self.dma()
            e("s_waitcnt vmcnt(8)")
            e("s_barrier")
            e(f"s_branch {L('next', shared=True)}")
        e(f"{L('next', shared=True)}:")
        e(f"s_add_u32 s{SJ}, s{SJ}, 1")
        e(f"s_cmp_lt_i32 s{SJ}, {op('jend')}")
        e(f"s_cbranch_scc1 {L('disp', shared=True)}")
        # ---- after the last iteration (j = jend): dQ of the wave's last tile if it is
        # the workgroup's last tile ----
        e(f"s_add_u32 s{ST}, {op('jl')}, 1")
        e(f"s_cmp_eq_u32 s{SJ}, s{ST}")
        e(f"s_cbranch_scc0 {L('out', shared=True)}")
        e(f"s_cmp_gt_i32 s{SJ}, 0")
        e(f"s_cbranch_scc0 {L('out', shared=True)}")
        e(f"s_and_b32 s{ST}, s{SJ}, 1")
        e(f"s_cmp_eq_u32 s{ST}, 0")
        e(f"s_cbranch_scc0 {L('drain0', shared=True)}")
        for par, lbl in ((1, None), (0, L('drain0', shared=True))):
            # j even: the last tile (j - 1) has odd parity, its dS in SET[1]
            if lbl:
                e(f"{lbl}:")
            e("s_nop 7")
            e("s_nop 7")
            self.es(self.slot(f"s{ST}", -1))
            self.es(self.tcur_ops(f"s{ST}"))
            reads, mf = self.q_prod(par)
            self.interleave(reads, mf, QDIST)
            e(f"s_branch {L('out', shared=True)}")
        e(f"{L('out', shared=True)}:")
        # every wave is done with the ring: dQ^T goes to this wave's 16 blocks of LDS, OSTR apart
        for _ in range(2):
            e("s_nop 15")
        e("s_waitcnt vmcnt(0) lgkmcnt(0)")
        e("s_barrier")
        for g in range(16):
            e(f"ds_write_b128 {op('olds')}, {ar(4 * g, 4)} offset:{g * OSTR}")
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
    out = ["// Generated by gen_dq_pipe.py; do not edit.", "#pragma once", ""]
    for bf16, name in ((False, "FAL_DQP_ASM_F16"), (True, "FAL_DQP_ASM_BF16")):
        lines = Emitter(bf16).program()
        out.append(f"#define {name} \\")
        for ln in lines:
            out.append(f'  "{ln}\\n" \\')
        out.append("")
    ins = ", ".join(f'"{c}"({x})' for _, c, x in INS)
    clob = ", ".join([f'"v{i}"' for i in range(DN, 256)] + [f'"a{i}"' for i in range(0, 64)] +
                     [f'"a{i}"' for i in range(AR, 256)] + [f'"s{i}"' for i in range(84, 100)] +
                     ['"vcc"', '"scc"', '"memory"'])
    out.append("#define FAL_DQP_OUTS")
    out.append(f"#define FAL_DQP_INS {ins}")
    out.append(f"#define FAL_DQP_CLOBBERS {clob}")
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

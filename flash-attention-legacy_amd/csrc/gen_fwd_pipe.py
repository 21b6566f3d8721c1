"""Generates fal_fwd_pipe.inc: the key-tile loop of the head_dim-128 forward kernel
with 64 query rows per wave at one wave per SIMD (fwd_kernel with RB = 2), as a
single inline-asm block.

Why assembly: the loop is software-pipelined inside one wave.  Iteration j runs
  * the PV products of tile j-1 (32 MFMAs, V^T from LDS by transposed reads),
  * the softmax of tile j (about 100 VALU instructions: score FMA, exp2, fp16/bf16
    packing, per-lane row sums), and
  * the S products of tile j+1 (32 MFMAs, K fragments from LDS),
with the softmax instructions placed between the MFMAs, so the MFMA pipe does not wait
for the softmax.  In C++ the compiler sinks the exponentials to their consumers, waits
for every vector-memory operation before LDS reads, and spills around the two score
sets; here every instruction is placed by hand.

Semantics are those of fwd_kernel's C++ tile loop: scores s = q.k, exponent
s * c - m with c = scale * log2(e) and m the row's reference max (log2 domain); m moves
only when a tile's per-lane P sum could leave fp16 range (> 2^15) or the row has no max
yet, and then O and l are rescaled by 2^(m_old - m_new); masked scores (key > row for
causal, key >= nk) are -inf.

LDS: a ring of 4 slots of 32 KB (K tile 16 KB, then V tile 16 KB), XOR-swizzled as
SwizzledTile<128>.  Tile t is copied into slot t % 4 by buffer->LDS loads two
iterations ahead.  One barrier per iteration, after the PV products of tile j-1 and
before the S products of tile j+1: it publishes tile j+1 and frees the slot of tile
j-1.  After the last tile the wave writes its O accumulators to LDS (32 blocks of 1 KB,
OSTR bytes apart, from the `olds` address; the ring is free by then) for the C++
epilogue.

Waves of a workgroup can own different tile ranges (causal: each wave stops at its
diagonal tile); every wave runs every iteration's copy and barrier, and selects the
iteration's work by uniform branches.

Register plan (per lane; one wave per SIMD: 256 VGPRs and 256 AGPRs):
  a[0:127]                O^T accumulators, (rb*4 + db)*16 + i
  a[208:239], a[240:255]  K fragment ring (8 x 4), V^T fragment ring (4 x 4)
  v[128:191], v[192:255]  S^T of two consecutive tiles, rb*32 + kb*16 + i; a tile's
                          P^T (fp16/bf16 pairs) is packed in place into the first 8
                          registers of each 16-register block
  v[112:119], v[120:127]  K fragment and V^T LDS addresses of the current tile
  v104/v105 per-lane P sums, v106/v107 -m, v108..v111 temporaries
  s[84:85] compare mask, s86 caller's m0, s87 rows left from the next tile to copy,
  s[88:91]/s[92:95] K/V copy resources,
  s96 tile j, s97 next tile to copy, s98/s99 temporaries
  v0..v103, a128..a207 and s0..s83 are left to the compiler (Q arrives in AGPRs).

The output is deterministic text, tracked under csrc/gen/; build.py checks the tracked
file against render() and rewrites it only when asked (--regen).
"""

import os
import sys

NBUF = 4            # LDS ring slots
OSTR = 1040         # bytes between a wave's O blocks in the LDS hand-off (kPipeOStr in fal_fwd.hip)
VOFF = 16384        # V offset inside a slot (bytes)
# Knobs (set by configure(); the values here are the product kernel's)
DEFAULTS = {
    "KDIST": 2,       # K read-ahead (k-steps of 2 fragments)
    "VRING": 4,       # V^T fragment ring (pairs of transposed reads)
    "VDIST": 3,       # V^T read-ahead (fragment pairs), < VRING
    "DMA_AUX": "",    # cache-policy bits of the tile copies
    "GSTRIDE": 1,     # MFMAs between two copy instructions
    # measurement builds only (wrong results): comma-separated subset of
    # nodma, nowait, nobar, novalu, nolds, dmasame, dmazero
    "ABL": "",
}
KDIST, VRING, VDIST, DMA_AUX, GSTRIDE = 2, 4, 3, "", 1
MEASURE, ABL = False, set()
DEFAULT_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "gen", "fal_fwd_pipe.inc")

SA = (128, 192)
VF = 256 - 4 * VRING   # AGPR: V^T ring at the top, K ring below it
KF = VF - 32
KC = 112
VC = 120
LT = (104, 105)
NM = (106, 107)
T0, T1, T2, T3 = 108, 109, 110, 111
SM, SM0, SR = 84, 86, 87
SK, SV = 88, 92
SJ, SD, ST, ST2 = 96, 97, 98, 99
NEG_INF = "0xff800000"

# ---- operands: (name, constraint, C++ expression) ----
OUTS = [("m0", "+v", "m_run[0]"), ("m1", "+v", "m_run[1]"), ("l0", "+v", "l_run[0]"), ("l1", "+v", "l_run[1]")]
INS = []
for rb in range(2):
    for t in range(8):
        INS.append((f"Q{rb}{t}", "a", f"qreg[{rb}][{t}]"))
for i in range(4):
    INS.append((f"kvo{i}", "v", f"kvo[{i}]"))
for i in range(4):
    INS.append((f"vvo{i}", "v", f"vvo[{i}]"))
for t in range(8):
    INS.append((f"ka{t}", "v", f"p_ka[{t}]"))
for hf in range(2):
    for db in range(4):
        INS.append((f"va{hf}{db}", "v", f"p_va[{hf}][{db}]"))
INS += [("row0", "v", "p_row[0]"), ("row1", "v", "p_row[1]"), ("hh4", "v", "p_hh4"), ("olds", "v", "p_olds")]
for i in range(4):
    INS.append((f"kr{i}", "s", f"pk_rs[{i}]"))
for i in range(4):
    INS.append((f"vr{i}", "s", f"pv_rs[{i}]"))
INS += [("c", "s", "c"), ("jbeg", "s", "p_jbeg"), ("jend", "s", "p_jend"), ("jl", "s", "p_jl"),
        ("wrow", "s", "p_wrow"), ("nk", "s", "p_nk"), ("ktb", "s", "p_ktb"), ("vtb", "s", "p_vtb"),
        ("krb", "s", "p_krb"), ("vrb", "s", "p_vrb"), ("rows", "s", "p_rows"),
        ("lbase", "s", "p_lbase"), ("npre", "s", "p_npre")]
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

    # -- instruction streams -------------------------------------------------
    def softmax_ops(self, par, rb, fma=True):
        """Softmax of row block rb of the tile whose scores are in SA[par]: exponent
        FMA, exp2, per-lane P sum (fp32 adds of the exponentials), packing into P^T
        (in place).  Streamed element by element (e = 2*i + kb over the two 16-score
        blocks) so the quarter-rate exponentials spread evenly between the MFMAs: the
        FMA runs two elements ahead, an element is summed one step after its
        exponential, and a pair is packed one step after its second exponential.
        (v_dot2c sums of the packed pairs stall the MFMA pipe: 24% of the loop.)"""
        b0 = SA[par] + rb * 32
        ops = [f"v_mov_b32 {v(LT[rb])}, 0"]
        if "novalu" in ABL:
            return ops
        reg = lambda e: b0 + (e % 2) * 16 + e // 2
        fmas = [f"v_fma_f32 {v(reg(e))}, {v(reg(e))}, {op('c')}, {v(NM[rb])}" for e in range(32)] if fma else []
        cvt_at = {}
        for kb in range(2):
            for k in range(8):
                last = 4 * k + 2 + kb           # element index of the pair's second exponential
                b = b0 + kb * 16
                cvt_at.setdefault(last + 1, []).append(f"{self.cvt} {v(b + k)}, {v(b + 2 * k)}, {v(b + 2 * k + 1)}")
        ops += fmas[:2]
        for e in range(36):
            if e + 2 < len(fmas):
                ops.append(fmas[e + 2])
            if e < 32:
                ops.append(f"v_exp_f32 {v(reg(e))}, {v(reg(e))}")
            if 0 <= e - 1 < 32:
                ops.append(f"v_add_f32 {v(LT[rb])}, {v(LT[rb])}, {v(reg(e - 1))}")
            ops += cvt_at.get(e, [])
        return ops

    def slot(self, dst, delta):
        """dst = ((j + delta) mod NBUF) * 32 KB"""
        return [f"s_add_u32 {dst}, s{SJ}, {delta % NBUF}", f"s_and_b32 {dst}, {dst}, {NBUF - 1}",
                f"s_lshl_b32 {dst}, {dst}, 15"]

    def kcur_ops(self, sreg):
        return [f"v_add_u32 {v(KC + t)}, {sreg}, {op(f'ka{t}')}" for t in range(8)]

    def vcur_ops(self, sreg):
        return [f"v_add_u32 {v(VC + hf * 4 + db)}, {sreg}, {op(f'va{hf}{db}')}" for hf in range(2) for db in range(4)]

    def dma_groups(self):
        """Copy of tile s97 into its slot (8 buffer->LDS loads), then the copy resources
        advance one tile (rows past the copy range read as zeros)."""
        # record counts of this tile: its rows inside the copy range (0..64) times the
        # row stride, so rows past the range read as zeros
        groups = [[f"s_and_b32 s{ST}, s{SD}, {NBUF - 1}", f"s_lshl_b32 s{ST}, s{ST}, 15",
                   f"s_add_u32 s{ST}, s{ST}, {op('lbase')}",
                   f"s_max_i32 s{SK + 2}, s{SR}, 0", f"s_min_i32 s{SK + 2}, s{SK + 2}, 64",
                   f"s_mul_i32 s{SV + 2}, s{SK + 2}, {op('vrb')}", f"s_mul_i32 s{SK + 2}, s{SK + 2}, {op('krb')}"]]
        for part, rs, vo in (("k", SK, "kvo"), ("v", SV, "vvo")):
            for i in range(4):
                off = i * 4096 + (VOFF if part == "v" else 0)
                groups.append([f"s_add_u32 m0, s{ST}, {off}", "s_nop 0"] + ([] if "nodma" in ABL else
                               [f"buffer_load_dwordx4 {op(f'{vo}{i}')}, s[{rs}:{rs + 3}], 0 offen{DMA_AUX} lds"]))
        if "dmasame" in ABL:
            groups.append([f"s_add_u32 s{SD}, s{SD}, 1"])
            return groups
        groups.append([
            f"s_add_u32 s{SK}, s{SK}, {op('ktb')}", f"s_addc_u32 s{SK + 1}, s{SK + 1}, 0",
            f"s_add_u32 s{SV}, s{SV}, {op('vtb')}", f"s_addc_u32 s{SV + 1}, s{SV + 1}, 0",
            f"s_sub_i32 s{SR}, s{SR}, 64",
            f"s_add_u32 s{SD}, s{SD}, 1"])
        return groups

    def dma(self):
        for g in self.dma_groups():
            self.es(g)

    def s_prod(self, par):
        """S^T = K Q^T of the tile whose K fragment addresses are in KC, into SA[par]."""
        reads, mf = [], []
        for t in range(8):
            for kb in range(2):
                slot = (2 * t + kb) % 8
                reads.append(f"ds_read_b128 {ar(KF + 4 * slot, 4)}, {v(KC + t)} offset:{kb * 8192}")
        for t in range(8):
            for kb in range(2):
                slot = (2 * t + kb) % 8
                for rb in range(2):
                    d = vr(SA[par] + rb * 32 + kb * 16, 16)
                    c = "0" if t == 0 else d
                    mf.append((f"{self.mf} {d}, {ar(KF + 4 * slot, 4)}, {op(f'Q{rb}{t}')}, {c}", 2 * t + kb))
        return reads, mf

    def pv_prod(self, par):
        """O^T += V^T P^T of the tile whose P^T is packed in SA[par], V^T addresses in VC."""
        reads, mf = [], []
        for ks in range(4):
            for db in range(4):
                p = (ks * 4 + db) % VRING
                for hf in range(2):
                    reads.append(f"ds_read_b64_tr_b16 {ar(VF + 4 * p + 2 * hf, 2)}, {v(VC + hf * 4 + db)} "
                                 f"offset:{VOFF + ks * 4096}")
        for ks in range(4):
            kb, t2 = ks // 2, ks % 2
            for db in range(4):
                p = (ks * 4 + db) % VRING
                for rb in range(2):
                    o = ar((rb * 4 + db) * 16, 16)
                    pb = vr(SA[par] + rb * 32 + kb * 16 + 4 * t2, 4)
                    mf.append((f"{self.mf} {o}, {ar(VF + 4 * p, 4)}, {pb}, {o}", 2 * (ks * 4 + db) + 1))
        return reads, mf

    @staticmethod
    def cost(ins):
        """Issue cycles of a VALU instruction (wave64 on the 16-lane SIMD; the
        exponential is quarter rate)."""
        if ins.startswith("v_exp"):
            return 16
        if ins.startswith("s_nop"):
            return int(ins.split()[1]) + 1
        return 4

    def interleave(self, reads, mf, dist, valu=(), groups=()):
        """MFMAs with their LDS reads issued `dist` reads ahead and the VALU stream and
        instruction groups spread between them, the VALU by issue cycles so that no gap
        between two MFMAs holds much more than one MFMA's 32 cycles of work.  LDS reads
        complete in issue order, so the wait before an MFMA lets the reads issued after
        its last one stay in flight."""
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
            self.e(ins)
            if groups and k % GSTRIDE == 0:
                self.es(groups.pop(0))
            goal = total * (k + 1) / len(mf)
            while valu and (done < goal or k == len(mf) - 1):
                x = valu.pop(0)
                done += self.cost(x)
                self.e(x)
        assert not valu and not groups and issued == len(reads)

    # -- blocks ----------------------------------------------------------------
    def mask_block(self, par, lbl):
        """Scores of tile j in SA[par] set to -inf where key > row (causal) or key >= nk.
        Skipped (branch to lbl) when no key of the tile can be masked for this wave."""
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
        e(f"v_mov_b32 {v(T3)}, {NEG_INF}")
        e(f"s_sub_u32 s{ST2}, {op('nk')}, s{ST}")
        e(f"s_sub_u32 s{ST2}, s{ST2}, 1")                 # last valid key of the tile, local
        for rb in range(2):
            # thr = min(row - n0, nk - 1 - n0) - hh*4: key kb*32 + c_i (+ hh*4) is kept iff
            # c_i + kb*32 <= thr
            e(f"v_subrev_u32 {v(T0)}, s{ST}, {op(f'row{rb}')}")
            e(f"v_min_i32 {v(T0)}, s{ST2}, {v(T0)}")
            e(f"v_sub_u32 {v(T0)}, {v(T0)}, {op('hh4')}")
            for kb in range(2):
                e(f"v_subrev_u32 {v(T1)}, {kb * 32}, {v(T0)}")
                for i in range(16):
                    ci = (i // 4) * 8 + i % 4
                    r = SA[par] + rb * 32 + kb * 16 + i
                    e(f"v_cmp_le_i32 vcc, {ci}, {v(T1)}")
                    e(f"v_cndmask_b32 {v(r)}, {v(T3)}, {v(r)}, vcc")
        e(f"{lbl}:")

    def init_max(self, lbl):
        """Rows without a max yet (m = -inf) take the max of the first tile's scaled
        scores (SA[0])."""
        e = self.e
        e(f"v_cmp_eq_f32 vcc, {NEG_INF}, {op('m0')}")
        e(f"s_cbranch_vccz {lbl}")
        for rb in range(2):
            b0 = SA[0] + rb * 32
            e(f"v_mov_b32 {v(T2)}, {NEG_INF}")
            for i in range(0, 32, 2):
                e(f"v_mul_f32 {v(T0)}, {op('c')}, {v(b0 + i)}")
                e(f"v_mul_f32 {v(T1)}, {op('c')}, {v(b0 + i + 1)}")
                e(f"v_max3_f32 {v(T2)}, {v(T2)}, {v(T0)}, {v(T1)}")
            e(f"v_mov_b32 {v(T3)}, {v(T2)}")
            e("s_nop 1")                                           # VALU write -> permlane swap read
            e(f"v_permlane32_swap_b32 {v(T2)}, {v(T3)}")
            e(f"v_max_f32 {v(T2)}, {v(T2)}, {v(T3)}")
            e(f"v_mov_b32 {op(f'm{rb}')}, {v(T2)}")
            e(f"v_cmp_eq_f32 vcc, {NEG_INF}, {v(T2)}")
            e(f"v_cndmask_b32_e64 {v(NM[rb])}, -{v(T2)}, 0, vcc")
        e(f"{lbl}:")

    def s_simple(self, par):
        """S of tile j (slot in s98) into SA[par], not interleaved (first tile, redo)."""
        self.es(self.kcur_ops(f"s{ST}"))
        reads, mf = self.s_prod(par)
        self.interleave(reads, mf, 2 * KDIST)
        for _ in range(4):
            self.e("s_nop 15")

    def fix_block(self, par, lbl, lbl_cont, lbl_m):
        """Tile j redone with a new row max: S recomputed from its K slot, masked, the
        max taken, O and l rescaled, P and its sums recomputed."""
        e = self.e
        e(f"{lbl}:")
        e("s_nop 15")
        self.es(self.slot(f"s{ST}", 0))
        self.s_simple(par)
        self.mask_block(par, lbl_m)
        e("s_nop 4")
        for rb in range(2):
            b0 = SA[par] + rb * 32
            for i in range(32):
                r = b0 + i
                e(f"v_fma_f32 {v(r)}, {v(r)}, {op('c')}, {v(NM[rb])}")
            e(f"v_mov_b32 {v(T0)}, {NEG_INF}")
            for i in range(0, 32, 2):
                e(f"v_max3_f32 {v(T0)}, {v(T0)}, {v(b0 + i)}, {v(b0 + i + 1)}")
            e(f"v_mov_b32 {v(T1)}, {v(T0)}")
            e("s_nop 1")
            e(f"v_permlane32_swap_b32 {v(T0)}, {v(T1)}")
            e(f"v_max_f32 {v(T0)}, {v(T0)}, {v(T1)}")             # mx (log2 domain, relative to m)
            m = op(f"m{rb}")
            # first row: dlt = mx, m = mx, alpha = 1; otherwise dlt = max(mx, 0), m += dlt,
            # alpha = 2^-dlt; mx = -inf: dlt = 0
            e(f"v_max_f32 {v(T1)}, 0, {v(T0)}")
            e(f"v_cmp_class_f32_e64 s[{SM}:{SM + 1}], {m}, 4")        # first: m = -inf
            e("s_nop 1")
            e(f"v_cndmask_b32_e64 {v(T1)}, {v(T1)}, {v(T0)}, s[{SM}:{SM + 1}]")
            e(f"v_cmp_eq_f32 vcc, {NEG_INF}, {v(T0)}")
            e(f"v_cndmask_b32_e64 {v(T1)}, {v(T1)}, 0, vcc")          # dlt
            e(f"v_add_f32 {v(T2)}, {m}, {v(T1)}")
            e(f"v_cndmask_b32_e64 {m}, {v(T2)}, {v(T0)}, s[{SM}:{SM + 1}]")
            e(f"v_exp_f32_e64 {v(T2)}, -{v(T1)}")
            e("s_nop 0")
            e(f"v_cndmask_b32_e64 {v(T2)}, {v(T2)}, 1.0, s[{SM}:{SM + 1}]")   # alpha
            e(f"v_mul_f32 {op(f'l{rb}')}, {op(f'l{rb}')}, {v(T2)}")
            for k in range(64):
                a = rb * 64 + k
                e(f"v_accvgpr_read_b32 {v(T3)}, a{a}")
                e(f"v_mul_f32 {v(T3)}, {v(T3)}, {v(T2)}")
                e("s_nop 1")
                e(f"v_accvgpr_write_b32 a{a}, {v(T3)}")
            for i in range(32):
                r = b0 + i
                e(f"v_sub_f32 {v(r)}, {v(r)}, {v(T1)}")
            e(f"v_cmp_eq_f32 vcc, {NEG_INF}, {m}")
            e(f"v_cndmask_b32_e64 {v(NM[rb])}, -{m}, 0, vcc")
            self.es(self.softmax_ops(par, rb, fma=False))
        e(f"s_branch {lbl_cont}")

    def fix_check(self, lbl_fix):
        """Redo the tile if some lane's P sum exceeds 2^15 or a row still has no max."""
        e = self.e
        e(f"s_mov_b32 s{ST2}, 0x47000000")                # 2^15
        e(f"v_cmp_nge_f32 vcc, s{ST2}, {v(LT[0])}")
        e(f"v_cmp_nge_f32_e64 s[{SM}:{SM + 1}], s{ST2}, {v(LT[1])}")
        e(f"s_or_b64 vcc, vcc, s[{SM}:{SM + 1}]")
        e(f"v_cmp_class_f32_e64 s[{SM}:{SM + 1}], {op('m0')}, 4")   # m = -inf
        e(f"s_or_b64 vcc, vcc, s[{SM}:{SM + 1}]")
        e(f"v_cmp_class_f32_e64 s[{SM}:{SM + 1}], {op('m1')}, 4")
        e(f"s_or_b64 vcc, vcc, s[{SM}:{SM + 1}]")
        e(f"s_cbranch_vccnz {lbl_fix}")

    def soft_iteration(self, par, pv, snext, L):
        """Iteration j with the softmax of tile j (scores in SA[par])."""
        e = self.e
        self.mask_block(par, L("nomask"))
        if pv:
            self.es(self.slot(f"s{ST}", -1))
            self.es(self.vcur_ops(f"s{ST}"))
        if snext:
            self.es(self.slot(f"s{ST2}", 1))
        soft0 = ["s_nop 7"] + self.softmax_ops(par, 0) + (self.kcur_ops(f"s{ST2}") if snext else [])
        if pv:
            reads, mf = self.pv_prod(par ^ 1)
            self.interleave(reads, mf, 2 * VDIST, soft0, self.dma_groups())
        else:
            self.dma()
            self.es(soft0)
        if "nowait" not in ABL:
            e("s_waitcnt vmcnt(8)")
        if "nobar" not in ABL:
            e("s_barrier")
        soft1 = self.softmax_ops(par, 1)
        if snext:
            reads, mf = self.s_prod(par ^ 1)
            self.interleave(reads, mf, 2 * KDIST, soft1)
        else:
            self.es(soft1)
        if not ABL:
            self.fix_check(L(f"fix{par}", shared=True))
        e(f"s_branch {L(f'cont{par}', shared=True)}")

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
        e(f"s_mov_b32 s{SJ}, {op('jbeg')}")
        e(f"s_mov_b32 s{SR}, {op('rows')}")
        if "dmazero" in ABL:
            e(f"s_mov_b32 s{SR}, 0")
        e(f"s_mov_b32 s{SD}, {op('jbeg')}")
        for a in range(128):
            e(f"v_accvgpr_write_b32 a{a}, 0")
        for rb in range(2):
            e(f"v_cmp_eq_f32 vcc, {NEG_INF}, {op(f'm{rb}')}")
            e(f"v_cndmask_b32_e64 {v(NM[rb])}, -{op(f'm{rb}')}, 0, vcc")
        # the first two tiles, unless the caller already issued their copies (npre = 2:
        # the copy resources, the row count and the tile index then start two tiles on)
        e(f"s_cmp_eq_u32 {op('npre')}, 0")
        e(f"s_cbranch_scc0 {L('pre', shared=True)}")
        self.dma()
        self.dma()
        e(f"s_branch {L('predone', shared=True)}")
        e(f"{L('pre', shared=True)}:")
        e(f"s_add_u32 s{SD}, s{SD}, {op('npre')}")
        e(f"{L('predone', shared=True)}:")
        e("s_waitcnt vmcnt(8)")
        e("s_barrier")
        # S of the first tile (if this wave has any tile), masked, then the first max
        e(f"s_cmp_gt_i32 s{SJ}, {op('jl')}")
        e(f"s_cbranch_scc1 {L('disp', shared=True)}")
        self.es(self.slot(f"s{ST}", 0))
        self.s_simple(0)
        self.mask_block(0, L("pmask"))
        e("s_nop 4")
        self.init_max(L("noinit"))

        # ---- per-iteration dispatch (uniform per wave) ----
        e(f"{L('disp', shared=True)}:")
        e(f"s_sub_u32 s{ST}, s{SJ}, {op('jbeg')}")
        e(f"s_and_b32 s{ST}, s{ST}, 1")
        e(f"s_cmp_eq_u32 s{ST}, 0")
        e(f"s_cbranch_scc0 {L('disp1', shared=True)}")
        for par in (0, 1):
            if par == 1:
                e(f"{L('disp1', shared=True)}:")
            e(f"s_cmp_gt_i32 s{SJ}, {op('jl')}")
            e(f"s_cbranch_scc1 {L(f'nosoft{par}', shared=True)}")
            e(f"s_cmp_eq_u32 s{SJ}, {op('jbeg')}")
            e(f"s_cbranch_scc1 {L(f'first{par}', shared=True)}")
            e(f"s_cmp_eq_u32 s{SJ}, {op('jl')}")
            e(f"s_cbranch_scc1 {L(f'last{par}', shared=True)}")
            self.soft_iteration(par, True, True, L)
            e(f"{L(f'last{par}', shared=True)}:")
            self.soft_iteration(par, True, False, L)
            e(f"{L(f'first{par}', shared=True)}:")
            e(f"s_cmp_eq_u32 s{SJ}, {op('jl')}")
            e(f"s_cbranch_scc1 {L(f'firstlast{par}', shared=True)}")
            self.soft_iteration(par, False, True, L)
            e(f"{L(f'firstlast{par}', shared=True)}:")
            self.soft_iteration(par, False, False, L)
            # no softmax: PV of the wave's last tile (j = jl + 1), or nothing
            e(f"{L(f'nosoft{par}', shared=True)}:")
            e(f"s_add_u32 s{ST}, {op('jl')}, 1")
            e(f"s_cmp_eq_u32 s{SJ}, s{ST}")
            e(f"s_cbranch_scc0 {L(f'idle{par}', shared=True)}")
            e(f"s_cmp_gt_i32 s{SJ}, {op('jbeg')}")
            e(f"s_cbranch_scc0 {L(f'idle{par}', shared=True)}")
            self.es(self.slot(f"s{ST}", -1))
            self.es(self.vcur_ops(f"s{ST}"))
            reads, mf = self.pv_prod(par ^ 1)
            self.interleave(reads, mf, 2 * VDIST, (), self.dma_groups())
            e("s_waitcnt vmcnt(8)")
            e("s_barrier")
            e(f"s_branch {L('next', shared=True)}")
            e(f"{L(f'idle{par}', shared=True)}:")
            self.dma()
            e("s_waitcnt vmcnt(8)")
            e("s_barrier")
            e(f"s_branch {L('next', shared=True)}")
            # tile j's P could leave fp16 range, or a row had no max: redo it
            self.fix_block(par, L(f"fix{par}", shared=True), L(f"cont{par}", shared=True), L("fmask"))
            e(f"{L(f'cont{par}', shared=True)}:")
            e(f"v_add_f32 {op('l0')}, {op('l0')}, {v(LT[0])}")
            e(f"v_add_f32 {op('l1')}, {op('l1')}, {v(LT[1])}")
            e(f"s_branch {L('next', shared=True)}")
        e(f"{L('next', shared=True)}:")
        e(f"s_add_u32 s{SJ}, s{SJ}, 1")
        e(f"s_cmp_lt_i32 s{SJ}, {op('jend')}")
        e(f"s_cbranch_scc1 {L('disp', shared=True)}")
        # ---- after the last iteration (j = jend): PV of the wave's last tile if it is
        # the workgroup's last tile ----
        e(f"s_add_u32 s{ST}, {op('jl')}, 1")
        e(f"s_cmp_eq_u32 s{SJ}, s{ST}")
        e(f"s_cbranch_scc0 {L('out', shared=True)}")
        e(f"s_cmp_gt_i32 s{SJ}, {op('jbeg')}")
        e(f"s_cbranch_scc0 {L('out', shared=True)}")
        e(f"s_sub_u32 s{ST}, s{SJ}, {op('jbeg')}")
        e(f"s_and_b32 s{ST}, s{ST}, 1")
        e(f"s_cmp_eq_u32 s{ST}, 0")
        e(f"s_cbranch_scc0 {L('drain0', shared=True)}")
        for par, lbl in ((1, None), (0, L('drain0', shared=True))):
            # j - jbeg even: the last tile (j - 1) has odd parity, its P is in SA[1]
            if lbl:
                e(f"{lbl}:")
            self.es(self.slot(f"s{ST}", -1))
            self.es(self.vcur_ops(f"s{ST}"))
            reads, mf = self.pv_prod(par)
            self.interleave(reads, mf, 2 * VDIST)
            e(f"s_branch {L('out', shared=True)}")
        e(f"{L('out', shared=True)}:")
        # every wave is done with the ring: O goes to this wave's 32 KB of LDS
        for _ in range(2):
            e("s_nop 15")
        e("s_waitcnt vmcnt(0) lgkmcnt(0)")
        e("s_barrier")
        for g in range(32):
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
    if cfg["ABL"] and not measure:
        raise ValueError("ablation knobs (ABL) give wrong results; they need a measurement build")
    g = globals()
    for k in DEFAULTS:
        g[k] = type(DEFAULTS[k])(cfg[k]) if k != "ABL" else set(x for x in str(cfg[k]).split(",") if x)
    g["MEASURE"] = bool(measure)
    g["VF"] = 256 - 4 * g["VRING"]
    g["KF"] = g["VF"] - 32

def render(knobs=None, measure=False):
    """The generated text for the given knobs (defaults: the product kernel)."""
    configure(knobs, measure)
    try:
        return _render()
    finally:
        configure()


def _render():
    out = ["// Generated by gen_fwd_pipe.py; do not edit.", "#pragma once", ""]
    for bf16, name in ((False, "FAL_PIPE_ASM_F16"), (True, "FAL_PIPE_ASM_BF16")):
        lines = Emitter(bf16).program()
        out.append(f"#define {name} \\")
        for ln in lines:
            out.append(f'  "{ln}\\n" \\')
        out.append("")
    outs = ", ".join(f'"{c}"({x})' for _, c, x in OUTS)
    ins = ", ".join(f'"{c}"({x})' for _, c, x in INS)
    clob = ", ".join([f'"v{i}"' for i in range(104, 256)] + [f'"a{i}"' for i in range(0, 128)] +
                     [f'"a{i}"' for i in range(KF, 256)] + [f'"s{i}"' for i in range(84, 100)] +
                     ['"vcc"', '"scc"', '"memory"'])
    out.append(f"#define FAL_PIPE_OUTS {outs}")
    out.append(f"#define FAL_PIPE_INS {ins}")
    out.append(f"#define FAL_PIPE_CLOBBERS {clob}")
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

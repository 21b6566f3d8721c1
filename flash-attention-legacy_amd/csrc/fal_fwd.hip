// Attention forward for gfx950: online softmax with QK^T and PV on MFMA.
//
// Semantics follow the reference forward (csrc/kernels/flash_attn_fwd_volta.cu:170-345
// batched, :350-523 varlen): s = (q . k) * scale; keys with index >= seqlen_k or, when
// causal, key > query (top-left aligned, local indices for varlen) are excluded;
// O = sum(p v) / sum(p); L = max + ln(max(sum, 1e-20)) in natural log; a row with no
// valid key gives O = 0 and L = -inf.
//
// Work decomposition (one workgroup = NW waves = 32*NW*RB query rows of one head):
// * each wave owns 32 query rows (RB = 1); its Q slice stays in VGPRs for the
//   whole kernel as the B operand of
//   S^T = K Q^T, so the accumulator puts one query row per lane (two lanes per row,
//   one per wave half) and row reductions are in-lane plus one permlane32 swap;
// * K/V tiles of BN keys are copied HBM -> LDS by buffer loads that bypass VGPRs,
//   into XOR-swizzled, double-buffered tiles (conflict-free row and transposed
//   reads); one buffer resource per tile zero-fills rows past the sequence end;
// * one FMA per score gives the exponent s*scale*log2(e) - m of P, m being the row's
//   reference max; the row max is recomputed only when a tile's P
//   could leave fp16 range (its per-lane p sum exceeds 2^15) or on a row's first tile;
// * P^T goes straight from the S^T accumulator into the B operand of O^T = V^T P^T;
//   V^T comes from the row-major V tile through ds_read_b64_tr_b16;
// * causal tiles above the diagonal are never visited; fully-masked waves inside a
//   diagonal tile skip their MFMAs.
#include <algorithm>
#include <type_traits>

#include "fal_kernels.h"
#include "fal_fwd_pipe.inc"

namespace fal {

// Tunables (compile-time): minimum waves per SIMD the register budget must allow,
// KV tile width for head_dim <= 128, K fragment read-ahead (k-steps).
#ifndef FAL_FWD_WPE
#define FAL_FWD_WPE 2
#endif
#ifndef FAL_FWD_BN
#define FAL_FWD_BN 64
#endif
#ifndef FAL_PRESCALE_FP16
#define FAL_PRESCALE_FP16 0
#endif
#ifndef FAL_FWD_KDEPTH
#define FAL_FWD_KDEPTH 2
#endif
#ifndef FAL_FWD_SUM_F32
#define FAL_FWD_SUM_F32 1   // row sums: 1 = fp32 adds of exp2 values, 0 = v_dot2c of the packed P
#endif
#ifndef FAL_FWD_PIPE
#define FAL_FWD_PIPE 1   // head_dim 128 at two row blocks per wave: software-pipelined tile loop
#endif

// A workgroup's (batch or sequence, query head, query tile) and its row ranges.
struct FwdItem {
  int b, hq, qt, q_off, k_off, nq, nk, split;
  int pre;    // persistent schedule: copies of the first two K/V tiles already issued (2) or not (0)
  int qpre;   // persistent schedule: this item's Q slices already loaded (by the previous item)
};

// Item `item` of the varlen forward work list for at most 64 sequences, derived in the
// wave from cu_seqlens (no schedule kernel): the same order as the grouped list of
// varlen_schedule_kernel, i.e. sequences by tile count, most tiles first (ties by
// index), each sequence's tiles contiguous, its last (heaviest causal) tile first.
// Lane s holds sequence s; every wave of the workgroup computes the same result.
// False past the end of the list.
__device__ __forceinline__ bool varlen_item_small(const int* cu, int num_seqs, int total, int tile, int item,
                                                  int& seq, int& qtile) {
  const int lane = threadIdx.x & 63;
  int nt = 0;
  if (lane < num_seqs) {
    int off, len;
    seg_bounds(cu, lane, total, off, len);
    nt = cdiv(len, tile);
  }
  // first list index of this lane's sequence: the tiles of every sequence ordered before it
  int start = 0;
  for (int s = 0; s < num_seqs; ++s) {
    const int ns = __builtin_amdgcn_readlane(nt, s);
    start += (ns > nt || (ns == nt && s < lane)) ? ns : 0;
  }
  const bool mine = lane < num_seqs && item >= start && item < start + nt;
  const uint64_t m = __builtin_amdgcn_ballot_w64(mine);
  if (!m) return false;
  const int src = __builtin_ctzll(m);
  seq = src;
  qtile = __builtin_amdgcn_readlane(nt, src) - 1 - (item - __builtin_amdgcn_readlane(start, src));
  return true;
}

// Resolves the work item of this workgroup (query tiles of `bm` rows); false for a
// padding block, which exits.
template <bool CAUSAL>
__device__ __forceinline__ bool fwd_item(const FwdParams& p, FwdItem& it, int bm) {
  it.pre = 0;
  it.qpre = 0;
  if (p.cu_q) {
    // 1-D grid over (work item, KV head) groups of G query heads.  Block i runs on XCD
    // i % 8 as that XCD's (i / 8)-th block; the groups are dealt to the XCDs round-robin
    // in work-list order (heaviest first), and the G heads of a group, which read the
    // same K/V, run back to back on one XCD (one L2).  The grid is padded to a multiple
    // of 8 groups; padding blocks exit.
    // gqa4: one workgroup per four query heads of a group (wave w takes head 4*hg + w)
    const int g = p.Hq / p.Hkv;
    const int ng = p.gqa4 ? g >> 2 : g;
    const int k8 = blockIdx.x >> 3;
    const int grp = (k8 / ng) * 8 + (blockIdx.x & 7);
    const int item = grp / p.Hkv;
    if (item >= p.n_qtiles) return false;
    int seq, qt;
    if (p.work) {
      const int2 wk = p.work[item];
      seq = wk.x;
      qt = wk.y;
      if (seq < 0) return false;
    } else if (!varlen_item_small(p.cu_q, p.num_seqs, p.total_q, bm, item, seq, qt)) {
      return false;
    }
    it.hq = __builtin_amdgcn_readfirstlane((grp % p.Hkv) * g +
                                           (p.gqa4 ? (k8 % ng) * 4 + (int)(threadIdx.x >> 6) : k8 % ng));
    it.b = 0;
    it.split = 0;
    it.qt = qt;
    seg_bounds(p.cu_q, seq, p.total_q, it.q_off, it.nq);
    seg_bounds(p.cu_k, seq, p.total_k, it.k_off, it.nk);
  } else {
    // 1-D grid; group heads of one KV head and the query tiles of a head together so the
    // workgroups an XCD runs at once share K/V in that XCD's L2 (workgroups are dealt to
    // the 8 XCDs round-robin by linear id).
    const int total = gridDim.x;
    int id = blockIdx.x;
    if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
    it.split = id % p.nsplit;   // the splits of a query tile run next to each other
    id /= p.nsplit;
    const int g = p.Hq / p.Hkv;
    const int ng = p.gqa4 ? g / 4 : g;           // workgroups per (KV head, query tile)
    const int hg = id % ng;
    int rest = id / ng;
    const int t = rest % p.n_qtiles;
    rest /= p.n_qtiles;                          // = b * Hkv + hkv
    it.qt = CAUSAL ? (p.n_qtiles - 1 - t) : t;   // heaviest causal tiles first
    it.b = rest / p.Hkv;
    // gqa4: wave w takes query head 4*hg + w of the group
    it.hq = __builtin_amdgcn_readfirstlane((rest % p.Hkv) * g + (p.gqa4 ? hg * 4 + (int)(threadIdx.x >> 6) : hg));
    it.q_off = 0;
    it.k_off = 0;
    it.nq = p.Nq;
    it.nk = p.Nk;
  }
  return true;
}

// Pipelined loop's O hand-off in LDS: 32 blocks of 1 KB per wave, 1040 bytes apart so the
// row-wise reads of the epilogue spread over the banks.
constexpr int kPipeOStr = 1040;
constexpr int kPipeOWave = 32 * kPipeOStr;

// One work item (query tile of one head, or of four heads under gqa4) of fwd_kernel.
// Every wave of the workgroup takes the same early returns.
// Persistent schedule (`next` valid when has_next): returns pre | (qpre << 2) for the next
// item -- pre = 2 when this item issued the copies of its first two K/V tiles, qpre = 1
// when it loaded its Q slices into qio (the Q registers, free once the tile loop is done).
template <class T, int D, int NW, int BN, bool CAUSAL, int RB>
__device__ __forceinline__ int fwd_body(const FwdParams& p, const FwdItem& it, T* smem, const FwdItem& next,
                                        bool has_next, vec8<T> (&qio)[RB][D / 16]) {
  using TL = SwizzledTile<D>;
  using V8 = vec8<T>;
  using V4 = vec4<T>;
  // Q stays exact and the fp32 scores are scaled (one FMA per score).  FAL_PRESCALE_FP16
  // instead pre-multiplies an fp16 Q by scale*log2(e), rounded once to fp16: that saves
  // the FMA but shifts large scores by up to ~1e-2 in log2 units, so it is off.
  constexpr bool PRESCALE = FAL_PRESCALE_FP16 && std::is_same<T, half_t>::value;
  // PIPE: the key-tile loop is the software-pipelined asm block (head_dim 128, 64 query
  // rows per wave, one wave per SIMD) with a ring of 4 K/V tiles copied two tiles ahead.
  constexpr bool PIPE = FAL_FWD_PIPE && D == 128 && RB == 2 && NW == 4 && BN == 64 && !FAL_PRESCALE_FP16;
  constexpr bool PIPE_SIGN = PIPE;
  constexpr int BM = NW * 32 * RB;  // query rows per workgroup (RB 32-row blocks per wave)
  constexpr int KS = D / 16;        // MFMA k-steps over the head dim
  constexpr int NKB = BN / 32;      // 32-key blocks per tile
  constexpr int DB = D / 32;        // 32-wide blocks of the output head dim
  constexpr int CPR = TL::CPR;      // 16-byte chunks per row
  constexpr int PART = BN * CPR * 8;          // elements of one K (or V) tile
  constexpr int IPT = BN * CPR / (NW * 64);   // direct-to-LDS loads per wave per part
  constexpr int NSLOT = PIPE ? 4 : 2;   // K/V tile buffers in LDS
  static_assert(BN * CPR % (NW * 64) == 0, "tile must split evenly over the waves");

  // (an opaque copy: under the persistent schedule the per-lane addresses below are
  // recomputed per item instead of being hoisted out of the item loop and kept live,
  // spilled, across the asm block)
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  int pre_next = 0, qpre_next = 0;
  bool stored = false;   // the pipelined path wrote O and L itself

  const int b = it.b, hq = it.hq, qt = it.qt, q_off = it.q_off, k_off = it.k_off, nq = it.nq, nk = it.nk;
  const int hkv = hq / (p.Hq / p.Hkv);
  // gqa4 (pipelined loop only): the waves share 64 query rows of different heads
  const bool gqa4 = PIPE && p.gqa4;
  const int BMW = gqa4 ? 32 * RB : BM;      // query rows per workgroup and head
  const int m0 = qt * BMW;
  if (m0 >= nq) return 0;

  const T* qbase = (const T*)p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)q_off * p.q_ss;
  const T* kbase = (const T*)p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh + (int64_t)k_off * p.k_ss;
  const T* vbase = (const T*)p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh + (int64_t)k_off * p.v_ss;
  T* obase = (T*)p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + (int64_t)q_off * p.o_ss;
  float* lbase = p.lse + (int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)q_off * p.l_ss;

  // ---- per-lane addressing of the swizzled tiles ----
  // Load instruction i of wave ws fills LDS chunks [(i*NW + ws)*64, +64) of the tile;
  // the per-lane global offsets are relative to the tile's first row, so they do not
  // depend on the tile.
  const int ws = __builtin_amdgcn_readfirstlane(w);   // wave index as a scalar
  int kvo[IPT], vvo[IPT];             // byte offsets from the tile's first row
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int I = i * NW + ws;
    const int pch = I * 64 + lane;
    const int r = pch / CPR;
    const int cc = TL::logical_chunk(r, pch % CPR);
    kvo[i] = (int)(r * p.k_ss + cc * 8) * 2;
    vvo[i] = (int)(r * p.v_ss + cc * 8) * 2;
  }
  // The first two K/V tiles of item x into slots 0 and 1: the copies the pipelined loop's
  // prologue would issue (it then starts at tile 2).  Returns 2 when issued (x has two
  // tiles or more), else 0.  Only for the whole key range (no split-KV).
  auto issue_first2 = [&](const FwdItem& x) -> int {
    if (!PIPE || p.kchunk) return 0;
    const int xm0 = x.qt * BMW;
    if (xm0 >= x.nq) return 0;
    const int xkend = CAUSAL ? min(x.nk, xm0 + BMW) : x.nk;
    const int xjend = cdiv(xkend, BN);
    if (xjend < 2) return 0;
    const int xhkv = x.hq / (p.Hq / p.Hkv);
    const T* xkb = (const T*)p.k + (int64_t)x.b * p.k_sb + (int64_t)xhkv * p.k_sh + (int64_t)x.k_off * p.k_ss;
    const T* xvb = (const T*)p.v + (int64_t)x.b * p.v_sb + (int64_t)xhkv * p.v_sh + (int64_t)x.k_off * p.v_ss;
    const int64_t xrows = min(x.nk, xjend * BN);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int64_t rt = min(max(xrows - (int64_t)t * BN, (int64_t)0), (int64_t)BN);
      // record counts clamped as in load_tile (rt <= BN rows: below 2^31 under the host's
      // sequence-stride limit anyway)
      const __amdgpu_buffer_rsrc_t krs =
          make_rsrc(xkb + (int64_t)t * BN * p.k_ss, (uint32_t)min(rt * p.k_ss * 2, (int64_t)0x7fffffff));
      const __amdgpu_buffer_rsrc_t vrs =
          make_rsrc(xvb + (int64_t)t * BN * p.v_ss, (uint32_t)min(rt * p.v_ss * 2, (int64_t)0x7fffffff));
      T* kdst = smem + t * 2 * PART;
#pragma unroll
      for (int i = 0; i < IPT; ++i) {
        const int I = i * NW + ws;
        buffer_to_lds16(krs, kvo[i], kdst + I * 64 * 8);
        buffer_to_lds16(vrs, vvo[i], kdst + PART + I * 64 * 8);
      }
    }
    return 2;
  };
  // this item's first tiles, unless the previous item issued them: in flight with the Q loads
  const int pre_cur = it.pre ? it.pre : issue_first2(it);

  // ---- Q slices of this wave into registers (B operand: n = query row, k = head dim) ----
  // Row block rb of wave w covers rows m0 + (w*RB + rb)*32 ..; each K or V fragment read
  // from LDS feeds RB MFMAs.  c = softmax_scale * log2(e), the sign included, takes
  // the scores to the log2 domain.
  // The pipelined loop masks raw scores with -inf, which needs c > 0: a negative scale
  // is folded into Q (exact) and a zero scale becomes 1e-30 (every exponent rounds to 0).
  const bool negq = PIPE_SIGN && p.scale_log2 < 0.f;
  const float c = PIPE_SIGN ? fmaxf(fabsf(p.scale_log2), 1e-30f) : p.scale_log2;
  int row[RB];
  V8 (&qreg)[RB][KS] = qio;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) row[rb] = m0 + ((gqa4 ? 0 : w) * RB + rb) * 32 + l32;
#pragma unroll
  for (int rb = 0; rb < RB && !it.qpre; ++rb) {
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      V8 x = row[rb] < nq ? ld8(qbase + (int64_t)row[rb] * p.q_ss + t * 16 + hh * 8) : zero8<T>();
      if (PRESCALE) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = (T)((float)x[e] * c);
      }
      if (negq) {
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = -x[e];
      }
      qreg[rb][t] = x;
    }
  }

  // ---- key range: tiles [jbeg, jend), the whole range or this workgroup's split ----
  const int kend = CAUSAL ? min(nk, m0 + BMW) : nk;
  int jbeg = 0, jend = cdiv(kend, BN);
  if (p.kchunk) {
    jbeg = it.split * p.kchunk;
    jend = min(jend, jbeg + p.kchunk);
    if (jbeg >= jend && it.split > 0) return 0;   // split past this tile's keys (split 0 always reports)
  }
  // tiles below this index need no masking for any row of the workgroup
  const int nfull = CAUSAL ? min(nk / BN, (m0 + 1) / BN) : nk / BN;

  int kaddr[KS];                     // K fragment (row l32, chunk 2t+hh) for 32-key block 0
#pragma unroll
  for (int t = 0; t < KS; ++t) kaddr[t] = TL::offset(l32, 2 * t + hh);
  int vaddr[2][DB];                  // transposed V reads: rows hf*8 + hh*4 + i/4 of each 16-key step
  {
    const int i = lane & 15;
    const int rl = hh * 4 + (i >> 2);
    const int cl = 2 * ((lane >> 4) & 1) + ((lane >> 1) & 1);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int db = 0; db < DB; ++db) vaddr[hf][db] = TL::offset(hf * 8 + rl, db * 4 + cl) + 4 * (lane & 1);
  }

  // Tile `tile` of K and V into LDS buffer `buf` without passing through VGPRs.  One
  // buffer resource per tile starts at its first row and ends at the last key, so rows
  // past the end of the sequence read as zeros.
  auto load_tile = [&](int tile, int buf) {
    const int n0 = tile * BN;
    T* kdst = smem + buf * 2 * PART;
    T* vdst = kdst + PART;
    const int64_t left = (int64_t)max(nk - n0, 0);
    const __amdgpu_buffer_rsrc_t krs =
        make_rsrc(kbase + (int64_t)n0 * p.k_ss, (uint32_t)min(left * p.k_ss * 2, (int64_t)0x7fffffff));
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc(vbase + (int64_t)n0 * p.v_ss, (uint32_t)min(left * p.v_ss * 2, (int64_t)0x7fffffff));
#pragma unroll
    for (int i = 0; i < IPT; ++i) {
      const int I = i * NW + ws;
      buffer_to_lds16(krs, kvo[i], kdst + I * 64 * 8);
      buffer_to_lds16(vrs, vvo[i], vdst + I * 64 * 8);
    }
  };

  f32x16 oacc[RB][DB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int i = 0; i < DB; ++i) oacc[rb][i] = zero_f16();
  // m_run: reference max of the row (log2 domain); it may lag the true running max, as
  // long as every p = exp2(s - m_run) of a tile fits fp16 (the tile's p sum <= 2^15).
  // nm: -m_run, the addend of the score FMA; negm: the same broadcast over an
  // accumulator block, the starting value of S^T under FAL_PRESCALE_FP16.
  float m_run[RB], l_run[RB];
  f32x16 negm[RB];
  float nm[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    m_run[rb] = -INFINITY;
    l_run[rb] = 0.f;
    negm[rb] = zero_f16();
    nm[rb] = 0.f;
  }

  auto tile_body = [&](auto masked, int j, int buf) {
    constexpr bool MASK = decltype(masked)::value;
    const int n0 = j * BN;
    const T* ks = smem + buf * 2 * PART;
    const T* vs = ks + PART;
    // S^T = K Q^T, the 32-key blocks interleaved so consecutive MFMAs are independent.
    // K fragments are read FAL_FWD_KDEPTH k-steps ahead of the MFMAs that use them.
    f32x16 sacc[RB][NKB];
    V8 kfrag[KS][NKB];
#pragma unroll
    for (int t = 0; t < FAL_FWD_KDEPTH && t < KS; ++t)
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) kfrag[t][kb] = ld8(ks + kaddr[t] + kb * 32 * CPR * 8);
    __builtin_amdgcn_sched_group_barrier(0x100, (FAL_FWD_KDEPTH < KS ? FAL_FWD_KDEPTH : KS) * NKB, 0);
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      if (t + FAL_FWD_KDEPTH < KS) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
          kfrag[t + FAL_FWD_KDEPTH][kb] = ld8(ks + kaddr[t + FAL_FWD_KDEPTH] + kb * 32 * CPR * 8);
        __builtin_amdgcn_sched_group_barrier(0x100, NKB, 0);   // the reads ...
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
          sacc[rb][kb] = mfma32(kfrag[t][kb], qreg[rb][t], t == 0 ? (PRESCALE ? negm[rb] : zero_f16()) : sacc[rb][kb]);
      __builtin_amdgcn_sched_group_barrier(0x008, NKB * RB, 0);  // ... then the MFMAs of step t
    }
    if (!PRESCALE) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) sacc[rb][kb][i] = fmaf(sacc[rb][kb][i], c, nm[rb]);
    }
    if (MASK) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = n0 + kb * 32 + (i >> 2) * 8 + hh * 4 + (i & 3);
            if (key >= nk || (CAUSAL && key > row[rb])) sacc[rb][kb][i] = -INFINITY;
          }
    }
    // P^T = exp2(s - m_run) in fp16 (the B operand of O^T += V^T P^T) and this tile's
    // per-lane p sum
    V8 pb[RB][NKB][2];
    float lt[RB];
    auto make_p = [&]() {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        lt[rb] = 0.f;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int t2 = 0; t2 < 2; ++t2) {
            V8 h;
#if FAL_FWD_SUM_F32
            // fp32 adds of the exponentials (v_dot2c sums of the packed P stall the MFMAs)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float pe = fast_exp2(sacc[rb][kb][t2 * 8 + e]);
              h[e] = (T)pe;
              lt[rb] += pe;
            }
#else
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (T)fast_exp2(sacc[rb][kb][t2 * 8 + e]);
            lt[rb] = sum8(h, lt[rb]);
#endif
            pb[rb][kb][t2] = h;
          }
      }
    };
    make_p();
    // The reference max moves only when some p of the tile could leave fp16 range
    // (or on a row's first keys): then rescale O and l to the tile's true max.
    bool fix = false;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) fix |= !(lt[rb] <= 32768.f) || m_run[rb] == -INFINITY;
    if (__builtin_amdgcn_ballot_w64(fix)) {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[rb][kb][i]);
        mx = pair_max(mx);
        // scores are s - m_use, m_use = (m_run == -inf ? 0 : m_run)
        const bool first = m_run[rb] == -INFINITY;
        const float dlt = (mx == -INFINITY) ? 0.f : (first ? mx : fmaxf(mx, 0.f));
        if (first) {
          if (mx != -INFINITY) m_run[rb] = mx;
        } else {
          m_run[rb] += dlt;
          const float alpha = fast_exp2(-dlt);
          l_run[rb] *= alpha;
#pragma unroll
          for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int i = 0; i < 16; ++i) oacc[rb][db][i] *= alpha;
        }
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) sacc[rb][kb][i] -= dlt;
        nm[rb] = (m_run[rb] == -INFINITY) ? 0.f : -m_run[rb];
        if (PRESCALE) {
#pragma unroll
          for (int i = 0; i < 16; ++i) negm[rb][i] = nm[rb];
        }
      }
      make_p();
    }
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) l_run[rb] += lt[rb];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        const int kofs = (kb * 2 + t2) * 16 * CPR * 8;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const V8 va = join8(lds_tr(vs + vaddr[0][db] + kofs), lds_tr(vs + vaddr[1][db] + kofs));
#pragma unroll
          for (int rb = 0; rb < RB; ++rb) oacc[rb][db] = mfma32(va, pb[rb][kb][t2], oacc[rb][db]);
        }
      }
  };
  // One pipeline step: wait for tile j, prefetch tile j+1 into the other buffer, consume j.
  auto step = [&](auto masked, int j, int buf) {
    wait_vmcnt0();
    __syncthreads();                       // tile j visible; tile j-1 reads finished
    if (j + 1 < jend) load_tile(j + 1, buf ^ 1);
    tile_body(masked, j, buf);
  };

  const int wrow_hi = m0 + (w * RB + RB - 1) * 32 + 31;   // last query row of this wave
  if constexpr (PIPE) {
    // The whole key-tile loop is one software-pipelined asm block (fal_fwd_pipe.inc,
    // generated by gen_fwd_pipe.py): a 4-slot K/V ring copied two tiles ahead, PV of
    // tile j-1 and S of tile j+1 interleaved with the softmax of tile j, masking of the
    // diagonal and last tiles, and the row-max fix-up.  It leaves m and l in registers
    // and this wave's O in LDS.
    typedef __attribute__((address_space(3))) T lds_t;
    const uint32_t lds0 = (uint32_t)(uintptr_t)((lds_t*)smem);
    uint32_t p_ka[KS], p_va[2][DB];
#pragma unroll
    for (int t = 0; t < KS; ++t) p_ka[t] = lds0 + 2 * kaddr[t];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int db = 0; db < DB; ++db) p_va[hf][db] = lds0 + 2 * vaddr[hf][db];
    const uint32_t p_lbase = __builtin_amdgcn_readfirstlane(lds0 + ws * 64 * 16);
    const uint32_t p_olds = lds0 + ws * kPipeOWave + lane * 16;
    int p_row[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) p_row[rb] = CAUSAL ? row[rb] : 0x3fffffff;
    const int p_hh4 = hh * 4;
    // copy resources of tile jbeg over the rows [jbeg*BN, min(nk, jend*BN)); each copy
    // advances them by one tile, so rows past that range read as zeros
    // (with pre_cur = 2 the copies of tiles jbeg and jbeg+1 into slots 0 and 1 are already
    // issued, and the loop starts copying at jbeg + 2)
    const int p_npre = __builtin_amdgcn_readfirstlane(pre_cur);
    const int64_t rows_left = max((int64_t)min(nk, jend * BN) - (int64_t)(jbeg + p_npre) * BN, (int64_t)0);
    const uint64_t ka0 = (uint64_t)(uintptr_t)(kbase + (int64_t)(jbeg + p_npre) * BN * p.k_ss);
    const uint64_t va0 = (uint64_t)(uintptr_t)(vbase + (int64_t)(jbeg + p_npre) * BN * p.v_ss);
    const uint32_t pk_rs[4] = {(uint32_t)ka0, (uint32_t)(ka0 >> 32) & 0xffffu,
                               (uint32_t)min(rows_left * p.k_ss * 2, (int64_t)0x7fffffff), 0x00020000u};
    const uint32_t pv_rs[4] = {(uint32_t)va0, (uint32_t)(va0 >> 32) & 0xffffu,
                               (uint32_t)min(rows_left * p.v_ss * 2, (int64_t)0x7fffffff), 0x00020000u};
    const uint32_t p_ktb = (uint32_t)(BN * p.k_ss * 2), p_vtb = (uint32_t)(BN * p.v_ss * 2);
    // per-tile record counts: the tile's rows inside [jbeg*BN, min(nk, jend*BN)) times the
    // row stride (a single count over the whole range could exceed 2^31 bytes)
    const uint32_t p_krb = (uint32_t)(p.k_ss * 2), p_vrb = (uint32_t)(p.v_ss * 2);
    const int p_rows = (int)rows_left;
    // tiles of this wave: [jbeg, jl]; causal waves stop at their diagonal tile, waves
    // whose rows are all past the sequence have none
    const int wrow0 = m0 + (gqa4 ? 0 : ws) * RB * 32;
    int jl = CAUSAL ? min(jend - 1, (wrow0 + RB * 32 - 1) / BN) : jend - 1;
    if (wrow0 >= nq) jl = jbeg - 1;
    const int p_jl = __builtin_amdgcn_readfirstlane(jl);
    const int p_jbeg = jbeg, p_jend = jend, p_nk = nk;
    const int p_wrow = CAUSAL ? wrow0 : 0x3fffffff;
    if constexpr (std::is_same<T, half_t>::value)
      asm volatile(FAL_PIPE_ASM_F16 : FAL_PIPE_OUTS : FAL_PIPE_INS : FAL_PIPE_CLOBBERS);
    else
      asm volatile(FAL_PIPE_ASM_BF16 : FAL_PIPE_OUTS : FAL_PIPE_INS : FAL_PIPE_CLOBBERS);
    // persistent schedule: the next item's Q slices load while this item's O goes out
    // (buffer loads: rows past the sequence read as zeros; a negative scale, folded into
    // Q, keeps the loads at the item's start)
    if (p.persist && has_next && !negq && next.qt * BMW < next.nq) {
      // one resource over the item's rows (offsets from its first row stay small)
      const int nm0 = next.qt * BMW;
      const T* nqb = (const T*)p.q + (int64_t)next.b * p.q_sb + (int64_t)next.hq * p.q_sh +
                     (int64_t)(next.q_off + nm0) * p.q_ss;
      // (at most 256 rows of a sequence stride below 2^22 elements: the byte counts and
      // offsets below are under 2^31; computed in 64 bits and clamped all the same)
      const __amdgpu_buffer_rsrc_t qrs =
          make_rsrc(nqb, (uint32_t)min((int64_t)min(next.nq - nm0, BMW) * p.q_ss * 2, (int64_t)0x7fffffff));
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int nrow = ((gqa4 ? 0 : w) * RB + rb) * 32 + l32;   // row within the item
        const int qoff = (int)min((int64_t)nrow * p.q_ss * 2 + hh * 16, (int64_t)0x7fffffff);
#pragma unroll
        for (int t = 0; t < KS; ++t)
          qio[rb][t] = __builtin_bit_cast(V8, __builtin_amdgcn_raw_buffer_load_b128(qrs, qoff + t * 32, 0, 0));
      }
      qpre_next = 1;
    }
    // O^T accumulator block g (= (rb*DB + db)*4 + g4) of lane l is at byte
    // ws*kPipeOWave + l*16 + g*kPipeOStr: 16 bytes of a row (MFMA layout)
    const char* wbase = (const char*)smem + ws * kPipeOWave;
    if (p.kchunk) {
      // split-KV partials: back into the accumulator layout
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const f32x4 x = *reinterpret_cast<const f32x4*>(wbase + lane * 16 + ((rb * DB + db) * 4 + g4) * kPipeOStr);
#pragma unroll
            for (int e = 0; e < 4; ++e) oacc[rb][db][g4 * 4 + e] = x[e];
          }
    } else {
      // O and L straight from LDS: each store instruction writes 4 whole rows (16 lanes
      // x 16 bytes per row), where stores from the accumulator layout would write 16
      // bytes into each of 32 rows
      float inv[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const float l_tot = pair_sum(l_run[rb]);
        inv[rb] = l_tot > 0.f ? 1.f / l_tot : 0.f;
        if (hh == 0 && row[rb] < nq)
          lbase[(int64_t)row[rb] * p.l_ss] = l_tot > 0.f ? (m_run[rb] + fast_log2(l_tot)) * kLn2 : -INFINITY;
      }
      const int cch = lane & 15;               // 16-byte chunk of the row
      const int wr0 = m0 + (gqa4 ? 0 : ws) * RB * 32;   // (ws: the wave index as a scalar)
      // one buffer resource over this wave's rows inside the sequence: stores past its
      // end are dropped, so a store needs no branch and no 64-bit address (at most 64
      // rows of a sequence stride below 2^22 elements: offsets below 2^31)
      const __amdgpu_buffer_rsrc_t ors =
          make_rsrc(obase + (int64_t)wr0 * p.o_ss,
                    (uint32_t)min((int64_t)max(min(nq - wr0, RB * 32), 0) * p.o_ss * 2, (int64_t)0x7fffffff));
      const int ovo = ((lane >> 4) * (int)p.o_ss + cch * 8) * 2;
      // per 16 rows: all LDS reads and row factors first, then the stores (one wait, not
      // one per row)
#pragma unroll
      for (int hb = 0; hb < 2 * RB; ++hb) {
        const int rb = hb >> 1;
        f32x4 a0[4], a1[4];
        float iv[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int l32w = (hb & 1) * 16 + jj * 4 + (lane >> 4);
          const int g = rb * 16 + cch;
          a0[jj] = *reinterpret_cast<const f32x4*>(wbase + l32w * 16 + g * kPipeOStr);
          a1[jj] = *reinterpret_cast<const f32x4*>(wbase + (32 + l32w) * 16 + g * kPipeOStr);
          iv[jj] = __shfl(inv[rb], l32w);
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = hb * 16 + jj * 4 + (lane >> 4);   // row of the wave, 0..63
          V8 h;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            h[e] = (T)(a0[jj][e] * iv[jj]);
            h[4 + e] = (T)(a1[jj][e] * iv[jj]);
          }
          buffer_store16(ors, ovo + (r - (lane >> 4)) * (int)p.o_ss * 2, __builtin_bit_cast(u32x4, h));
        }
      }
      stored = true;
    }
    if (p.persist) __syncthreads();   // every wave has its O out of LDS (the next item reuses it)
  } else {
  if (jbeg < jend) load_tile(jbeg, 0);
  // Tiles that need no mask for any row of the workgroup: straight-line, unrolled by
  // two so both LDS buffer offsets are constants (tile j uses buffer (j - jbeg) & 1).
  const int fend = min(nfull, jend);
  int j = jbeg;
  for (; j + 1 < fend; j += 2) {
    step(std::false_type{}, j, 0);
    step(std::false_type{}, j + 1, 1);
  }
  if (j < fend) {
    step(std::false_type{}, j, 0);
    ++j;
  }
  // Diagonal and tail tiles; waves whose rows all precede the tile only keep the
  // pipeline (barrier + prefetch) going.
  for (; j < jend; ++j) {
    wait_vmcnt0();
    __syncthreads();
    if (j + 1 < jend) load_tile(j + 1, (j + 1 - jbeg) & 1);
    if (!CAUSAL || j * BN <= wrow_hi) tile_body(std::true_type{}, j, (j - jbeg) & 1);
  }

  }

  if (p.kchunk) {
    // split-KV: this split's unnormalised O, its reference max m and its sum l
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const float l_tot = pair_sum(l_run[rb]);
      if (row[rb] < nq) {
        const int64_t prow = ((int64_t)(b * p.Hq + hq) * p.nsplit + it.split) * p.Nq + row[rb];
        float* po = p.part_o + prow * D;
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            f32x4 x;
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = oacc[rb][db][g4 * 4 + e];
            *reinterpret_cast<f32x4*>(po + db * 32 + g4 * 8 + hh * 4) = x;
          }
        if (hh == 0) *reinterpret_cast<float2*>(p.part_ml + prow * 2) = make_float2(m_run[rb], l_tot);
      }
    }
    return 0;
  }

  // ---- epilogue: normalise, write O and L ----
  // Through LDS when the tile buffers hold the workgroup's O: each wave stages its rows
  // (fp16/bf16, rows padded by 16 bytes) and writes them back row-wise, 16 contiguous
  // bytes per lane, so every store instruction covers whole rows; from the accumulator
  // layout each store would put 8 bytes into each of 32 rows.
  constexpr int OROW = D * 2 + 16;
  constexpr bool ROWST = !PIPE && (NW * RB * 32 * OROW <= NSLOT * 2 * PART * 2);
  if (ROWST && !stored) {
    __syncthreads();   // every wave is done with the last K/V tile
    char* wst = (char*)smem + w * (RB * 32 * OROW);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const float l_tot = pair_sum(l_run[rb]);
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          V4 h;
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = (T)(oacc[rb][db][g4 * 4 + e] * inv);
          *reinterpret_cast<V4*>(wst + (rb * 32 + l32) * OROW + (db * 32 + g4 * 8 + hh * 4) * 2) = h;
        }
      if (hh == 0 && row[rb] < nq)
        lbase[(int64_t)row[rb] * p.l_ss] = l_tot > 0.f ? (m_run[rb] + fast_log2(l_tot)) * kLn2 : -INFINITY;
    }
    // (one wave's LDS accesses complete in order: its rows are staged before these reads)
    constexpr int CPRW = D / 8;
    const int wr0 = m0 + w * RB * 32;
#pragma unroll
    for (int i = lane; i < RB * 32 * CPRW; i += 64) {
      const int r = i / CPRW, c = i % CPRW;
      const u32x4 x = *reinterpret_cast<const u32x4*>(wst + r * OROW + c * 16);
      if (wr0 + r < nq) st_u4(obase + (int64_t)(wr0 + r) * p.o_ss + c * 8, x);
    }
    stored = true;
  }
#pragma unroll
  for (int rb = 0; rb < RB && !stored; ++rb) {
    const float l_tot = pair_sum(l_run[rb]);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    if (row[rb] < nq) {
      T* orow = obase + (int64_t)row[rb] * p.o_ss;
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          V4 h;
#pragma unroll
          for (int e = 0; e < 4; ++e) h[e] = (T)(oacc[rb][db][g4 * 4 + e] * inv);
          *reinterpret_cast<V4*>(orow + db * 32 + g4 * 8 + hh * 4) = h;
        }
      if (hh == 0) {
        float L = -INFINITY;
        if (l_tot > 0.f) L = (m_run[rb] + fast_log2(l_tot)) * kLn2;
        lbase[(int64_t)row[rb] * p.l_ss] = L;
      }
    }
  }
  // Persistent schedule: the next item's first two K/V tiles are copied after this item's
  // O stores, so their latency overlaps those stores and the next item's Q loads.
  if (PIPE && p.persist && has_next) pre_next = issue_first2(next);
  return pre_next | (qpre_next << 2);
}

// Persistent schedule (pipelined head_dim-128 kernel, batched calls with at least two
// items per CU; an item is 64 rows of four heads under gqa4, else 256 rows of one head):
// a grid of one workgroup per CU walks pairs of query tiles, (T-1-p, p) under a causal mask so every pair costs the same, (2p, 2p+1) without.  The
// pairs are numbered unit-major (unit = batch, KV head, group of four query heads) and
// round r gives workgroup w pair r*G + w', w' the XCD-major rank of w, so the
// workgroups of one XCD work on neighbouring pairs of one unit (shared K/V in that
// XCD's L2).  Between items no workgroup ends: the previous item's O stores are still
// in flight while the next item's Q and first K/V tiles load.
template <bool CAUSAL>
__device__ __forceinline__ bool fwd_item_persist(const FwdParams& p, FwdItem& it, int i) {
  const int G = gridDim.x, w = blockIdx.x;
  const int wr = (G & 7) == 0 ? (w & 7) * (G >> 3) + (w >> 3) : w;
  const int T = p.n_qtiles;
  const int npair = (T + 1) >> 1;
  const int g = p.Hq / p.Hkv, ng = p.gqa4 ? g >> 2 : g;   // workgroup units per KV head
  // (the host keeps B * Hkv * ng * npair below 2^31)
  const uint32_t e = (uint32_t)(i >> 1) * (uint32_t)G + (uint32_t)wr;
  if (e >= (uint32_t)(p.B * p.Hkv * ng * npair)) return false;
  const int u = (int)(e / (uint32_t)npair), pp = (int)(e % (uint32_t)npair);
  const int half = i & 1;
  it.qt = CAUSAL ? (half ? pp : T - 1 - pp) : 2 * pp + half;
  if (CAUSAL && half && pp == T - 1 - pp) it.qt = T;   // odd T: the middle tile has no partner
  const int hg = (int)((uint32_t)u % (uint32_t)ng), bh = (int)((uint32_t)u / (uint32_t)ng);
  it.b = (int)((uint32_t)bh / (uint32_t)p.Hkv);
  it.hq = __builtin_amdgcn_readfirstlane((bh - it.b * p.Hkv) * g +
                                         (p.gqa4 ? hg * 4 + (int)(threadIdx.x >> 6) : hg));
  it.q_off = 0;
  it.k_off = 0;
  it.nq = p.Nq;
  it.nk = p.Nk;
  it.split = 0;
  it.pre = 0;
  it.qpre = 0;
  return true;
}

// Packed sequences under the four-heads layout with a work list of pairs (schedule
// order 4): workgroup (pair, KV head, head quad) takes the pair's query tiles nt-1-j and
// j of one sequence, heaviest first, through the same two-item walk as the persistent
// grid (the second item's Q and first K/V tiles load during the first one's epilogue).
// i = 0: the heavy tile; i = 1: the light one unless it is the same tile.
template <bool CAUSAL>
__device__ __forceinline__ bool fwd_item_vpair(const FwdParams& p, FwdItem& it, int i) {
  if (i > 1) return false;
  const int g = p.Hq / p.Hkv, ng = g >> 2;
  const int k8 = blockIdx.x >> 3;
  const int grp = (k8 / ng) * 8 + (blockIdx.x & 7);
  const int item = grp / p.Hkv;
  if (item >= p.n_qtiles) return false;
  const int2 wk = p.work[item];
  const int seq = __builtin_amdgcn_readfirstlane(wk.x), j = __builtin_amdgcn_readfirstlane(wk.y);
  if (seq < 0) return false;
  int qo, nq, ko, nk;
  seg_bounds(p.cu_q, seq, p.total_q, qo, nq);
  seg_bounds(p.cu_k, seq, p.total_k, ko, nk);
  // (uniform values: the pipelined loop takes them as scalar operands)
  it.q_off = __builtin_amdgcn_readfirstlane(qo);
  it.nq = __builtin_amdgcn_readfirstlane(nq);
  it.k_off = __builtin_amdgcn_readfirstlane(ko);
  it.nk = __builtin_amdgcn_readfirstlane(nk);
  const int nt = cdiv(it.nq, 64);
  const int hi = nt - 1 - j, lo = j;
  if (i == 1 && lo >= hi) return false;
  it.qt = i == 0 ? hi : lo;
  it.b = 0;
  it.hq = __builtin_amdgcn_readfirstlane((grp % p.Hkv) * g + (k8 % ng) * 4 + (int)(threadIdx.x >> 6));
  it.split = 0;
  it.pre = 0;
  it.qpre = 0;
  return true;
}

// VPAIR: packed sequences, each workgroup walking the two items of one pair of the
// work list (fwd_item_vpair); a separate instantiation, so the batched kernel keeps
// its own register allocation.
template <class T, int D, int NW, int BN, bool CAUSAL, int RB, bool VPAIR = false>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu((RB == 2 && D >= 128) ? 1 : (D <= 128 ? FAL_FWD_WPE : 1), 8)))
fwd_kernel(FwdParams p) {
  constexpr bool PIPE = FAL_FWD_PIPE && D == 128 && RB == 2 && NW == 4 && BN == 64 && !FAL_PRESCALE_FP16;
  constexpr int PART = BN * SwizzledTile<D>::CPR * 8;
  constexpr int NSLOT = PIPE ? 4 : 2;
  // the pipelined loop's O hand-off (4 x kPipeOWave bytes) reaches past the 128 KB ring
  constexpr int NSMEM = PIPE ? (4 * kPipeOWave) / 2 : NSLOT * 2 * PART;
  __shared__ __attribute__((aligned(1024))) T smem[NSMEM];
  FwdItem it;
  if (PIPE && p.persist) {
    // items past the tile count (qt >= n_qtiles) are skipped inside fwd_body; each item
    // ends with a barrier after its O left LDS and may issue the next item's first copies
    FwdItem nx;
    vec8<T> qio[RB][D / 16];
    auto item = [&](FwdItem& x, int i) {
      if constexpr (VPAIR)
        return fwd_item_vpair<CAUSAL>(p, x, i);
      else
        return fwd_item_persist<CAUSAL>(p, x, i);
    };
    bool have = item(it, 0);
    for (int i = 0; have; ++i) {
      const bool more = item(nx, i + 1);
      const int r = fwd_body<T, D, NW, BN, CAUSAL, RB>(p, it, smem, nx, more, qio);
      nx.pre = r & 3;
      nx.qpre = r >> 2;
      it = nx;
      have = more;
    }
    return;
  }
  // ---- resolve this workgroup's (batch/sequence, head, query tile) ----
  if (!fwd_item<CAUSAL>(p, it, p.gqa4 ? 64 : NW * 32 * RB)) return;
  vec8<T> qio[RB][D / 16];
  fwd_body<T, D, NW, BN, CAUSAL, RB>(p, it, smem, it, false, qio);
}

// ---------------------------------------------------------------------------
// Split-KV combine: one group of D/8 lanes per query row merges the row's splits,
// O = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s with M = max_s m_s, and writes
// O and L = (M + log2 sum) * ln 2 (-inf for a row with no visible key).
// ---------------------------------------------------------------------------
template <class T, int D, int BM, int BN, bool CAUSAL>
__global__ void __launch_bounds__(256)
fwd_combine_kernel(FwdParams p) {
  constexpr int G = D / 8;              // lanes per row, 8 columns each
  if (threadIdx.x >= (256 / G) * G) return;
  const int r = blockIdx.x * (256 / G) + threadIdx.x / G;
  const int c = (threadIdx.x % G) * 8;
  const int rows = p.B * p.Hq * p.Nq;
  if (r >= rows) return;
  const int n = r % p.Nq;
  const int bh = r / p.Nq;
  const int m0 = (n / BM) * BM;
  const int kend = CAUSAL ? min(p.Nk, m0 + BM) : p.Nk;
  const int ns = max(1, cdiv(cdiv(kend, BN), p.kchunk));
  const int64_t base = (int64_t)bh * p.nsplit * p.Nq + n;   // split s: base + s * Nq
  float M = -INFINITY;
  for (int s = 0; s < ns; ++s) M = fmaxf(M, p.part_ml[(base + (int64_t)s * p.Nq) * 2]);
  const float Mu = M == -INFINITY ? 0.f : M;
  float lsum = 0.f;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int s = 0; s < ns; ++s) {
    const int64_t pr = base + (int64_t)s * p.Nq;
    const float2 ml = *reinterpret_cast<const float2*>(p.part_ml + pr * 2);
    const float wgt = ml.y > 0.f ? fast_exp2(ml.x - Mu) : 0.f;
    lsum = fmaf(wgt, ml.y, lsum);
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(p.part_o + pr * D + c);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(p.part_o + pr * D + c + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      acc[e] = fmaf(wgt, x0[e], acc[e]);
      acc[e + 4] = fmaf(wgt, x1[e], acc[e + 4]);
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  const int b = bh / p.Hq, hq = bh % p.Hq;
  vec8<T> h;
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = (T)(acc[e] * inv);
  st_u4((T*)p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + (int64_t)n * p.o_ss + c, __builtin_bit_cast(u32x4, h));
  if (c == 0)
    p.lse[(int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)n * p.l_ss] =
        lsum > 0.f ? (Mu + fast_log2(lsum)) * kLn2 : -INFINITY;
}

// ---------------------------------------------------------------------------
// Varlen scheduler: turns cu_seqlens into a list of (sequence, tile) work items
// on the device (no host synchronisation).  Items are bucketed by tile index so
// that, for causal attention, the most expensive tiles start first
// (descending=1: tile t costs ~t+1 KV tiles in the forward) or, for the KV-outer
// backward, the tiles with the most query rows below them start first
// (descending=0).  Unused trailing slots get (-1, -1).
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(1024)
varlen_schedule_kernel(const int* __restrict__ cu, int num_seqs, int rows, int tile, int nbuckets,
                       int descending, int2* __restrict__ work, int capacity, ZeroRows zero) {
  extern __shared__ int sh[];            // [nbuckets] counts, then [nbuckets] cursors
  int* cnt = sh;
  int* cur = sh + nbuckets;
  __shared__ int seg_end;
  for (int i = threadIdx.x; i < nbuckets; i += blockDim.x) cnt[i] = 0;
  if (threadIdx.x == 0) seg_end = 0;
  __syncthreads();
  if (zero.a) {
    // rows [0, start of segment 0) and [end of the last segment, rows) are in no segment
    // (for a monotone cu_seqlens): write zeros there, as the reference's per-sequence
    // backward leaves them (zeros_like, flash_attn.py:125-131)
    for (int s = threadIdx.x; s < num_seqs; s += blockDim.x) {
      int off, len;
      seg_bounds(cu, s, rows, off, len);
      atomicMax(&seg_end, off + len);
    }
    __syncthreads();
    int first = rows, flen = 0;
    if (num_seqs > 0) seg_bounds(cu, 0, rows, first, flen);
    const int last = seg_end;
    const int cpr = zero.heads * (zero.d / 8);   // 16-byte chunks per row
    const int nlo = first, nhi = rows - max(last, first);
    const int64_t nchunks = (int64_t)(nlo + nhi) * cpr;
    for (int64_t i = threadIdx.x; i < nchunks; i += blockDim.x) {
      const int rr = (int)(i / cpr);
      const int r = rr < nlo ? rr : max(last, first) + (rr - nlo);
      const int ch = (int)(i % cpr);
      const int h = ch / (zero.d / 8), c8 = (ch % (zero.d / 8)) * 8;
      st_u4(static_cast<half_t*>(zero.a) + (int64_t)r * zero.a_row + (int64_t)h * zero.a_head + c8,
            u32x4{0, 0, 0, 0});
      if (zero.b)
        st_u4(static_cast<half_t*>(zero.b) + (int64_t)r * zero.b_row + (int64_t)h * zero.b_head + c8,
              u32x4{0, 0, 0, 0});
    }
  }
  if (descending >= 2) {
    // Grouped by sequence: longest sequences first (bucketed by tile count), each
    // sequence's tiles contiguous; 2: last tile first (query-outer causal work grows
    // with the tile index), 3: first tile first (KV-outer causal work shrinks with it),
    // 4: pairs (s, j) for j < ceil(nt/2), the tiles nt-1-j and j of one workgroup.
    // The workgroups an XCD runs at once then share one or two sequences' data in L2.
    for (int s = threadIdx.x; s < num_seqs; s += blockDim.x) {
      int off, len;
      seg_bounds(cu, s, rows, off, len);
      const int nt = cdiv(len, tile);
      if (nt > 0) atomicAdd(&cnt[min(nt - 1, nbuckets - 1)], descending == 4 ? (nt + 1) / 2 : nt);
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int acc = 0;
      for (int k = nbuckets - 1; k >= 0; --k) {
        cur[k] = acc;
        acc += cnt[k];
      }
      cnt[0] = acc;
    }
    __syncthreads();
    const int total = cnt[0];
    for (int s = threadIdx.x; s < num_seqs; s += blockDim.x) {
      int off, len;
      seg_bounds(cu, s, rows, off, len);
      const int nt = cdiv(len, tile);
      if (nt == 0) continue;
      const int ne = descending == 4 ? (nt + 1) / 2 : nt;
      const int pos = atomicAdd(&cur[min(nt - 1, nbuckets - 1)], ne);
      for (int t = 0; t < ne; ++t)
        if (pos + t < capacity) work[pos + t] = make_int2(s, descending == 2 ? nt - 1 - t : t);
    }
    for (int i = total + threadIdx.x; i < capacity; i += blockDim.x) work[i] = make_int2(-1, -1);
    return;
  }
  for (int s = threadIdx.x; s < num_seqs; s += blockDim.x) {
    int off, len;
    seg_bounds(cu, s, rows, off, len);
    const int nt = cdiv(len, tile);
    for (int t = 0; t < nt; ++t) atomicAdd(&cnt[min(t, nbuckets - 1)], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = 0;
    for (int k = 0; k < nbuckets; ++k) {
      const int bkt = descending ? (nbuckets - 1 - k) : k;
      cur[bkt] = acc;
      acc += cnt[bkt];
    }
    cnt[0] = acc;   // total items
  }
  __syncthreads();
  const int total = cnt[0];
  for (int s = threadIdx.x; s < num_seqs; s += blockDim.x) {
    int off, len;
    seg_bounds(cu, s, rows, off, len);
    const int nt = cdiv(len, tile);
    for (int t = 0; t < nt; ++t) {
      const int pos = atomicAdd(&cur[min(t, nbuckets - 1)], 1);
      if (pos < capacity) work[pos] = make_int2(s, t);
    }
  }
  for (int i = total + threadIdx.x; i < capacity; i += blockDim.x) work[i] = make_int2(-1, -1);
}

// ---------------------------------------------------------------------------
// Host-side launchers
// ---------------------------------------------------------------------------
#ifndef FAL_FWD_RB128
#define FAL_FWD_RB128 2   // 32-row blocks per wave for head_dim 128 (2: the pipelined loop)
#endif
#ifndef FAL_FWD_NW128
#define FAL_FWD_NW128 4   // waves per workgroup for head_dim 128
#endif
#ifndef FAL_FWD_BN32
#define FAL_FWD_BN32 128   // head_dim 32: 128-key tiles (+25% causal, +3% non-causal over 64)
#endif
#ifndef FAL_FWD_BN64
#define FAL_FWD_BN64 FAL_FWD_BN
#endif
#ifndef FAL_FWD_RB32
#define FAL_FWD_RB32 1
#endif
#ifndef FAL_FWD_RB64
#define FAL_FWD_RB64 1
#endif
#ifndef FAL_FWD_RB128_VARLEN
#define FAL_FWD_RB128_VARLEN 1   // varlen keeps 128-row tiles (less waste on short sequences: +3% on C4)
#endif
// VARLEN: the configuration of packed-sequence calls (cu_seqlens set)
template <int D, bool VARLEN = false>
struct FwdCfg {
  static constexpr int NW = D == 128 ? FAL_FWD_NW128 : 4;
  static constexpr int BN = (D >= 256) ? 32 : D == 32 ? FAL_FWD_BN32 : D == 64 ? FAL_FWD_BN64 : FAL_FWD_BN;
  static constexpr int RB = D == 128 ? (VARLEN ? FAL_FWD_RB128_VARLEN : FAL_FWD_RB128)
                            : D == 32 ? FAL_FWD_RB32 : D == 64 ? FAL_FWD_RB64 : 1;
};

template <class T, int D, bool VARLEN>
static hipError_t launch_fwd_t(const FwdParams& p, int causal, dim3 grid, hipStream_t st) {
  constexpr int NW = FwdCfg<D, VARLEN>::NW, BN = FwdCfg<D, VARLEN>::BN, RB = FwdCfg<D, VARLEN>::RB;
  if constexpr (!VARLEN && D == 128 && RB == 2) {
    if (p.cu_q && p.persist) {
      if (causal)
        hipLaunchKernelGGL((fwd_kernel<T, D, NW, BN, true, RB, true>), grid, dim3(NW * 64), 0, st, p);
      else
        hipLaunchKernelGGL((fwd_kernel<T, D, NW, BN, false, RB, true>), grid, dim3(NW * 64), 0, st, p);
      return hipGetLastError();
    }
  }
  if (causal)
    hipLaunchKernelGGL((fwd_kernel<T, D, NW, BN, true, RB>), grid, dim3(NW * 64), 0, st, p);
  else
    hipLaunchKernelGGL((fwd_kernel<T, D, NW, BN, false, RB>), grid, dim3(NW * 64), 0, st, p);
  return hipGetLastError();
}
template <int D>
static hipError_t launch_fwd_d(const FwdParams& p, int causal, dim3 grid, hipStream_t st) {
  // packed sequences keep their own tile configuration, except under the four-heads
  // layout, which runs the batched (pipelined) kernel over the work list
  if (p.cu_q && !p.gqa4)
    return p.bf16 ? launch_fwd_t<bf16_t, D, true>(p, causal, grid, st)
                  : launch_fwd_t<half_t, D, true>(p, causal, grid, st);
  return p.bf16 ? launch_fwd_t<bf16_t, D, false>(p, causal, grid, st)
                : launch_fwd_t<half_t, D, false>(p, causal, grid, st);
}

template <int D, bool VARLEN = false>
constexpr int fwd_bm() { return FwdCfg<D, VARLEN>::NW * 32 * FwdCfg<D, VARLEN>::RB; }

template <int D>
constexpr int fwd_bn() { return FwdCfg<D>::BN; }

int fwd_block_n(int d) {
  switch (d) {
    case 32: return fwd_bn<32>();
    case 64: return fwd_bn<64>();
    case 96: return fwd_bn<96>();
    case 128: return fwd_bn<128>();
    default: return fwd_bn<256>();
  }
}

#ifndef FAL_FWD_SPLIT
#define FAL_FWD_SPLIT 1   // split the key range of grids smaller than the GPU
#endif
#ifndef FAL_FWD_SPLIT_MIN_TILES
#define FAL_FWD_SPLIT_MIN_TILES 4   // key tiles per split, at least
#endif

// Split-KV plan.  Measured on MI355X (workgroup timestamps, head_dim 64): a workgroup
// takes about 5 us of start-up and epilogue plus about 0.7 us per key tile, so a grid
// with fewer workgroups than CUs ends with its longest chain of key tiles.  Splitting
// the chain costs the partial outputs: fp32 rows written back to HBM when the kernel
// ends (about 2.5 TB/s) and read again by the combine kernel, plus about 5 us for that
// second launch.  A split is taken only when the chain time it saves exceeds that cost
// (so C1, 2 x 8 heads x 1024 rows, stays whole: 16 tiles save 5.6 us at two splits but
// cost 11.7 us), with the split count that saves the most.
size_t fwd_split_plan(int64_t B, int64_t Hq, int64_t Nq, int64_t Nk, int d, int causal, int* kchunk, int* nsplit) {
  *kchunk = 0;
  *nsplit = 1;
  if (!FAL_FWD_SPLIT || B <= 0 || Nq <= 0 || Nk <= 0) return 0;
  const int64_t bm = fwd_block_m(d), bn = fwd_block_n(d);
  const int64_t nwg = B * Hq * ((Nq + bm - 1) / bm);
  const int64_t kspan = causal ? std::min<int64_t>(Nk, (Nq + bm - 1) / bm * bm) : Nk;
  const int64_t maxtiles = (kspan + bn - 1) / bn;
  if (nwg >= 256 || maxtiles < 2 * FAL_FWD_SPLIT_MIN_TILES) return 0;
  const double us_per_tile = 0.7 * (d / 64.0 < 1.0 ? 1.0 : d / 64.0) * (bn / 64.0);
  double best = 0.0;
  for (int64_t ns = 2; ns <= 64 && nwg * ns <= 2048; ns *= 2) {
    const int64_t chunk = std::max<int64_t>(FAL_FWD_SPLIT_MIN_TILES, (maxtiles + ns - 1) / ns);
    const int64_t nsr = (maxtiles + chunk - 1) / chunk;
    if (nsr < 2) break;
    const double bytes = (double)(B * Hq * nsr * Nq) * (d + 2) * 4.0;
    const double gain = us_per_tile * (double)(maxtiles - chunk) - 5.0 - 2.0 * bytes / 2.5e6;
    if (gain > best && bytes <= (double)(size_t(256) << 20)) {
      best = gain;
      *kchunk = (int)chunk;
      *nsplit = (int)nsr;
    }
  }
  if (!*kchunk) return 0;
  return (size_t)(B * Hq * *nsplit * Nq) * (size_t)(d + 2) * sizeof(float) + 256;
}

template <class T, int D>
static hipError_t launch_combine_t(const FwdParams& p, int causal, hipStream_t st) {
  constexpr int BM = FwdCfg<D>::NW * 32 * FwdCfg<D>::RB, BN = FwdCfg<D>::BN;
  const int64_t rows = (int64_t)p.B * p.Hq * p.Nq;
  const dim3 grid((unsigned)((rows + 256 / (D / 8) - 1) / (256 / (D / 8))));
  if (causal)
    hipLaunchKernelGGL((fwd_combine_kernel<T, D, BM, BN, true>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((fwd_combine_kernel<T, D, BM, BN, false>), grid, dim3(256), 0, st, p);
  return hipGetLastError();
}
template <int D>
static hipError_t launch_combine_d(const FwdParams& p, int causal, hipStream_t st) {
  return p.bf16 ? launch_combine_t<bf16_t, D>(p, causal, st) : launch_combine_t<half_t, D>(p, causal, st);
}
hipError_t launch_fwd_combine(const FwdParams& p, int d, int causal, hipStream_t st) {
  switch (d) {
    case 32: return launch_combine_d<32>(p, causal, st);
    case 64: return launch_combine_d<64>(p, causal, st);
    case 96: return launch_combine_d<96>(p, causal, st);
    case 128: return launch_combine_d<128>(p, causal, st);
    case 256: return launch_combine_d<256>(p, causal, st);
    default: return hipErrorInvalidValue;
  }
}

#ifndef FAL_FWD_GQA4
#define FAL_FWD_GQA4 1
#endif
// True when a batched (not split) forward of this head dim and head ratio runs the
// pipelined kernel with the four-heads-per-workgroup layout (FwdParams::gqa4).
bool fwd_pipe_ok(int d) {
  return FAL_FWD_PIPE && !FAL_PRESCALE_FP16 && d == 128 && FwdCfg<128>::RB == 2 && FwdCfg<128>::NW == 4 &&
         FwdCfg<128>::BN == 64;
}
bool fwd_gqa4_ok(int d, int64_t heads_q, int64_t heads_kv) {
  return FAL_FWD_GQA4 && fwd_pipe_ok(d) && heads_kv > 0 && (heads_q / heads_kv) % 4 == 0;
}

int fwd_block_m(int d) {
  switch (d) {
    case 32: return fwd_bm<32>();
    case 64: return fwd_bm<64>();
    case 96: return fwd_bm<96>();
    case 128: return fwd_bm<128>();
    default: return fwd_bm<256>();
  }
}

int fwd_block_m_varlen(int d) {
  switch (d) {
    case 32: return fwd_bm<32, true>();
    case 64: return fwd_bm<64, true>();
    case 96: return fwd_bm<96, true>();
    case 128: return fwd_bm<128, true>();
    default: return fwd_bm<256, true>();
  }
}

hipError_t launch_fwd(const FwdParams& p, int d, int causal, dim3 grid, hipStream_t st) {
  switch (d) {
    case 32: return launch_fwd_d<32>(p, causal, grid, st);
    case 64: return launch_fwd_d<64>(p, causal, grid, st);
    case 96: return launch_fwd_d<96>(p, causal, grid, st);
    case 128: return launch_fwd_d<128>(p, causal, grid, st);
    case 256: return launch_fwd_d<256>(p, causal, grid, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_varlen_schedule(const int* cu, int num_seqs, int rows, int tile, int nbuckets, int descending,
                                  int2* work, int capacity, hipStream_t st, const ZeroRows* zero) {
  const size_t shmem = 2 * sizeof(int) * (size_t)nbuckets;
  ZeroRows z{};
  if (zero) z = *zero;
  hipLaunchKernelGGL(varlen_schedule_kernel, dim3(1), dim3(1024), shmem, st, cu, num_seqs, rows, tile,
                     nbuckets, descending, work, capacity, z);
  return hipGetLastError();
}

}  // namespace fal

// KV-cache decode for gfx950: split-K over the cache plus a log-sum-exp combine.
//
// The reference has no decode kernel: for q_len != kv_len it runs eager PyTorch
// (flash_attn_legacy/integrations.py:77-98): repeat K/V over the GQA group,
// s = q k^T * scale (+ additive mask), softmax over the keys, @ v.  This file computes
// the same result without materialising the repeated K/V or the score row.
//
// Work items (sequence, split): for batches of up to 64 sequences each split workgroup
// derives its own item from cache_seqlens (full splits first); larger batches use a
// schedule kernel that builds a longest-first list on the device.  Neither needs a
// host synchronisation.
// Split kernel: one workgroup per (work item, KV head, group of up to 16 query heads)
// covers `chunk` cache rows.
// * The query heads of the KV head ride in one 16x16x32 MFMA tile: S^T = K Q^T with
//   M = 16 cache rows and N = the heads, so every K/V byte is read once from HBM for
//   the whole group.
// * Each wave streams its own 32-row steps, two steps ahead: K rows are loaded
//   straight into the A operand, V rows go through a wave-private LDS ring (buffer
//   loads with the nontemporal bit) and come back transposed (ds_read_b64_tr_b16) as
//   the A operand of O^T = V^T P^T.
// * The waves' (max, sum, O) are merged in LDS in a fixed order (the output is
//   deterministic); the workgroup writes one normalised partial O (fp32) and its
//   log2-domain LSE.
// Combine kernel: one wave per (sequence, query head) merges the splits' partials.
#include <type_traits>

#include "fal_kernels.h"

namespace fal {

// Waves per workgroup.  Each wave streams its own 32-row steps of the split with a
// two-step prefetch: K rows straight into MFMA operand registers, V rows into a
// wave-private LDS ring (read back transposed).  No workgroup barrier until the
// final merge.
#ifndef FAL_DEC_NW
#define FAL_DEC_NW 4
#endif
#ifndef FAL_DEC_VAUX
#define FAL_DEC_VAUX 2   // cache-policy bits of the V loads: nt (read once, evict first)
#endif
// K rows loaded a whole 128-byte line per instruction (8 rows x 128 B, both halves of a
// pair of MFMA k-steps), swapped into the MFMA layout with two row_ror:8 DPP moves per
// dword, so the K loads can carry the nontemporal bit too (a half-line load with nt
// drops the line before the next instruction reads its other half).
#ifndef FAL_DEC_KLINE
#define FAL_DEC_KLINE 1
#endif
#ifndef FAL_DEC_KAUX
#define FAL_DEC_KAUX (FAL_DEC_KLINE ? 2 : 0)
#endif

// A pair of K loads in line order -> MFMA order.  Loaded: a = (lane n < 8: row n chunk g;
// n >= 8: row n-8 chunk 4+g), b = (n < 8: row n+8 chunk g; n >= 8: row n chunk 4+g)
// for lane 16g + n.  Wanted: a = row n chunk g, b = row n chunk 4+g.  Lanes 8-15 of
// each 16-lane row take b from 8 lanes below, lanes 0-7 take a from 8 lanes above
// (row_ror:8; bank_mask selects 4-lane banks).
template <class V8>
__device__ __forceinline__ void kline_unswap(V8& a, V8& b) {
  auto ua = __builtin_bit_cast(u32x4, a);
  auto ub = __builtin_bit_cast(u32x4, b);
  u32x4 na, nb;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    na[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)ua[i], (int)ub[i], 0x128, 0xf, 0xc, false);
    nb[i] = (uint32_t)__builtin_amdgcn_update_dpp((int)ub[i], (int)ua[i], 0x128, 0xf, 0x3, false);
  }
  a = __builtin_bit_cast(V8, na);
  b = __builtin_bit_cast(V8, nb);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

// Combine with the value of the lanes 16 and 32 apart (the four 16-lane rows).
__device__ __forceinline__ float rows4_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  return pair_max(x);
}
__device__ __forceinline__ float rows4_sum(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  return pair_sum(x);
}

// V slice: 16 cache rows x D columns in 16-byte chunks, chunk index XOR-swizzled by
// the row so a transposed read of 16 rows x 32 bytes spreads over all banks.
template <int D>
__device__ __forceinline__ int vswz(int r) {
  return D == 96 ? (r & 3) : (r & ((D / 8 < 16 ? D / 8 : 16) - 1));
}

// Work item `item` for a batch of at most 64 sequences, computed by every wave from
// cache_seqlens (one load per lane), so no schedule kernel runs first: every full split
// of every sequence (sequence-major), then the shorter last splits, longest first (ties
// in sequence order), as the schedule kernel orders them.  False past the last item.
__device__ __forceinline__ bool decode_item_small(const DecodeParams& p, int item, int& b, int& split) {
  const int lane = threadIdx.x & 63;
  const int L = lane < p.B ? min(max(p.seqlens[lane], 0), p.max_seqlen) : 0;
  const int nf = L / p.chunk;
  int inc = nf;   // inclusive prefix sum of the full splits over the sequences
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o);
    if (lane >= o) inc += t;
  }
  const int F = __shfl(inc, 63);
  if (item < F) {
    const int bl = __builtin_ctzll(__ballot(inc > item));
    b = bl;
    split = item - (__shfl(inc, bl) - __shfl(nf, bl));
    return true;
  }
  const int rem = L % p.chunk;
  const unsigned long long part = __ballot(rem != 0);
  const int j = item - F;
  if (j >= __popcll(part)) return false;
  int rank = 0;
  for (int k = 0; k < p.B; ++k) {
    const int rk = __builtin_amdgcn_readlane(rem, k);
    rank += (rk > rem || (rk == rem && k < lane)) ? 1 : 0;
  }
  const int bl = __builtin_ctzll(__ballot(rem != 0 && rank == j));
  b = bl;
  split = __shfl(nf, bl);
  return true;
}

template <class T, int D, int NW>
__global__ void __launch_bounds__(NW * 64)
decode_split_kernel(DecodeParams p) {
  constexpr int KS = D / 32;              // 16x16x32 k-steps over the head dim
  constexpr int DBN = D / 16;             // 16-wide output blocks
  constexpr int CPR = D / 8;              // 16-byte chunks per row
  constexpr int SLICE = 16 * CPR * 8;     // elements of one 16-row V slice
  constexpr int VI = 16 * CPR / 64;       // direct loads per V slice
  constexpr int LPS = 2 * KS + 2 * VI;    // loads issued per 32-row step
  static_assert(16 * CPR % 64 == 0, "slice must be whole load instructions");
  using V8 = vec8<T>;
  __shared__ __attribute__((aligned(1024))) T vsm[NW][4 * SLICE];   // 2 steps x 2 slices
  __shared__ float m_s[NW][16];
  __shared__ float l_s[NW][16];
  __shared__ float inv_s[16];

  const int nhg = cdiv(p.Hq / p.Hkv, 16);
  const int heads_tiles = p.Hkv * nhg;
  int b, split;
  if (p.work) {
    const int2 wk = p.work[blockIdx.x / heads_tiles];
    if (wk.x < 0) return;
    b = wk.x;
    split = wk.y;
  } else {
    if (!decode_item_small(p, (int)(blockIdx.x / heads_tiles), b, split)) return;
    b = __builtin_amdgcn_readfirstlane(b);
    split = __builtin_amdgcn_readfirstlane(split);
  }
  const int hkv = (blockIdx.x % heads_tiles) / nhg;
  const int hg = (blockIdx.x % heads_tiles) % nhg;
  const int L = min(max(p.seqlens[b], 0), p.max_seqlen);
  const int k_begin = split * p.chunk;
  if (k_begin >= L) return;
  const int k_end = min(L, k_begin + p.chunk);
  const int nsteps = cdiv(k_end - k_begin, 32);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int ws = __builtin_amdgcn_readfirstlane(w);
  const int l16 = lane & 15;
  const int g4 = lane >> 4;
  const int G = p.Hq / p.Hkv;
  const int hbase = hkv * G + hg * 16;           // first query head of this tile
  const int nh = min(16, G - hg * 16);


  const T* kbase = (const T*)p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh;
  const T* vbase = (const T*)p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh;
  // K: lane loads row l16, columns t*32 + g4*8 .. +8 of each slice (A operand layout);
  // with FAL_DEC_KLINE a pair of k-steps (t, t+1) is loaded as whole lines instead
  // (kline_unswap restores the layout)
  const int kvo = (int)(l16 * p.k_ss + g4 * 8) * 2;
  const int kvl = (int)((l16 & 7) * p.k_ss + (g4 + 4 * (l16 >> 3)) * 8) * 2;
  const int kvl8 = kvl + (int)(8 * p.k_ss) * 2;
  // V: load instruction I of a slice fills chunks [I*64, I*64+64)
  int vvo[VI];
#pragma unroll
  for (int I = 0; I < VI; ++I) {
    const int pch = I * 64 + lane;
    const int r = pch / CPR;
    const int cch = (pch % CPR) ^ vswz<D>(r);
    vvo[I] = (int)(r * p.v_ss + cch * 8) * 2;
  }
  T* vring = &vsm[ws][0];

  // one 32-row step = two 16-row slices
  V8 kreg[2][2][KS];
  auto issue = [&](int step, int buf) {
    const int r0 = k_begin + step * 32;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      const int rs = r0 + sl * 16;
      const int64_t left = (int64_t)max(k_end - rs, 0);
      const __amdgpu_buffer_rsrc_t krs =
          make_rsrc(kbase + (int64_t)rs * p.k_ss, (uint32_t)min(left * p.k_ss * 2, (int64_t)0x7fffffff));
      const __amdgpu_buffer_rsrc_t vrs =
          make_rsrc(vbase + (int64_t)rs * p.v_ss, (uint32_t)min(left * p.v_ss * 2, (int64_t)0x7fffffff));
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        if (FAL_DEC_KLINE && (t & 1) == 0 && t + 1 < KS)
          kreg[buf][sl][t] = __builtin_bit_cast(
              V8, __builtin_amdgcn_raw_buffer_load_b128(krs, kvl + t * 64, 0, FAL_DEC_KAUX));
        else if (FAL_DEC_KLINE && (t & 1) == 1)
          kreg[buf][sl][t] = __builtin_bit_cast(
              V8, __builtin_amdgcn_raw_buffer_load_b128(krs, kvl8 + (t - 1) * 64, 0, FAL_DEC_KAUX));
        else
          kreg[buf][sl][t] = __builtin_bit_cast(V8, __builtin_amdgcn_raw_buffer_load_b128(krs, kvo + t * 64, 0, 0));
      }
#pragma unroll
      for (int I = 0; I < VI; ++I)
        buffer_to_lds16<FAL_DEC_VAUX>(vrs, vvo[I], vring + (buf * 2 + sl) * SLICE + I * 64 * 8);
    }
  };
  // this wave's steps: ws, ws + NW, ...
  int j = ws;
  if (j < nsteps) issue(j, 0);
  if (j + NW < nsteps) issue(j + NW, 1);

  // queries of the head tile as the B operand (n = head, k = head dim)
  V8 qreg[KS];
  const T* qrow = (const T*)p.q + (int64_t)b * p.q_sb + (int64_t)(hbase + l16) * p.q_sh;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    qreg[t] = l16 < nh ? ld8(qrow + t * 32 + g4 * 8) : zero8<T>();
    if (p.negate_q) qreg[t] = -qreg[t];
  }
  const float c = p.scale_log2;
  const float* bias = p.bias ? p.bias + (int64_t)b * p.bias_sb : nullptr;

  // transposed V reads: lane i of 16-lane group g4 reads row 4*g4 + i/4, columns
  // db*16 + 4*(i%4) .. +4 of a slice
  const int vr = 4 * g4 + (l16 >> 2);
  const int vrbase = vr * CPR * 8 + 4 * (l16 & 1);
  const int vrc0 = ((l16 >> 1) & 1) ^ vswz<D>(vr);   // chunk of block 0; block db is vrc0 ^ 2*db
#define VRD(db) (vrbase + ((vrc0 ^ (2 * (db))) << 3))

  f32x4 oacc[DBN];
#pragma unroll
  for (int i = 0; i < DBN; ++i) oacc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;

  auto step = [&](auto bufc) {
    constexpr int buf = decltype(bufc)::value;
    if (j + NW < nsteps) wait_vmcnt<LPS>();
    else wait_vmcnt<0>();
    // S^T for the two slices (element i: row 16*sl + 4*g4 + i, head l16)
    f32x4 s[2];
#pragma unroll
    for (int sl = 0; sl < 2; ++sl) {
      if (FAL_DEC_KLINE) {
#pragma unroll
        for (int t = 0; t + 1 < KS; t += 2) kline_unswap(kreg[buf][sl][t], kreg[buf][sl][t + 1]);
      }
      s[sl] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < KS; ++t) s[sl] = mfma16(kreg[buf][sl][t], qreg[t], s[sl]);
    }
    const int r0 = k_begin + j * 32;
    float mx = -INFINITY;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = r0 + sl * 16 + 4 * g4 + i;
        float x = s[sl][i] * c;
        if (bias && r < k_end) x = fmaf(bias[r], kLog2e, x);
        if (r >= k_end) x = -INFINITY;
        s[sl][i] = x;
        mx = fmaxf(mx, x);
      }
    mx = rows4_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    V8 pb;
#pragma unroll
    for (int sl = 0; sl < 2; ++sl)
#pragma unroll
      for (int i = 0; i < 4; ++i) pb[sl * 4 + i] = (T)fast_exp2(s[sl][i] - m_use);
    l_run = sum8(pb, l_run * alpha);
#pragma unroll
    for (int db = 0; db < DBN; ++db) oacc[db] *= alpha;
    // O^T += V^T P^T over the 32 rows
    const T* v0 = vring + (buf * 2) * SLICE;
#pragma unroll
    for (int db = 0; db < DBN; ++db) {
      oacc[db] = mfma16(join8(lds_tr(v0 + VRD(db)), lds_tr(v0 + SLICE + VRD(db))), pb, oacc[db]);
    }
    // LDS reads of this buffer must finish before the next loads overwrite it
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (j + 2 * NW < nsteps) issue(j + 2 * NW, buf);
    j += NW;
  };
  // two steps per trip so the register ring index is a compile-time constant
  while (j < nsteps) {
    step(std::integral_constant<int, 0>{});
    if (j >= nsteps) break;
    step(std::integral_constant<int, 1>{});
  }

  // ---- merge: heads are lanes l16; rows split over the four 16-lane groups ----
  const float l_tot = rows4_sum(l_run);
  if (lane < 16) {
    m_s[w][l16] = m_run;
    l_s[w][l16] = l_tot;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < NW; ++i) M = fmaxf(M, m_s[i][l16]);
  const float M_use = (M == -INFINITY) ? 0.f : M;
  const float wscale = fast_exp2(m_run - M_use);
  // Each wave's rescaled O goes to its own (now idle) V ring slab; the slabs are summed
  // in wave order below, so the result does not depend on timing.
  float* part = reinterpret_cast<float*>(&vsm[ws][0]);
  static_assert(sizeof(vsm[0]) >= 16 * D * sizeof(float), "a wave's slab holds its partial O");
  if (l16 < nh) {
#pragma unroll
    for (int db = 0; db < DBN; ++db)
#pragma unroll
      for (int i = 0; i < 4; ++i) part[l16 * D + db * 16 + 4 * g4 + i] = oacc[db][i] * wscale;
  }
  const int64_t pbase = ((int64_t)b * p.Hq + hbase) * p.max_splits + split;
  if (w == 0 && lane < nh) {
    float Lsum = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) Lsum += l_s[i][l16] * fast_exp2(m_s[i][l16] - M_use);
    inv_s[l16] = Lsum > 0.f ? 1.f / Lsum : 0.f;
    p.part_m[pbase + (int64_t)l16 * p.max_splits] = (Lsum > 0.f) ? M_use + fast_log2(Lsum) : -INFINITY;
  }
  __syncthreads();
  for (int i = tid; i < nh * D; i += NW * 64) {
    const int h = i / D, d = i % D;
    float o = 0.f;
#pragma unroll
    for (int ww = 0; ww < NW; ++ww) o += reinterpret_cast<const float*>(&vsm[ww][0])[h * D + d];
    p.part_o[(pbase + (int64_t)h * p.max_splits) * D + d] = o * inv_s[h];
  }
}

// One wave per (sequence, query head): merge the splits' partial outputs, sixteen splits
// per round trip.
template <class T, int D>
__global__ void __launch_bounds__(64)
decode_combine_kernel(DecodeParams p) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int L = min(max(p.seqlens[b], 0), p.max_seqlen);
  const int ns = cdiv(max(L, 0), p.chunk);
  const int64_t base = ((int64_t)b * p.Hq + hq) * p.max_splits;
  constexpr int DJ = (D + 63) / 64;
  constexpr int CH = 16;   // splits whose loads are all in flight together
  float acc[DJ];
#pragma unroll
  for (int j = 0; j < DJ; ++j) acc[j] = 0.f;
  float M = -INFINITY, wsum = 0.f;
  // chunks of CH splits, merged with an online max: every load of a chunk is issued
  // before any of them is used
  for (int s0 = 0; s0 < ns; s0 += CH) {
    float pm[CH], x[CH][DJ];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const bool ok = s0 + u < ns;
      pm[u] = ok ? p.part_m[base + s0 + u] : -INFINITY;
      const float* po = p.part_o + (base + s0 + u) * D;
#pragma unroll
      for (int j = 0; j < DJ; ++j) x[u][j] = (ok && lane + 64 * j < D) ? po[lane + 64 * j] : 0.f;
    }
    float cm = -INFINITY;
#pragma unroll
    for (int u = 0; u < CH; ++u) cm = fmaxf(cm, pm[u]);
    const float Mn = fmaxf(M, cm);
    if (Mn == -INFINITY) continue;
    const float r = fast_exp2(M - Mn);   // 0 on the first chunk with a finite max
    wsum *= r;
#pragma unroll
    for (int j = 0; j < DJ; ++j) acc[j] *= r;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const float wgt = fast_exp2(pm[u] - Mn);
      wsum += wgt;
#pragma unroll
      for (int j = 0; j < DJ; ++j) acc[j] = fmaf(wgt, x[u][j], acc[j]);
    }
    M = Mn;
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  T* orow = (T*)p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh;
#pragma unroll
  for (int j = 0; j < DJ; ++j) {
    const int d = lane + 64 * j;
    if (d < D) orow[d] = (T)(acc[j] * inv);
  }
  if (p.lse && lane == 0)
    p.lse[(int64_t)b * p.Hq + hq] = (wsum > 0.f && M != -INFINITY) ? (M + fast_log2(wsum)) * kLn2 : -INFINITY;
}

#ifndef FAL_DEC_CHUNK
#define FAL_DEC_CHUNK 2048
#endif

// Cache rows per split: start from FAL_DEC_CHUNK and halve (down to one tile) until
// the grid has at least ~4 workgroups per CU for the longest sequence.
// Work list of (sequence, split) items, longest first: every full chunk, then the
// partial last chunks by descending length (64 length buckets).  Heavy workgroups
// start first, so the kernel does not end on a tail of long splits.  Built on the
// device from cache_seqlens; unused trailing slots get (-1, -1).
__global__ void __launch_bounds__(1024)
decode_schedule_kernel(const int* __restrict__ seqlens, int B, int max_seqlen, int chunk, int2* __restrict__ work,
                       int capacity) {
  __shared__ int hist[64], cur[64], full_total, full_cur;
  for (int i = threadIdx.x; i < 64; i += blockDim.x) hist[i] = 0;
  if (threadIdx.x == 0) full_total = 0;
  __syncthreads();
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    const int L = min(max(seqlens[b], 0), max_seqlen);
    if (L / chunk) atomicAdd(&full_total, L / chunk);
    if (L % chunk) atomicAdd(&hist[(L % chunk) * 64 / chunk], 1);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int acc = full_total;
    for (int k = 63; k >= 0; --k) {
      cur[k] = acc;
      acc += hist[k];
    }
    full_cur = 0;
    hist[0] = acc;   // total items
  }
  __syncthreads();
  const int total = hist[0];
  for (int b = threadIdx.x; b < B; b += blockDim.x) {
    const int L = min(max(seqlens[b], 0), max_seqlen);
    const int nf = L / chunk;
    if (nf) {
      const int pos = atomicAdd(&full_cur, nf);
      for (int s = 0; s < nf; ++s)
        if (pos + s < capacity) work[pos + s] = make_int2(b, s);
    }
    if (L % chunk) {
      const int pos = atomicAdd(&cur[(L % chunk) * 64 / chunk], 1);
      if (pos < capacity) work[pos] = make_int2(b, nf);
    }
  }
  for (int i = total + threadIdx.x; i < capacity; i += blockDim.x) work[i] = make_int2(-1, -1);
}

int decode_chunk(int d, int B, int Hkv, int max_seqlen) {
  (void)d;
  const int tile = FAL_DEC_NW * 32;
  int chunk = FAL_DEC_CHUNK;
  while (chunk > tile && (long)B * Hkv * cdiv(max_seqlen, chunk) < 1024) chunk >>= 1;
  return chunk < tile ? tile : chunk;
}

#ifndef FAL_DEC_INLINE_ITEMS
#define FAL_DEC_INLINE_ITEMS 1   // batches of <= 64 sequences: work items computed in the split kernel
#endif


template <class T, int D>
static hipError_t launch_decode_t(const DecodeParams& pin, hipStream_t st) {
  DecodeParams p = pin;
  const int nhg = cdiv(p.Hq / p.Hkv, 16);
  const int capacity = p.B * p.max_splits;
  if (FAL_DEC_INLINE_ITEMS && p.B <= 64) {
    p.work = nullptr;
  } else {
    hipLaunchKernelGGL(decode_schedule_kernel, dim3(1), dim3(1024), 0, st, p.seqlens, p.B, p.max_seqlen, p.chunk,
                       const_cast<int2*>(p.work), capacity);
    hipError_t e0 = hipGetLastError();
    if (e0 != hipSuccess) return e0;
  }
  hipLaunchKernelGGL((decode_split_kernel<T, D, FAL_DEC_NW>), dim3((unsigned)capacity * p.Hkv * nhg),
                     dim3(FAL_DEC_NW * 64), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_combine_kernel<T, D>), dim3(p.Hq, p.B), dim3(64), 0, st, p);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_decode_d(const DecodeParams& p, hipStream_t st) {
  return p.bf16 ? launch_decode_t<bf16_t, D>(p, st) : launch_decode_t<half_t, D>(p, st);
}

hipError_t launch_decode(const DecodeParams& p, int d, hipStream_t st) {
  switch (d) {
    case 32: return launch_decode_d<32>(p, st);
    case 64: return launch_decode_d<64>(p, st);
    case 96: return launch_decode_d<96>(p, st);
    case 128: return launch_decode_d<128>(p, st);
    case 256: return launch_decode_d<256>(p, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fal

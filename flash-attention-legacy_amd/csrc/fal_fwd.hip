// Attention forward for gfx950: online softmax with QK^T and PV on MFMA.
//
// Semantics follow the reference forward (csrc/kernels/flash_attn_fwd_volta.cu:170-345
// batched, :350-523 varlen): s = (q . k) * scale; keys with index >= seqlen_k or, when
// causal, key > query (top-left aligned, local indices for varlen) are excluded;
// O = sum(p v) / sum(p); L = max + ln(max(sum, 1e-20)) in natural log; a row with no
// valid key gives O = 0 and L = -inf.
//
// Work decomposition (one workgroup = NW waves = 32*NW query rows of one head):
// * each wave owns 32 query rows; its Q slice stays in VGPRs for the whole kernel as
//   the B operand of S^T = K Q^T, so the accumulator puts one query row per lane
//   (two lanes per row, one per wave half) and row max / row sum are in-lane plus
//   one permlane32 swap;
// * K/V tiles of BN keys are staged row-major in LDS, double-buffered, and fetched
//   one tile ahead into registers with 16-byte global loads;
// * P^T goes straight from the S^T accumulator into the B operand of O^T = V^T P^T;
//   V^T comes from the row-major V tile through ds_read_b64_tr_b16;
// * causal tiles above the diagonal are never visited; fully-masked waves inside a
//   diagonal tile skip their MFMAs.
#include "fal_kernels.h"

namespace fal {

template <int D, int NW, int BN, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64)
fwd_kernel(FwdParams p) {
  constexpr int BM = NW * 32;
  constexpr int KS = D / 16;        // MFMA k-steps over the head dim
  constexpr int NKB = BN / 32;      // 32-key blocks per tile
  constexpr int DB = D / 32;        // 32-wide blocks of the output head dim
  constexpr int LDK = D + 8;        // padded LDS row (elements)
  constexpr int CHUNKS = BN * D / 8;                 // 16-byte chunks per K (or V) tile
  constexpr int CPT = (CHUNKS + NW * 64 - 1) / (NW * 64);
  constexpr int CPR = D / 8;                         // chunks per row

  __shared__ __attribute__((aligned(16))) half_t smem[2 * 2 * BN * LDK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  // ---- resolve this workgroup's (batch/sequence, head, query tile) ----
  int b, hq, qt, q_off, k_off, nq, nk;
  if (p.cu_q) {
    const int2 wk = p.work[blockIdx.x];
    if (wk.x < 0) return;
    hq = blockIdx.y;
    b = 0;
    qt = wk.y;
    q_off = p.cu_q[wk.x];
    nq = p.cu_q[wk.x + 1] - q_off;
    k_off = p.cu_k[wk.x];
    nk = p.cu_k[wk.x + 1] - k_off;
  } else {
    // 1-D grid; group heads of one KV head and the query tiles of a head together so the
    // workgroups an XCD runs at once share K/V in that XCD's L2 (workgroups are dealt to
    // the 8 XCDs round-robin by linear id).
    const int total = gridDim.x;
    int id = blockIdx.x;
    if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
    const int g = p.Hq / p.Hkv;
    const int hg = id % g;
    int rest = id / g;
    const int t = rest % p.n_qtiles;
    rest /= p.n_qtiles;                       // = b * Hkv + hkv
    qt = CAUSAL ? (p.n_qtiles - 1 - t) : t;   // heaviest causal tiles first
    b = rest / p.Hkv;
    hq = (rest % p.Hkv) * g + hg;
    q_off = 0;
    k_off = 0;
    nq = p.Nq;
    nk = p.Nk;
  }
  const int hkv = hq / (p.Hq / p.Hkv);
  const int m0 = qt * BM;
  if (m0 >= nq) return;

  const half_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)q_off * p.q_ss;
  const half_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh + (int64_t)k_off * p.k_ss;
  const half_t* vbase = p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh + (int64_t)k_off * p.v_ss;
  half_t* obase = p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + (int64_t)q_off * p.o_ss;
  float* lbase = p.lse + (int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)q_off * p.l_ss;

  // ---- Q slice of this wave into registers (B operand: n = query row, k = head dim) ----
  const int row = m0 + w * 32 + l32;
  half8 qreg[KS];
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    qreg[t] = row < nq ? load_h8(qbase + (int64_t)row * p.q_ss + t * 16 + hh * 8) : zero_h8();
    if (p.negate_q) qreg[t] = -qreg[t];
  }
  const float c = p.scale_log2;   // |scale| * log2(e); the sign was folded into Q

  // ---- key range ----
  const int kend = CAUSAL ? min(nk, m0 + BM) : nk;
  const int ntiles = cdiv(kend, BN);

  f32x16 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) oacc[i] = zero_f16();
  float m_run = -INFINITY;   // running max, log2 domain
  float l_run = 0.f;         // running sum (this lane's keys only)

  u32x4 kpre[CPT], vpre[CPT];
  auto fetch = [&](int tile) {
    const int n0 = tile * BN;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int ch = tid + i * NW * 64;
      const int r = ch / CPR;
      const int cc = (ch % CPR) * 8;
      const bool ok = (CHUNKS % (NW * 64) == 0 || ch < CHUNKS) && (n0 + r < nk);
      kpre[i] = ok ? load_u4(kbase + (int64_t)(n0 + r) * p.k_ss + cc) : u32x4{0, 0, 0, 0};
      vpre[i] = ok ? load_u4(vbase + (int64_t)(n0 + r) * p.v_ss + cc) : u32x4{0, 0, 0, 0};
    }
  };
  auto stash = [&](int buf) {
    half_t* ks = smem + buf * 2 * BN * LDK;
    half_t* vs = ks + BN * LDK;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int ch = tid + i * NW * 64;
      if (CHUNKS % (NW * 64) == 0 || ch < CHUNKS) {
        const int r = ch / CPR;
        const int cc = (ch % CPR) * 8;
        store_u4(ks + r * LDK + cc, kpre[i]);
        store_u4(vs + r * LDK + cc, vpre[i]);
      }
    }
  };

  if (ntiles > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();

  const int wrow_lo = m0 + w * 32;        // first query row of this wave
  const int vofs = tr_offset(lane, LDK);

  for (int j = 0; j < ntiles; ++j) {
    if (j + 1 < ntiles) fetch(j + 1);
    const int n0 = j * BN;
    const half_t* ks = smem + (j & 1) * 2 * BN * LDK;
    const half_t* vs = ks + BN * LDK;

    if (!CAUSAL || n0 <= wrow_lo + 31) {
      // S^T = K Q^T : one 32x32 block per 32 keys
      f32x16 sacc[NKB];
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        sacc[kb] = zero_f16();
#pragma unroll
        for (int t = 0; t < KS; ++t) {
          const half8 a = load_h8(ks + (kb * 32 + l32) * LDK + t * 16 + hh * 8);
          sacc[kb] = mfma32(a, qreg[t], sacc[kb]);
        }
      }
      // masking (only on tiles that touch the sequence end or the diagonal)
      const bool need_mask = (n0 + BN > nk) || (CAUSAL && n0 + BN - 1 > wrow_lo);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = n0 + kb * 32 + (i >> 2) * 8 + hh * 4 + (i & 3);
            if (key >= nk || (CAUSAL && key > row)) sacc[kb][i] = -INFINITY;
          }
      }
      // online softmax for this lane's query row
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, sacc[kb][i]);
      mx = pair_max(mx);
      const float m_new = fmaxf(m_run, mx * c);
      const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
      const float alpha = fast_exp2(m_run - m_use);
      m_run = m_new;
      float rs = 0.f;
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float e = fast_exp2(fmaf(sacc[kb][i], c, -m_use));
          sacc[kb][i] = e;
          rs += e;
        }
      l_run = fmaf(l_run, alpha, rs);
#pragma unroll
      for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
      // O^T += V^T P^T
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int t2 = 0; t2 < 2; ++t2) {
          const half8 pb = cvt8(sacc[kb], t2);
          const int krow = kb * 32 + t2 * 16;
#pragma unroll
          for (int db = 0; db < DB; ++db) {
            const half8 va = lds_kslab_tr(vs + vofs + db * 32, krow, hh, LDK);
            oacc[db] = mfma32(va, pb, oacc[db]);
          }
        }
    }

    if (j + 1 < ntiles) stash((j + 1) & 1);
    __syncthreads();
  }

  // ---- epilogue: normalise, write O and L ----
  const float l_tot = pair_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (row < nq) {
    half_t* orow = obase + (int64_t)row * p.o_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        half4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (half_t)(oacc[db][g4 * 4 + e] * inv);
        *reinterpret_cast<half4*>(orow + db * 32 + g4 * 8 + hh * 4) = h;
      }
    if (hh == 0) {
      float L = -INFINITY;
      if (m_run != -INFINITY) L = (m_run + fast_log2(fmaxf(l_tot, 1e-20f))) * kLn2;
      lbase[(int64_t)row * p.l_ss] = L;
    }
  }
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
varlen_schedule_kernel(const int* __restrict__ cu, int num_seqs, int tile, int nbuckets,
                       int descending, int2* __restrict__ work, int capacity) {
  extern __shared__ int sh[];            // [nbuckets] counts, then [nbuckets] cursors
  int* cnt = sh;
  int* cur = sh + nbuckets;
  for (int i = threadIdx.x; i < nbuckets; i += blockDim.x) cnt[i] = 0;
  __syncthreads();
  for (int s = threadIdx.x; s < num_seqs; s += blockDim.x) {
    const int nt = cdiv(max(cu[s + 1] - cu[s], 0), tile);
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
    const int nt = cdiv(max(cu[s + 1] - cu[s], 0), tile);
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
template <int D>
struct FwdCfg {
  static constexpr int NW = 4;
  static constexpr int BN = (D >= 256) ? 32 : 64;
};

template <int D>
static hipError_t launch_fwd_d(const FwdParams& p, int causal, dim3 grid, hipStream_t st) {
  constexpr int NW = FwdCfg<D>::NW, BN = FwdCfg<D>::BN;
  if (causal)
    hipLaunchKernelGGL((fwd_kernel<D, NW, BN, true>), grid, dim3(NW * 64), 0, st, p);
  else
    hipLaunchKernelGGL((fwd_kernel<D, NW, BN, false>), grid, dim3(NW * 64), 0, st, p);
  return hipGetLastError();
}

int fwd_block_m(int d) {
  (void)d;
  return 4 * 32;
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

hipError_t launch_varlen_schedule(const int* cu, int num_seqs, int tile, int nbuckets, int descending,
                                  int2* work, int capacity, hipStream_t st) {
  const size_t shmem = 2 * sizeof(int) * (size_t)nbuckets;
  hipLaunchKernelGGL(varlen_schedule_kernel, dim3(1), dim3(1024), shmem, st, cu, num_seqs, tile,
                     nbuckets, descending, work, capacity);
  return hipGetLastError();
}

}  // namespace fal

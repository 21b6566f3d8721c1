// KV-cache decode for gfx950: split-K over the cache plus a log-sum-exp combine.
//
// The reference has no decode kernel: for q_len != kv_len it runs eager PyTorch
// (flash_attn_legacy/integrations.py:77-98): repeat K/V over the GQA group,
// s = q k^T * scale (+ additive mask), softmax over the keys, @ v.  This file computes
// the same result without materialising the repeated K/V or the score row.
//
// Split kernel: one workgroup per (split, kv head, sequence) covers `chunk` cache rows.
// * All G = Hq/Hkv query heads of the KV head ride in one MFMA tile: S^T = K Q^T with
//   M = 32 cache rows and N = the G heads (padded to 32 lanes), so every K/V byte is
//   read once from HBM for the whole group.
// * Each wave streams its own 32-row slices: K rows are loaded straight into the A
//   operand, V rows go through a wave-private LDS slab and come back transposed
//   (ds_read_b64_tr_b16) as the A operand of O^T = V^T P^T.  The next slice's loads
//   are issued before the current slice is consumed.
// * The waves' (max, sum, O) are merged in LDS and the workgroup writes one
//   normalised partial O (fp32) and its log2-domain LSE.
// Combine kernel: one wave per (sequence, query head) merges its splits.
#include "fal_kernels.h"

namespace fal {

constexpr int kDecNW = 4;

template <int D, int NW>
__global__ void __launch_bounds__(NW * 64)
decode_split_kernel(DecodeParams p) {
  constexpr int KS = D / 16;
  constexpr int DB = D / 32;
  constexpr int LDV = D + 8;
  __shared__ __attribute__((aligned(16))) half_t v_s[NW][32 * LDV];
  __shared__ float m_s[NW][32];
  __shared__ float l_s[NW][32];
  __shared__ float o_s[32 * D];

  const int split = blockIdx.x;
  const int hkv = blockIdx.y;
  const int b = blockIdx.z;
  const int L = p.seqlens[b];
  const int k_begin = split * p.chunk;
  if (k_begin >= L) return;
  const int k_end = min(L, k_begin + p.chunk);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;
  const int G = p.Hq / p.Hkv;

  for (int i = tid; i < 32 * D; i += NW * 64) o_s[i] = 0.f;

  // queries of the group as the B operand (n = head, k = head dim)
  half8 qreg[KS];
  const half_t* qrow = p.q + (int64_t)b * p.q_sb + (int64_t)(hkv * G + l32) * p.q_sh;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    qreg[t] = l32 < G ? load_h8(qrow + t * 16 + hh * 8) : zero_h8();
    if (p.negate_q) qreg[t] = -qreg[t];
  }
  const float c = p.scale_log2;
  const half_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh;
  const half_t* vbase = p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh;
  const float* bias = p.bias ? p.bias + (int64_t)b * p.bias_sb : nullptr;

  f32x16 oacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) oacc[i] = zero_f16();
  float m_run = -INFINITY, l_run = 0.f;

  half8 kc[KS];
  u32x4 vc[KS];
  auto load_slice = [&](int s0, half8* kk, u32x4* vv) {
    const int r = s0 + l32;
    const bool ok = r < k_end;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      kk[t] = ok ? load_h8(kbase + (int64_t)r * p.k_ss + t * 16 + hh * 8) : zero_h8();
      vv[t] = ok ? load_u4(vbase + (int64_t)r * p.v_ss + t * 16 + hh * 8) : u32x4{0, 0, 0, 0};
    }
  };

  half_t* vs = v_s[w];
  const int vofs = tr_offset(lane, LDV);
  int s0 = k_begin + w * 32;
  if (s0 < k_end) load_slice(s0, kc, vc);
  for (; s0 < k_end; s0 += NW * 32) {
    half8 kn[KS];
    u32x4 vn[KS];
    const int s1 = s0 + NW * 32;
    if (s1 < k_end) load_slice(s1, kn, vn);

#pragma unroll
    for (int t = 0; t < KS; ++t) store_u4(vs + l32 * LDV + t * 16 + hh * 8, vc[t]);

    f32x16 s = zero_f16();
#pragma unroll
    for (int t = 0; t < KS; ++t) s = mfma32(kc[t], qreg[t], s);
    // element i: cache row s0 + (i/4)*8 + hh*4 + i%4, head l32
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int r = s0 + (i >> 2) * 8 + hh * 4 + (i & 3);
      float t = s[i] * c;
      if (bias && r < k_end) t = fmaf(bias[r], kLog2e, t);
      if (r >= k_end) t = -INFINITY;
      s[i] = t;
      mx = fmaxf(mx, t);
    }
    mx = pair_max(mx);
    const float m_new = fmaxf(m_run, mx);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    m_run = m_new;
    float rs = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float e = fast_exp2(s[i] - m_use);
      s[i] = e;
      rs += e;
    }
    l_run = fmaf(l_run, alpha, rs);
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) oacc[db][i] *= alpha;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
#pragma unroll
    for (int t2 = 0; t2 < 2; ++t2) {
      const half8 pb = cvt8(s, t2);
#pragma unroll
      for (int db = 0; db < DB; ++db)
        oacc[db] = mfma32(lds_kslab_tr(vs + vofs + db * 32, t2 * 16, hh, LDV), pb, oacc[db]);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      kc[t] = kn[t];
      vc[t] = vn[t];
    }
  }

  // ---- merge the waves ----
  __shared__ float inv_s[32];
  const float l_tot = pair_sum(l_run);
  if (hh == 0) {
    m_s[w][l32] = m_run;
    l_s[w][l32] = l_tot;
  }
  __syncthreads();
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < NW; ++i) M = fmaxf(M, m_s[i][l32]);
  const float M_use = (M == -INFINITY) ? 0.f : M;
  const float wscale = fast_exp2(m_run - M_use);   // this wave's weight for head l32
  if (l32 < G) {
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int d = db * 32 + (i >> 2) * 8 + hh * 4 + (i & 3);
        atomicAdd(&o_s[l32 * D + d], oacc[db][i] * wscale);
      }
  }
  const int64_t pbase = ((int64_t)b * p.Hq + hkv * G) * p.max_splits + split;
  if (w == 0 && hh == 0 && l32 < G) {
    float Lsum = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) Lsum += l_s[i][l32] * fast_exp2(m_s[i][l32] - M_use);
    inv_s[l32] = Lsum > 0.f ? 1.f / Lsum : 0.f;
    p.part_m[pbase + (int64_t)l32 * p.max_splits] = (Lsum > 0.f) ? M_use + fast_log2(Lsum) : -INFINITY;
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += NW * 64) {
    const int h = i / D, d = i % D;
    p.part_o[(pbase + (int64_t)h * p.max_splits) * D + d] = o_s[h * D + d] * inv_s[h];
  }
}

// One wave per (sequence, query head): merge the splits' partial outputs.
template <int D>
__global__ void __launch_bounds__(64)
decode_combine_kernel(DecodeParams p) {
  const int hq = blockIdx.x;
  const int b = blockIdx.y;
  const int lane = threadIdx.x;
  const int L = p.seqlens[b];
  const int ns = cdiv(L, p.chunk);
  const int64_t base = ((int64_t)b * p.Hq + hq) * p.max_splits;
  float M = -INFINITY;
  for (int s = lane; s < ns; s += 64) M = fmaxf(M, p.part_m[base + s]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
  const float M_use = (M == -INFINITY) ? 0.f : M;
  float acc[(D + 63) / 64];
#pragma unroll
  for (int j = 0; j < (D + 63) / 64; ++j) acc[j] = 0.f;
  float wsum = 0.f;
  for (int s = 0; s < ns; ++s) {
    const float wgt = fast_exp2(p.part_m[base + s] - M_use);
    wsum += wgt;
    const float* po = p.part_o + (base + s) * D;
#pragma unroll
    for (int j = 0; j < (D + 63) / 64; ++j) {
      const int d = lane + 64 * j;
      if (d < D) acc[j] = fmaf(wgt, po[d], acc[j]);
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  half_t* orow = p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh;
#pragma unroll
  for (int j = 0; j < (D + 63) / 64; ++j) {
    const int d = lane + 64 * j;
    if (d < D) orow[d] = (half_t)(acc[j] * inv);
  }
  if (p.lse && lane == 0)
    p.lse[(int64_t)b * p.Hq + hq] = (wsum > 0.f && M != -INFINITY) ? (M + fast_log2(wsum)) * kLn2 : -INFINITY;
}

int decode_chunk(int d, int B, int Hkv, int max_seqlen) {
  (void)d;
  int spw = 4;
  while (spw > 1 && (long)B * Hkv * cdiv(max_seqlen, kDecNW * 32 * spw) < 2048) spw >>= 1;
  return kDecNW * 32 * spw;
}

template <int D>
static hipError_t launch_decode_d(const DecodeParams& p, hipStream_t st) {
  hipLaunchKernelGGL((decode_split_kernel<D, kDecNW>), dim3(p.max_splits, p.Hkv, p.B), dim3(kDecNW * 64), 0,
                     st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_combine_kernel<D>), dim3(p.Hq, p.B), dim3(64), 0, st, p);
  return hipGetLastError();
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

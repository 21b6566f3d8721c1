// Attention backward for gfx950.
//
// Math follows the reference backward (csrc/kernels/flash_attn_bwd.cu:76-107 for the
// preprocess, :425-647 for the KV-outer kernel): D = rowsum(dO * O);
// P = exp(S*scale - L); dV += P^T dO; dP = dO V^T; dS = P (dP - D) * scale;
// dK += dS^T Q; dQ += dS K accumulated in fp32 and cast at the end; dK/dV of a KV
// head sum over all query heads of its GQA group inside one workgroup.
//
// Work decomposition: one workgroup owns BN = 32*NW keys of one KV head and walks
// every (query head of the group, query tile of BMQ rows) that can see them.
// * Each wave owns 32 keys.  Its K and V rows live in VGPRs as the B operands of
//   S = Q K^T and dP = dO V^T, so those accumulators hold one key per lane.
// * P and dS leave the accumulators straight into the B operands of
//   dV^T += dO^T P and dK^T += Q^T dS; dO^T and Q^T come from the row-major
//   Q/dO tiles in LDS via ds_read_b64_tr_b16.  dK^T / dV^T stay in registers
//   for the whole kernel.
// * dS^T is staged in LDS (fp16) and each wave then computes one 32-column
//   block of dQ = dS K for the tile (K^T from the LDS K tile, again via the
//   transposed read) and adds it to the fp32 dQ accumulator with global atomics.
// * For head_dim 256 the dK/dV accumulators are split into two passes over the
//   query tiles (128 columns each); dQ is produced in the first pass.
#include "fal_kernels.h"

namespace fal {

// --------------------------------------------------------------------------
// Preprocess: delta = rowsum(dO * O) (fp32) and zero the fp32 dQ accumulator.
// One group of D/8 lanes per row (16-byte loads), reduced with xor shuffles.
// --------------------------------------------------------------------------
template <int D>
constexpr int row_group() { return D / 8 <= 4 ? 4 : D / 8 <= 8 ? 8 : D / 8 <= 16 ? 16 : 32; }

template <int D>
__global__ void __launch_bounds__(256)
bwd_pre_kernel(BwdParams p, int rows, int batched) {
  constexpr int G = row_group<D>();   // lanes per row (power of two; lanes past D idle)
  const int r = blockIdx.x * (256 / G) + threadIdx.x / G;
  const int c = (threadIdx.x % G) * 8;
  if (r >= rows) return;   // whole group exits together (G divides 64)
  int64_t o_off, do_off, l_off, qa_off;
  if (batched) {
    const int n = r % p.Nq;
    const int h = (r / p.Nq) % p.Hq;
    const int b = r / (p.Nq * p.Hq);
    o_off = b * p.o_sb + h * p.o_sh + (int64_t)n * p.o_ss;
    do_off = b * p.do_sb + h * p.do_sh + (int64_t)n * p.do_ss;
    l_off = b * p.l_sb + h * p.l_sh + (int64_t)n * p.l_ss;
    qa_off = b * p.dqa_sb + h * p.dqa_sh + (int64_t)n * p.dqa_ss;
  } else {
    const int tok = r / p.Hq;
    const int h = r % p.Hq;
    o_off = (int64_t)tok * p.o_ss + h * p.o_sh;
    do_off = (int64_t)tok * p.do_ss + h * p.do_sh;
    l_off = (int64_t)tok * p.l_ss + h * p.l_sh;
    qa_off = (int64_t)tok * p.dqa_ss + h * p.dqa_sh;
  }
  float s = 0.f;
  if (c < D) {
    const half8 a = load_h8(p.o + o_off + c);
    const half8 g = load_h8(p.dout + do_off + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) s = fmaf((float)a[j], (float)g[j], s);
  }
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (threadIdx.x % G == 0) p.delta[l_off] = s;
  if (c >= D) return;
  float* qa = p.dq_acc + qa_off + c;
  *reinterpret_cast<f32x4*>(qa) = f32x4{0.f, 0.f, 0.f, 0.f};
  *reinterpret_cast<f32x4*>(qa + 4) = f32x4{0.f, 0.f, 0.f, 0.f};
}

// dQ = fp16(dq_acc * scale)
template <int D>
__global__ void __launch_bounds__(256)
bwd_post_kernel(BwdParams p, int rows, int batched) {
  constexpr int G = row_group<D>();
  const int r = blockIdx.x * (256 / G) + threadIdx.x / G;
  const int c = (threadIdx.x % G) * 8;
  if (r >= rows || c >= D) return;
  int64_t qa_off, dq_off;
  if (batched) {
    const int n = r % p.Nq;
    const int h = (r / p.Nq) % p.Hq;
    const int b = r / (p.Nq * p.Hq);
    qa_off = b * p.dqa_sb + h * p.dqa_sh + (int64_t)n * p.dqa_ss;
    dq_off = b * p.dq_sb + h * p.dq_sh + (int64_t)n * p.dq_ss;
  } else {
    const int tok = r / p.Hq;
    const int h = r % p.Hq;
    qa_off = (int64_t)tok * p.dqa_ss + h * p.dqa_sh;
    dq_off = (int64_t)tok * p.dq_ss + h * p.dq_sh;
  }
  const f32x4 x0 = *reinterpret_cast<const f32x4*>(p.dq_acc + qa_off + c);
  const f32x4 x1 = *reinterpret_cast<const f32x4*>(p.dq_acc + qa_off + c + 4);
  half8 h;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = (half_t)(x0[j] * p.scale);
    h[j + 4] = (half_t)(x1[j] * p.scale);
  }
  store_u4(p.dq + dq_off + c, __builtin_bit_cast(u32x4, h));
}

// --------------------------------------------------------------------------
// Main KV-outer kernel
// --------------------------------------------------------------------------
template <int D, int NW, int BMQ, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64)
bwd_kernel(BwdParams p) {
  static_assert(BMQ == 32, "query tile is one 32-row MFMA block");
  constexpr int BN = NW * 32;
  constexpr int KS = D / 16;
  constexpr int DW = D > 128 ? 128 : D;   // dK/dV columns accumulated per pass
  constexpr int NPASS = D / DW;
  constexpr int DWB = DW / 32;
  constexpr int DQB = D / 32;
  constexpr int LDK = D + 8;
  constexpr int LDQ = BMQ + 8;
  constexpr int QCH = BMQ * D / 8;                   // 16B chunks per Q (or dO) tile
  constexpr int QCPT = (QCH + NW * 64 - 1) / (NW * 64);
  constexpr int CPR = D / 8;

  __shared__ __attribute__((aligned(16))) half_t ks_s[BN * LDK];
  __shared__ __attribute__((aligned(16))) half_t q_s[BMQ * LDK];
  __shared__ __attribute__((aligned(16))) half_t do_s[BMQ * LDK];
  __shared__ __attribute__((aligned(16))) half_t dst_s[BN * LDQ];
  __shared__ __attribute__((aligned(16))) float l_s[BMQ];
  __shared__ __attribute__((aligned(16))) float d_s[BMQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  int b, hkv, kt, q_off, k_off, nq, nk;
  if (p.cu_q) {
    const int2 wk = p.work[blockIdx.x];
    if (wk.x < 0) return;
    hkv = blockIdx.y;
    b = 0;
    kt = wk.y;
    q_off = p.cu_q[wk.x];
    nq = p.cu_q[wk.x + 1] - q_off;
    k_off = p.cu_k[wk.x];
    nk = p.cu_k[wk.x + 1] - k_off;
  } else {
    const int total = gridDim.x;
    int id = blockIdx.x;
    if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
    kt = id % p.n_ktiles;      // causal: low key tiles see the most query rows; run first
    const int bh = id / p.n_ktiles;
    b = bh / p.Hkv;
    hkv = bh % p.Hkv;
    q_off = 0;
    k_off = 0;
    nq = p.Nq;
    nk = p.Nk;
  }
  const int n0 = kt * BN;
  if (n0 >= nk) return;
  const int G = p.Hq / p.Hkv;
  const float c = p.scale_log2;

  const half_t* kbase = p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh + (int64_t)k_off * p.k_ss;
  const half_t* vbase = p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh + (int64_t)k_off * p.v_ss;

  // K/V rows of this wave (B operands: n = key, k = head dim)
  const int kw0 = n0 + w * 32;
  const int key = kw0 + l32;
  half8 kreg[KS], vreg[KS];
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    kreg[t] = key < nk ? load_h8(kbase + (int64_t)key * p.k_ss + t * 16 + hh * 8) : zero_h8();
    vreg[t] = key < nk ? load_h8(vbase + (int64_t)key * p.v_ss + t * 16 + hh * 8) : zero_h8();
  }
  // K tile, row-major, for dQ = dS K
  for (int ch = tid; ch < BN * CPR; ch += NW * 64) {
    const int r = ch / CPR, cc = (ch % CPR) * 8;
    const u32x4 x = (n0 + r < nk) ? load_u4(kbase + (int64_t)(n0 + r) * p.k_ss + cc) : u32x4{0, 0, 0, 0};
    store_u4(ks_s + r * LDK + cc, x);
  }

  const int nqt = cdiv(nq, BMQ);
  const int qt0 = CAUSAL ? (n0 / BMQ) : 0;
  const int tofs_q = tr_offset(lane, LDK);
  const int tofs_s = tr_offset(lane, LDQ);

  for (int pass = 0; pass < NPASS; ++pass) {
    const int dbase = pass * DW;
    f32x16 dk_acc[DWB], dv_acc[DWB];
#pragma unroll
    for (int i = 0; i < DWB; ++i) {
      dk_acc[i] = zero_f16();
      dv_acc[i] = zero_f16();
    }

    for (int g = 0; g < G; ++g) {
      const int hq = hkv * G + g;
      const half_t* qbase = p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)q_off * p.q_ss;
      const half_t* dobase = p.dout + (int64_t)b * p.do_sb + (int64_t)hq * p.do_sh + (int64_t)q_off * p.do_ss;
      const float* lbase = p.lse + (int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)q_off * p.l_ss;
      const float* dbase_p = p.delta + (int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)q_off * p.l_ss;
      float* qabase = p.dq_acc + (int64_t)b * p.dqa_sb + (int64_t)hq * p.dqa_sh + (int64_t)q_off * p.dqa_ss;

      u32x4 qpre[QCPT], dopre[QCPT];
      float lpre = 0.f, dpre = 0.f;
      auto fetch = [&](int qt) {
        const int q0 = qt * BMQ;
#pragma unroll
        for (int i = 0; i < QCPT; ++i) {
          const int ch = tid + i * NW * 64;
          const int r = ch / CPR, cc = (ch % CPR) * 8;
          const bool ok = (QCH % (NW * 64) == 0 || ch < QCH) && (q0 + r < nq);
          qpre[i] = ok ? load_u4(qbase + (int64_t)(q0 + r) * p.q_ss + cc) : u32x4{0, 0, 0, 0};
          dopre[i] = ok ? load_u4(dobase + (int64_t)(q0 + r) * p.do_ss + cc) : u32x4{0, 0, 0, 0};
        }
        if (tid < BMQ) {
          const int r = q0 + tid;
          float lv = INFINITY, dv = 0.f;
          if (r < nq) {
            const float L = lbase[(int64_t)r * p.l_ss];
            lv = (L == -INFINITY) ? INFINITY : L * kLog2e;
            dv = dbase_p[(int64_t)r * p.l_ss];
          }
          lpre = lv;
          dpre = dv;
        }
      };
      auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < QCPT; ++i) {
          const int ch = tid + i * NW * 64;
          if (QCH % (NW * 64) == 0 || ch < QCH) {
            const int r = ch / CPR, cc = (ch % CPR) * 8;
            store_u4(q_s + r * LDK + cc, qpre[i]);
            store_u4(do_s + r * LDK + cc, dopre[i]);
          }
        }
        if (tid < BMQ) {
          l_s[tid] = lpre;
          d_s[tid] = dpre;
        }
      };

      if (qt0 < nqt) {
        fetch(qt0);
        __syncthreads();   // previous users of q_s/do_s are done
        stash();
      }
      __syncthreads();

      for (int qt = qt0; qt < nqt; ++qt) {
        const int q0 = qt * BMQ;
        if (qt + 1 < nqt) fetch(qt + 1);
        const bool active = !CAUSAL || (q0 + BMQ - 1 >= kw0);
        if (active) {
          f32x16 s = zero_f16(), dp = zero_f16();
#pragma unroll
          for (int t = 0; t < KS; ++t) {
            s = mfma32(load_h8(q_s + l32 * LDK + t * 16 + hh * 8), kreg[t], s);
            dp = mfma32(load_h8(do_s + l32 * LDK + t * 16 + hh * 8), vreg[t], dp);
          }
          // P and dS (element i: query q0 + (i/4)*8 + hh*4 + i%4, key `key`)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const f32x4 lv = *reinterpret_cast<const f32x4*>(l_s + g4 * 8 + hh * 4);
            const f32x4 dv = *reinterpret_cast<const f32x4*>(d_s + g4 * 8 + hh * 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int i = g4 * 4 + e;
              const int qrow = q0 + g4 * 8 + hh * 4 + e;
              float pv = fast_exp2(fmaf(s[i], c, -lv[e]));
              if (key >= nk || (CAUSAL && key > qrow)) pv = 0.f;
              s[i] = pv;
              dp[i] = pv * (dp[i] - dv[e]);
            }
          }
          // dV^T += dO^T P ; dK^T += Q^T dS  (this pass's head-dim columns)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const half8 pb = cvt8(s, ks);
            const half8 sb = cvt8(dp, ks);
#pragma unroll
            for (int db = 0; db < DWB; ++db) {
              const int col = dbase + db * 32;
              dv_acc[db] = mfma32(lds_kslab_tr(do_s + tofs_q + col, ks * 16, hh, LDK), pb, dv_acc[db]);
              dk_acc[db] = mfma32(lds_kslab_tr(q_s + tofs_q + col, ks * 16, hh, LDK), sb, dk_acc[db]);
            }
          }
          if (pass == 0) {
            // dS^T (fp16) into LDS: row = key (local), columns = query rows
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              half4 h;
#pragma unroll
              for (int e = 0; e < 4; ++e) h[e] = (half_t)dp[g4 * 4 + e];
              *reinterpret_cast<half4*>(dst_s + (w * 32 + l32) * LDQ + g4 * 8 + hh * 4) = h;
            }
          }
        }
        __syncthreads();   // dS^T complete; q_s/do_s reads done

        if (pass == 0) {
          // dQ[q0:q0+32, db*32:+32] += dS K over the key blocks that are active
          for (int db = w; db < DQB; db += NW) {
            f32x16 acc = zero_f16();
            for (int ks = 0; ks < BN / 16; ++ks) {
              const int kwave0 = n0 + (ks >> 1) * 32;   // first key of the owning wave
              if (CAUSAL && q0 + BMQ - 1 < kwave0) break;
              acc = mfma32(lds_kslab_tr(dst_s + tofs_s, ks * 16, hh, LDQ),
                           lds_kslab_tr(ks_s + tofs_q + db * 32, ks * 16, hh, LDK), acc);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int qrow = q0 + (i >> 2) * 8 + hh * 4 + (i & 3);
              if (qrow < nq)
                unsafeAtomicAdd(qabase + (int64_t)qrow * p.dqa_ss + db * 32 + l32, acc[i]);
            }
          }
        }
        if (qt + 1 < nqt) stash();
        __syncthreads();
      }
    }

    // write dK (scaled) and dV for this pass's columns
    if (key < nk) {
      half_t* dkrow = p.dk + (int64_t)b * p.dk_sb + (int64_t)hkv * p.dk_sh + (int64_t)(k_off + key) * p.dk_ss;
      half_t* dvrow = p.dv + (int64_t)b * p.dv_sb + (int64_t)hkv * p.dv_sh + (int64_t)(k_off + key) * p.dv_ss;
#pragma unroll
      for (int db = 0; db < DWB; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          half4 hk, hv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            hk[e] = (half_t)(dk_acc[db][g4 * 4 + e] * p.scale);
            hv[e] = (half_t)dv_acc[db][g4 * 4 + e];
          }
          const int col = dbase + db * 32 + g4 * 8 + hh * 4;
          *reinterpret_cast<half4*>(dkrow + col) = hk;
          *reinterpret_cast<half4*>(dvrow + col) = hv;
        }
    }
  }
}

// --------------------------------------------------------------------------
// Launchers
// --------------------------------------------------------------------------
constexpr int kBwdNW = 4;

int bwd_block_n(int d) {
  (void)d;
  return kBwdNW * 32;
}

template <int D>
static hipError_t launch_bwd_d(const BwdParams& p, int causal, dim3 grid, hipStream_t st) {
  if (causal)
    hipLaunchKernelGGL((bwd_kernel<D, kBwdNW, 32, true>), grid, dim3(kBwdNW * 64), 0, st, p);
  else
    hipLaunchKernelGGL((bwd_kernel<D, kBwdNW, 32, false>), grid, dim3(kBwdNW * 64), 0, st, p);
  return hipGetLastError();
}

hipError_t launch_bwd(const BwdParams& p, int d, int causal, dim3 grid, hipStream_t st) {
  switch (d) {
    case 32: return launch_bwd_d<32>(p, causal, grid, st);
    case 64: return launch_bwd_d<64>(p, causal, grid, st);
    case 96: return launch_bwd_d<96>(p, causal, grid, st);
    case 128: return launch_bwd_d<128>(p, causal, grid, st);
    case 256: return launch_bwd_d<256>(p, causal, grid, st);
    default: return hipErrorInvalidValue;
  }
}

template <int D, bool PRE>
static hipError_t launch_rowwise(const BwdParams& p, int batched, hipStream_t st) {
  const int rows = batched ? p.B * p.Hq * p.Nq : p.total_q * p.Hq;
  if (rows == 0) return hipSuccess;
  constexpr int RPB = 256 / row_group<D>();
  dim3 grid(cdiv(rows, RPB));
  if (PRE)
    hipLaunchKernelGGL((bwd_pre_kernel<D>), grid, dim3(256), 0, st, p, rows, batched);
  else
    hipLaunchKernelGGL((bwd_post_kernel<D>), grid, dim3(256), 0, st, p, rows, batched);
  return hipGetLastError();
}

hipError_t launch_bwd_pre(const BwdParams& p, int d, int batched, hipStream_t st) {
  switch (d) {
    case 32: return launch_rowwise<32, true>(p, batched, st);
    case 64: return launch_rowwise<64, true>(p, batched, st);
    case 96: return launch_rowwise<96, true>(p, batched, st);
    case 128: return launch_rowwise<128, true>(p, batched, st);
    case 256: return launch_rowwise<256, true>(p, batched, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_bwd_post(const BwdParams& p, int d, hipStream_t st) {
  const int batched = p.cu_q == nullptr;
  switch (d) {
    case 32: return launch_rowwise<32, false>(p, batched, st);
    case 64: return launch_rowwise<64, false>(p, batched, st);
    case 96: return launch_rowwise<96, false>(p, batched, st);
    case 128: return launch_rowwise<128, false>(p, batched, st);
    case 256: return launch_rowwise<256, false>(p, batched, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace fal

// Attention backward for gfx950.
//
// Math follows the reference backward (csrc/kernels/flash_attn_bwd.cu:76-107 for the
// preprocess, :425-647 for the KV-outer kernel): D = rowsum(dO * O);
// P = exp(S*scale - L); dV += P^T dO; dP = dO V^T; dS = P (dP - D) * scale;
// dK += dS^T Q; dQ += dS K accumulated in fp32 and cast at the end; dK/dV of a KV
// head sum over all query heads of its GQA group inside one workgroup.
//
// Kernels:
// * head_dim 32/64/96/128 (FA2's split form, no atomics, deterministic):
//   - bwd_dq_kernel (query-outer, runs first): a workgroup owns 128 query rows;
//     Q and dO stay in VGPRs, K/V tiles stream through LDS; it computes D for its
//     rows, P, dS and dQ = dS K, written once in fp16;
//   - bwd2_kernel (KV-outer): a workgroup owns 64 keys of one KV head and walks every
//     (query head of the group, query tile) that can see them; P and dS leave the
//     accumulators straight into the B operands of dV^T += dO^T P and
//     dK^T += Q^T dS (dO^T and Q^T from the Q/dO tiles via ds_read_b64_tr_b16);
//     dK/dV stay in registers until the end.
// * head_dim 256: bwd_pre_kernel (D, zeroed fp32 dQ accumulator), bwd_kernel
//   (KV-outer, dS^T staged in LDS, dQ = dS K added with fp32 atomics; all 256 dK/dV
//   columns accumulate in one pass, with K read from its LDS tile) and bwd_post_kernel
//   (dQ cast to fp16).
#include <type_traits>

#include "fal_kernels.h"
#include "fal_bwd_pipe.inc"
#include "fal_dq_pipe.inc"

namespace fal {

// --------------------------------------------------------------------------
// Preprocess: delta = rowsum(dO * O) (fp32) and zero the fp32 dQ accumulator when
// the atomic dQ path is used.
// One group of D/8 lanes per row (16-byte loads), reduced with xor shuffles.
// --------------------------------------------------------------------------
template <int D>
constexpr int row_group() { return D / 8 <= 4 ? 4 : D / 8 <= 8 ? 8 : D / 8 <= 16 ? 16 : 32; }

template <class T, int D>
__global__ void __launch_bounds__(256)
bwd_pre_kernel(BwdParams p, int rows, int batched) {
  using V8 = vec8<T>;
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
    const V8 a = ld8((const T*)p.o + o_off + c);
    const V8 g = ld8((const T*)p.dout + do_off + c);
#pragma unroll
    for (int j = 0; j < 8; ++j) s = fmaf((float)a[j], (float)g[j], s);
  }
#pragma unroll
  for (int off = G / 2; off > 0; off >>= 1) s += __shfl_xor(s, off);
  if (threadIdx.x % G == 0) p.delta[l_off] = s;
  if (c >= D || !p.dq_acc) return;
  float* qa = p.dq_acc + qa_off + c;
  *reinterpret_cast<f32x4*>(qa) = f32x4{0.f, 0.f, 0.f, 0.f};
  *reinterpret_cast<f32x4*>(qa + 4) = f32x4{0.f, 0.f, 0.f, 0.f};
}

// dQ = fp16(dq_acc * scale)
template <class T, int D>
__global__ void __launch_bounds__(256)
bwd_post_kernel(BwdParams p, int rows, int batched) {
  using V8 = vec8<T>;
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
  V8 h;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    h[j] = (T)(x0[j] * p.scale);
    h[j + 4] = (T)(x1[j] * p.scale);
  }
  st_u4((T*)p.dq + dq_off + c, __builtin_bit_cast(u32x4, h));
}

#ifndef FAL_PRESCALE_FP16
#define FAL_PRESCALE_FP16 0
#endif
#ifndef FAL_BWD_KLDS
#define FAL_BWD_KLDS 1   // head_dim 256: K fragments from the LDS K tile (+20%: no K registers to spill)
#endif
#ifndef FAL_BWD_DW
#define FAL_BWD_DW 256   // head_dim 256: dK/dV columns held per pass (256: one pass, +11% over two passes of 128)
#endif

// --------------------------------------------------------------------------
// Main KV-outer kernel
// --------------------------------------------------------------------------
template <class T, int D, int NW, int BMQ, bool CAUSAL>
__global__ void __launch_bounds__(NW * 64)
bwd_kernel(BwdParams p) {
  using V8 = vec8<T>;
  using V4 = vec4<T>;
  static_assert(BMQ == 32, "query tile is one 32-row MFMA block");
  constexpr int BN = NW * 32;
  constexpr int KS = D / 16;
  constexpr int DW = D > FAL_BWD_DW ? FAL_BWD_DW : D;   // dK/dV columns accumulated per pass
  constexpr int NPASS = D / DW;
  constexpr int DWB = DW / 32;
  constexpr int DQB = D / 32;
  constexpr int LDK = D + 8;
  constexpr int LDQ = BMQ + 8;
  constexpr int QCH = BMQ * D / 8;                   // 16B chunks per Q (or dO) tile
  constexpr int QCPT = (QCH + NW * 64 - 1) / (NW * 64);
  constexpr int CPR = D / 8;

  __shared__ __attribute__((aligned(16))) T ks_s[BN * LDK];
  __shared__ __attribute__((aligned(16))) T q_s[BMQ * LDK];
  __shared__ __attribute__((aligned(16))) T do_s[BMQ * LDK];
  __shared__ __attribute__((aligned(16))) T dst_s[BN * LDQ];
  __shared__ __attribute__((aligned(16))) float l_s[BMQ];
  __shared__ __attribute__((aligned(16))) float d_s[BMQ];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  int b, hkv, kt, q_off, k_off, nq, nk;
  if (p.cu_q) {
    // 1-D grid, KV head fastest: block i runs on XCD i % 8, so for a multiple of 8 KV
    // heads each XCD walks one KV head's items in list order (grouped by sequence) and
    // the query tiles they all read stay in its L2
    const int2 wk = p.work[blockIdx.x / p.Hkv];
    if (wk.x < 0) return;
    hkv = blockIdx.x % p.Hkv;
    b = 0;
    kt = wk.y;
    seg_bounds(p.cu_q, wk.x, p.total_q, q_off, nq);
    seg_bounds(p.cu_k, wk.x, p.total_k, k_off, nk);
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

  const T* kbase = (const T*)p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh + (int64_t)k_off * p.k_ss;
  const T* vbase = (const T*)p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh + (int64_t)k_off * p.v_ss;

  // K/V rows of this wave (B operands: n = key, k = head dim)
  const int kw0 = n0 + w * 32;
  const int key = kw0 + l32;
  // K of this wave's keys is read from the K tile in LDS (FAL_BWD_KLDS), which leaves
  // the registers to V and the dK/dV accumulators
  V8 kreg[FAL_BWD_KLDS ? 1 : KS], vreg[KS];
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    if (!FAL_BWD_KLDS) kreg[t] = key < nk ? ld8(kbase + (int64_t)key * p.k_ss + t * 16 + hh * 8) : zero8<T>();
    vreg[t] = key < nk ? ld8(vbase + (int64_t)key * p.v_ss + t * 16 + hh * 8) : zero8<T>();
  }
  // K tile, row-major, for dQ = dS K
  for (int ch = tid; ch < BN * CPR; ch += NW * 64) {
    const int r = ch / CPR, cc = (ch % CPR) * 8;
    const u32x4 x = (n0 + r < nk) ? ld_u4(kbase + (int64_t)(n0 + r) * p.k_ss + cc) : u32x4{0, 0, 0, 0};
    st_u4(ks_s + r * LDK + cc, x);
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
      const T* qbase = (const T*)p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)q_off * p.q_ss;
      const T* dobase = (const T*)p.dout + (int64_t)b * p.do_sb + (int64_t)hq * p.do_sh + (int64_t)q_off * p.do_ss;
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
          qpre[i] = ok ? ld_u4(qbase + (int64_t)(q0 + r) * p.q_ss + cc) : u32x4{0, 0, 0, 0};
          dopre[i] = ok ? ld_u4(dobase + (int64_t)(q0 + r) * p.do_ss + cc) : u32x4{0, 0, 0, 0};
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
            st_u4(q_s + r * LDK + cc, qpre[i]);
            st_u4(do_s + r * LDK + cc, dopre[i]);
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
            s = mfma32(ld8(q_s + l32 * LDK + t * 16 + hh * 8),
                       FAL_BWD_KLDS ? ld8(ks_s + (w * 32 + l32) * LDK + t * 16 + hh * 8) : kreg[t], s);
            dp = mfma32(ld8(do_s + l32 * LDK + t * 16 + hh * 8), vreg[t], dp);
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
            const V8 pb = cvt8t<T>(s, ks);
            const V8 sb = cvt8t<T>(dp, ks);
#pragma unroll
            for (int db = 0; db < DWB; ++db) {
              const int col = dbase + db * 32;
              dv_acc[db] = mfma32(kslab_tr(do_s + tofs_q + col, ks * 16, hh, LDK), pb, dv_acc[db]);
              dk_acc[db] = mfma32(kslab_tr(q_s + tofs_q + col, ks * 16, hh, LDK), sb, dk_acc[db]);
            }
          }
          if (pass == 0) {
            // dS^T (fp16) into LDS: row = key (local), columns = query rows
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              V4 h;
#pragma unroll
              for (int e = 0; e < 4; ++e) h[e] = (T)dp[g4 * 4 + e];
              *reinterpret_cast<V4*>(dst_s + (w * 32 + l32) * LDQ + g4 * 8 + hh * 4) = h;
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
              acc = mfma32(kslab_tr(dst_s + tofs_s, ks * 16, hh, LDQ),
                           kslab_tr(ks_s + tofs_q + db * 32, ks * 16, hh, LDK), acc);
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
      T* dkrow = (T*)p.dk + (int64_t)b * p.dk_sb + (int64_t)hkv * p.dk_sh + (int64_t)(k_off + key) * p.dk_ss;
      T* dvrow = (T*)p.dv + (int64_t)b * p.dv_sb + (int64_t)hkv * p.dv_sh + (int64_t)(k_off + key) * p.dv_ss;
#pragma unroll
      for (int db = 0; db < DWB; ++db)
#pragma unroll
        for (int g4 = 0; g4 < 4; ++g4) {
          V4 hk, hv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            hk[e] = (T)(dk_acc[db][g4 * 4 + e] * p.scale);
            hv[e] = (T)dv_acc[db][g4 * 4 + e];
          }
          const int col = dbase + db * 32 + g4 * 8 + hh * 4;
          *reinterpret_cast<V4*>(dkrow + col) = hk;
          *reinterpret_cast<V4*>(dvrow + col) = hv;
        }
    }
  }
}

// Scheduling fence between MFMA steps of the head_dim-128 kernel: keeps the compiler
// from hoisting every operand read of a phase at once (which overflows the 256-register
// budget of two waves per SIMD).
#ifndef FAL_BWD_FENCES
#define FAL_BWD_FENCES 1
#endif
#if FAL_BWD_FENCES
#define FAL_BWD_FENCE() __builtin_amdgcn_sched_barrier(0)
#else
#define FAL_BWD_FENCE() ((void)0)
#endif

// --------------------------------------------------------------------------
// KV-outer dK/dV kernel for head_dim 32, 64, 96 and 128 (the dQ kernel below runs first and
// stores D = rowsum(dO * O)).
//
// A 4-wave workgroup owns BN = 64 keys of one KV head: wave w takes keys
// 32*(w%2) .. +32 and query half w/2 of each 64-row query tile.  It walks every
// (query head of the GQA group, query tile) item; per item each wave forms
// S = Q K^T and dP = dO V^T for its 32 keys x 32 rows, P = exp2(S - L*log2e),
// dS = P (dP - D), then dV^T += dO^T P and dK^T += Q^T dS in registers (Q^T, dO^T
// read transposed from LDS, P and dS taken from the accumulators as B operands).
//   - The S accumulator starts at -L*log2e / c (c = scale*log2e) and the dP
//     accumulator at -D, so the MFMAs produce the exponent of P over c and dP - D
//     directly: one multiply and an exp2 per element.
//   - Operands of MFMA step t+1 are read before the MFMAs of step t.
//   - Only tiles that straddle the diagonal apply the causal mask.
//   - MFMA phases run at raised wave priority, so a SIMD's other wave fills their
//     gaps rather than delaying them.
// K/V tiles and the single-buffered Q/dO tile are staged in swizzled LDS by direct
// buffer loads (66 KB, two workgroups per CU).  For causal attention a workgroup
// takes key tiles kt and n-1-kt, so all workgroups do the same work.  The two query
// halves' dK/dV partials are summed in LDS, in a fixed order.
// --------------------------------------------------------------------------
#ifndef FAL_BWD2_NW
#define FAL_BWD2_NW 4   // waves per workgroup: 4 (64 keys, 2 workgroups per CU) or 8 (128 keys, double-buffered Q/dO)
#endif
template <class T, int D, bool CAUSAL, bool FUSED>
__global__ void __launch_bounds__(FAL_BWD2_NW * 64) __attribute__((amdgpu_waves_per_eu(2, 8)))
bwd2_kernel(BwdParams p) {
  using V8 = vec8<T>;
  using V4 = vec4<T>;
  // K stays exact and scale*log2(e) is applied to the fp32 scores (one multiply).
  // FAL_PRESCALE_FP16 instead pre-multiplies an fp16 K tile in LDS
  // (rounded once) and starts the S accumulator at -L*log2e; that rounding costs
  // accuracy at large logits, so it is off.
  constexpr bool PRESCALE = FAL_PRESCALE_FP16 && std::is_same<T, half_t>::value;
  using TL = SwizzledTile<D>;
  constexpr int NW = FAL_BWD2_NW, BN = NW * 16, BMQ = 64;
  constexpr int NKG = NW / 2;             // key groups of 32 (x 2 query halves)
  constexpr bool DBUF = NW == 8;          // Q/dO double buffer (else one buffer, 2 WG/CU)
  constexpr int KS = D / 16;
  constexpr int DWB = D / 32;
  constexpr int CPR = TL::CPR;
  constexpr int KPART = BN * CPR * 8;     // elements of the K (or V) tile
  constexpr int QPART = BMQ * CPR * 8;    // elements of one Q (or dO) tile
  constexpr int KIPT = BN * CPR / (NW * 64);
  constexpr int QIPT = BMQ * CPR / (NW * 64);
  static_assert(BMQ * CPR % (NW * 64) == 0, "Q tile must split evenly over the waves");
  static_assert((DBUF ? 2 : 1) * 2 * QPART * 2 >= NKG * 32 * D * 4, "dK/dV reduction reuses the Q/dO buffers");
  static_assert(!(FUSED && PRESCALE), "the fused dQ product needs the unscaled K tile");
  static_assert(!FUSED || NW == 4, "the fused dQ product splits 64 rows x D over four waves");
  constexpr int LDQ = BMQ + 8;            // dS^T tile row stride (fused): 64 query rows + pad

  __shared__ __attribute__((aligned(1024))) T ks_s[KPART];
  __shared__ __attribute__((aligned(1024))) T vs_s[KPART];
  __shared__ __attribute__((aligned(1024))) T qd_s[(DBUF ? 2 : 1) * 2 * QPART];   // [buffer][Q, dO]
  __shared__ float l_s[2][BMQ];
  __shared__ float d_s[2][BMQ];
  // fused: dS^T of the current item, row = key of the tile, column = query row of the item
  __shared__ __attribute__((aligned(16))) T dst_s[FUSED ? BN * LDQ : 8];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int ws = __builtin_amdgcn_readfirstlane(w);
  const int kg = w % NKG;                 // key group
  const int qh = w / NKG;                 // query half
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  // ---- work item: up to two key tiles of one (batch, KV head) ----
  int b, hkv, q_off, k_off, nq, nk, kt_a, kt_b;
  if (p.cu_q) {
    // 1-D grid, KV head fastest: block i runs on XCD i % 8, so for a multiple of 8 KV
    // heads each XCD walks one KV head's items in list order (grouped by sequence) and
    // the query tiles they all read stay in its L2
    const int2 wk = p.work[blockIdx.x / p.Hkv];
    if (wk.x < 0) return;
    hkv = blockIdx.x % p.Hkv;
    b = 0;
    kt_a = wk.y;
    kt_b = -1;
    seg_bounds(p.cu_q, wk.x, p.total_q, q_off, nq);
    seg_bounds(p.cu_k, wk.x, p.total_k, k_off, nk);
  } else {
    const int total = gridDim.x;
    int id = blockIdx.x;
    if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
    const int nitems = CAUSAL ? (p.n_ktiles + 1) / 2 : p.n_ktiles;
    const int it = id % nitems;
    const int bh = id / nitems;
    b = bh / p.Hkv;
    hkv = bh % p.Hkv;
    kt_a = it;
    kt_b = (CAUSAL && p.n_ktiles - 1 - it != it) ? p.n_ktiles - 1 - it : -1;
    q_off = 0;
    k_off = 0;
    nq = p.Nq;
    nk = p.Nk;
  }
  const int G = p.Hq / p.Hkv;
  const float c = p.scale_log2;
  const T* kbase = (const T*)p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh + (int64_t)k_off * p.k_ss;
  const T* vbase = (const T*)p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh + (int64_t)k_off * p.v_ss;

  // per-lane direct-load byte offsets from a tile's first row (instruction i of wave ws
  // fills chunks [(i*NW+ws)*64, +64)); one buffer resource per tile bounds the rows
  auto dl_offset = [&](int i, int64_t ss) {
    const int I = i * NW + ws;
    const int pch = I * 64 + lane;
    const int r = pch / CPR;
    return (r * (int)ss + TL::logical_chunk(r, pch % CPR) * 8) * 2;
  };
  // Fragment reads (row l32 of a 32-row block, chunk 2t+hh) and transposed reads
  // (rows hf*8 + hh*4 + i/4 of a 16-row step, 32-column block db) of the swizzled
  // tiles.  The swizzle is an XOR on the chunk index, so every address is a lane
  // base XOR a compile-time chunk offset; keeping only the bases saves registers.
  const int fbase = TL::offset(l32, hh);
  int trb[2];
  {
    const int i = lane & 15;
    const int rl = hh * 4 + (i >> 2);
    const int cl = 2 * ((lane >> 4) & 1) + ((lane >> 1) & 1);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      trb[hf] = TL::offset(hf * 8 + rl, cl);
    }
  }
  const int tr_lo = 4 * (lane & 1);
  // (The XOR form needs a power-of-two row length in chunks; head_dim 96 has 12 and
  // takes the full offsets.)
  constexpr bool POW2 = (CPR & (CPR - 1)) == 0;
  auto faddr = [&](int t) { return POW2 ? (fbase ^ ((2 * t) << 3)) : TL::offset(l32, 2 * t + hh); };
  const int trl = hh * 4 + ((lane & 15) >> 2);
  const int trc = 2 * ((lane >> 4) & 1) + ((lane >> 1) & 1);
  auto tra = [&](int hf, int db) {
    return POW2 ? (trb[hf] ^ ((db * 4) << 3)) : TL::offset(hf * 8 + trl, db * 4 + trc);
  };
  // 8 k-slots for rows row0.. (multiple of 16) of a swizzled D-column tile, block db
  auto trk = [&](const T* base, int db, int row0) {
    const V4 lo = lds_tr(base + tra(0, db) + tr_lo + row0 * CPR * 8);
    const V4 hi = lds_tr(base + tra(1, db) + tr_lo + row0 * CPR * 8);
    return join8(lo, hi);
  };
  const int nqt = cdiv(nq, BMQ);

  for (int tile_i = 0; tile_i < 2; ++tile_i) {
    const int kt = tile_i == 0 ? kt_a : kt_b;
    if (kt < 0) break;
    const int n0 = kt * BN;
    if (n0 >= nk) continue;
    const int kw0 = n0 + kg * 32;
    const int key = kw0 + l32;

    __syncthreads();   // previous tile's readers of the LDS tiles are done
    {
      const int64_t left = (int64_t)max(nk - n0, 0);
      const __amdgpu_buffer_rsrc_t krs =
          make_rsrc(kbase + (int64_t)n0 * p.k_ss, (uint32_t)min(left * p.k_ss * 2, (int64_t)0x7fffffff));
      const __amdgpu_buffer_rsrc_t vrs =
          make_rsrc(vbase + (int64_t)n0 * p.v_ss, (uint32_t)min(left * p.v_ss * 2, (int64_t)0x7fffffff));
#pragma unroll
      for (int i = 0; i < KIPT; ++i) {
        const int I = i * NW + ws;
        buffer_to_lds16(krs, dl_offset(i, p.k_ss), ks_s + I * 64 * 8);
        buffer_to_lds16(vrs, dl_offset(i, p.v_ss), vs_s + I * 64 * 8);
      }
    }

    f32x16 dk_acc[DWB], dv_acc[DWB];
#pragma unroll
    for (int i = 0; i < DWB; ++i) {
      dk_acc[i] = zero_f16();
      dv_acc[i] = zero_f16();
    }
    // (FAL_PRESCALE_FP16 only) K tile *= scale*log2e, rounded once to fp16, so that S
    // comes out of the MFMAs in log2 units and its accumulator can start at -L*log2e
    wait_vmcnt0();
    __syncthreads();
#pragma unroll
    for (int i = 0; i < (PRESCALE ? KPART / (NW * 64 * 8) : 0); ++i) {
      T* ptr = ks_s + (i * NW * 64 + tid) * 8;
      V8 v = ld8(ptr);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (T)((float)v[e] * c);
      *reinterpret_cast<V8*>(ptr) = v;
    }
    const int qt0 = CAUSAL ? (n0 / BMQ) : 0;
    // (query head, query tile) items of this key tile, in one sequence so the Q/dO
    // double buffer alternates across head boundaries too: the fetch of item it+1
    // goes to the buffer item it-1 used, which every wave has finished with once it
    // passes item it's barrier.
    const int ntq = nqt > qt0 ? nqt - qt0 : 0;
    const int nitems_q = G * ntq;
    float lpre = 0.f, dpre = 0.f;
    // the next item to fetch, (query head, query tile), walked with counters: the
    // scalar unit has no divide
    int f_hq = hkv * G, f_qt = qt0;
    auto fetch = [&](int buf) {
      const int hq = f_hq;
      const int q0 = f_qt * BMQ;
      if (++f_qt == nqt) {
        f_qt = qt0;
        ++f_hq;
      }
      const T* qbase = (const T*)p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)(q_off + q0) * p.q_ss;
      const T* dobase =
          (const T*)p.dout + (int64_t)b * p.do_sb + (int64_t)hq * p.do_sh + (int64_t)(q_off + q0) * p.do_ss;
      const int64_t left = (int64_t)max(nq - q0, 0);
      const __amdgpu_buffer_rsrc_t qrs = make_rsrc(qbase, (uint32_t)min(left * p.q_ss * 2, (int64_t)0x7fffffff));
      const __amdgpu_buffer_rsrc_t dors = make_rsrc(dobase, (uint32_t)min(left * p.do_ss * 2, (int64_t)0x7fffffff));
#pragma unroll
      for (int i = 0; i < QIPT; ++i) {
        const int I = i * NW + ws;
        buffer_to_lds16(qrs, dl_offset(i, p.q_ss), qd_s + (buf * 2 + 0) * QPART + I * 64 * 8);
        buffer_to_lds16(dors, dl_offset(i, p.do_ss), qd_s + (buf * 2 + 1) * QPART + I * 64 * 8);
      }
      // -L*log2e and -D, the initial values of the S and dP accumulators; a row
      // past the end (or with no keys) gets -inf, so its P is 0
      if (tid < BMQ) {
        float nl = -INFINITY, nd = 0.f;
        if (q0 + tid < nq) {
          const int64_t o = (int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)(q_off + q0 + tid) * p.l_ss;
          const float L = p.lse[o];
          nl = (L == -INFINITY) ? -INFINITY : -L * kLog2e;
          nd = -p.delta[o];
        }
        // without the K pre-scale the S accumulator starts at -L*log2e / c, so that
        // c * S is the exponent (a row with L = -inf keeps exponent -inf for either sign of c)
        if (!PRESCALE) nl /= c;
        lpre = nl;
        dpre = nd;
      }
    };

    if (nitems_q > 0) fetch(0);
    int c_qt = qt0;   // query tile of the current item
    int c_hq = 0;     // its query head within the group
    for (int item = 0; item < nitems_q; ++item) {
      {
        const int buf = DBUF ? (item & 1) : 0;
        const int q0 = c_qt * BMQ;
        const int cur_hq = c_hq;
        if (++c_qt == nqt) {
          c_qt = qt0;
          ++c_hq;
        }
        (void)cur_hq;
        wait_vmcnt0();
        if (tid < BMQ) {
          l_s[buf][tid] = lpre;
          d_s[buf][tid] = dpre;
        }
        __syncthreads();                  // barrier A: item in LDS; readers of item-1 done
        if (DBUF && item + 1 < nitems_q) fetch(buf ^ 1);
        const T* q_s = qd_s + (buf * 2 + 0) * QPART + qh * 32 * CPR * 8;
        const T* do_s = qd_s + (buf * 2 + 1) * QPART + qh * 32 * CPR * 8;
        const int qr0 = q0 + qh * 32;     // first query row of this wave's half
        if (!CAUSAL || qr0 + 31 >= kw0) {
          // S = Q K^T - L*log2e/c and dP = dO V^T - D
          f32x16 s, dp;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const f32x4 ln = *reinterpret_cast<const f32x4*>(&l_s[buf][qh * 32 + g4 * 8 + hh * 4]);
            const f32x4 dn = *reinterpret_cast<const f32x4*>(&d_s[buf][qh * 32 + g4 * 8 + hh * 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              s[g4 * 4 + e] = ln[e];
              dp[g4 * 4 + e] = dn[e];
            }
          }
          __builtin_amdgcn_s_setprio(1);
          // operands of step t+1 are read before the MFMAs of step t
          const T* kw_s = ks_s + kg * 32 * CPR * 8;
          const T* vw_s = vs_s + kg * 32 * CPR * 8;
          V8 oq = ld8(q_s + faddr(0)), ok = ld8(kw_s + faddr(0));
          V8 od = ld8(do_s + faddr(0)), ov = ld8(vw_s + faddr(0));
#pragma unroll
          for (int t = 0; t < KS; ++t) {
            V8 nq = oq, nk = ok, nd = od, nv = ov;   // (unused after the last step)
            if (t + 1 < KS) {
              const int fa = faddr(t + 1);
              nq = ld8(q_s + fa);
              nk = ld8(kw_s + fa);
              nd = ld8(do_s + fa);
              nv = ld8(vw_s + fa);
            }
            s = mfma32(oq, ok, s);
            dp = mfma32(od, ov, dp);
            FAL_BWD_FENCE();
            oq = nq; ok = nk; od = nd; ov = nv;
          }
          __builtin_amdgcn_s_setprio(0);
          // P = exp2(S) and dS = P dP; element i: query qr0 + (i/4)*8 + hh*4 + i%4, key `key`.
          // Query rows past the end carry L = +inf (P = 0), and keys past the end only
          // feed dK/dV rows that are never written, so the causal test is the only mask:
          // key > query  <=>  key - qr0 - hh*4 > (i/4)*8 + i%4, a constant per element.
          const int cthr = key - qr0 - hh * 4;
          auto grad = [&](auto masked) {
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int i = g4 * 4 + e;
                float pv = fast_exp2(PRESCALE ? s[i] : s[i] * c);
                if (decltype(masked)::value && cthr > g4 * 8 + e) pv = 0.f;
                s[i] = pv;
                dp[i] = pv * dp[i];
              }
            }
          };
          // only a tile that straddles the diagonal has keys past some of its queries
          if (CAUSAL && kw0 + 31 > qr0) grad(std::integral_constant<bool, true>{});
          else grad(std::integral_constant<bool, false>{});
          // dV^T += dO^T P ; dK^T += Q^T dS
          __builtin_amdgcn_s_setprio(1);
          {
            V8 pb[2], sb[2];
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
              pb[ks] = cvt8t<T>(s, ks);
              sb[ks] = cvt8t<T>(dp, ks);
            }
            V8 ao = trk(do_s, 0, 0), aq = trk(q_s, 0, 0);
#pragma unroll
            for (int st = 0; st < 2 * DWB; ++st) {
              const int ks = st / DWB, db = st % DWB;
              V8 no = ao, nq = aq;   // (unused after the last step)
              if (st + 1 < 2 * DWB) {
                no = trk(do_s, (st + 1) % DWB, (st + 1) / DWB * 16);
                nq = trk(q_s, (st + 1) % DWB, (st + 1) / DWB * 16);
              }
              dv_acc[db] = mfma32(ao, pb[ks], dv_acc[db]);
              dk_acc[db] = mfma32(aq, sb[ks], dk_acc[db]);
              FAL_BWD_FENCE();
              ao = no; aq = nq;
            }
          }
          __builtin_amdgcn_s_setprio(0);
          if constexpr (FUSED) {
            // this wave's dS^T block (32 keys x 32 query rows) into the tile
            T* drow = dst_s + (kg * 32 + l32) * LDQ + qh * 32 + hh * 4;
#pragma unroll
            for (int g4 = 0; g4 < 4; ++g4) {
              V4 h;
#pragma unroll
              for (int e = 0; e < 4; ++e) h[e] = (T)dp[g4 * 4 + e];
              *reinterpret_cast<V4*>(drow + g4 * 8) = h;
            }
          }
        } else if constexpr (FUSED) {
          // every key of this wave is past every query row of its half: dS = 0
          T* drow = dst_s + (kg * 32 + l32) * LDQ + qh * 32 + hh * 4;
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) *reinterpret_cast<u32x2*>(drow + g4 * 8) = u32x2{0, 0};
        }
        if constexpr (FUSED) {
          // dQ[q, :] += dS[q, keys] K[keys, :] over the tile's 64 keys, added to the fp32
          // accumulator with atomics (the reference's scheme, flash_attn_bwd.cu:602-620).
          // Wave (kg, qh) takes query half qh and head-dim columns kg*D/2 .. +D/2.
          __syncthreads();                // barrier C: the dS^T tile is complete
          constexpr int QDB = D / 64;     // 32-wide head-dim blocks per wave
          const int tofs_s = tr_offset(lane, LDQ) + qh * 32;
          // one buffer resource over the item's accumulator rows: adds to rows past the
          // end of the sequence fall outside it and are dropped
          const float* qa = p.dq_acc + (int64_t)b * p.dqa_sb + (int64_t)(hkv * G + cur_hq) * p.dqa_sh +
                            (int64_t)(q_off + q0) * p.dqa_ss;
          const __amdgpu_buffer_rsrc_t qrs =
              make_rsrc(qa, (uint32_t)min((int64_t)max(nq - q0, 0) * p.dqa_ss * 4, (int64_t)0x7fffffff));
          // lane part of the byte offset in a VGPR, the row step of element i in the
          // instruction's scalar offset
          const int qrow_bytes = __builtin_amdgcn_readfirstlane((int)p.dqa_ss * 4);
          const int qoff = ((qh * 32 + hh * 4) * (int)p.dqa_ss + kg * QDB * 32 + l32) * 4;
#pragma unroll
          for (int j = 0; j < QDB; ++j) {
            // one 32-column block at a time (16 accumulator registers)
            f32x16 qacc = zero_f16();
#pragma unroll
            for (int ks = 0; ks < BN / 16; ++ks)
              qacc = mfma32(kslab_tr(dst_s + tofs_s, ks * 16, hh, LDQ), trk(ks_s, kg * QDB + j, ks * 16), qacc);
#pragma unroll
            for (int i = 0; i < 16; ++i)
              __builtin_amdgcn_raw_ptr_buffer_atomic_fadd_f32(qacc[i], qrs, qoff + j * 128,
                                                              ((i >> 2) * 8 + (i & 3)) * qrow_bytes, 0);
          }
        }
        if (!DBUF && item + 1 < nitems_q) {
          __syncthreads();                // barrier B: every wave is done with this item's tile
          fetch(0);
        }
      }
    }

    // ---- sum the two query halves' dK/dV and write this tile's rows ----
    __syncthreads();
    // The partner waves (same key group, same lane layout) meet in LDS: the second
    // query half stages its accumulators lane-contiguous, [kg][db][i][lane], and the
    // first adds them element by element (bank-conflict free, no transpose).
    float* red = reinterpret_cast<float*>(qd_s);
    auto reduce_write = [&](f32x16 (&acc)[DWB], T* row, float sc) {
      float* mine = red + (size_t)kg * DWB * 16 * 64 + lane;
      if (qh == 1) {
#pragma unroll
        for (int db = 0; db < DWB; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) mine[(db * 16 + i) * 64] = acc[db][i];
      }
      __syncthreads();
      if (qh == 0 && key < nk) {
#pragma unroll
        for (int db = 0; db < DWB; ++db)
#pragma unroll
          for (int g4 = 0; g4 < 4; ++g4) {
            const int col = db * 32 + g4 * 8 + hh * 4;
            V4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = (T)((acc[db][g4 * 4 + e] + mine[(db * 16 + g4 * 4 + e) * 64]) * sc);
            *reinterpret_cast<V4*>(row + col) = h;
          }
      }
      __syncthreads();
    };
    const int64_t krow = (int64_t)(k_off + min(key, max(nk - 1, 0)));
    reduce_write(dk_acc, (T*)p.dk + (int64_t)b * p.dk_sb + (int64_t)hkv * p.dk_sh + krow * p.dk_ss, p.scale);
    reduce_write(dv_acc, (T*)p.dv + (int64_t)b * p.dv_sb + (int64_t)hkv * p.dv_sh + krow * p.dv_ss, 1.f);
  }
}


// --------------------------------------------------------------------------
// dK/dV kernel for head_dim 128, batched (bwd_kv_pipe_kernel): one wave per SIMD and a
// software-pipelined query-tile loop written as one inline-asm block (fal_bwd_pipe.inc,
// generated by gen_bwd_pipe.py).  A workgroup owns 128 keys of one KV head, each wave
// 32 keys whose K and V fragments stay in registers; the items (query head of the
// group, 64-row query tile) stream through a 4-slot LDS ring of Q/dO tiles copied two
// items ahead.  Per item the S and dP accumulators start at -L*log2(e)/c and -D, read
// from the tile-major array `lsd` that bwd_dq_kernel writes, so P = exp2(c*S) and
// dS = P*dP.  The products of item i-1 (dV^T += dO^T P, dK^T += Q^T dS), the
// exponentials of item i and the products of item i+1 (S = Q K^T, dP = dO V^T)
// overlap inside the wave; no cross-wave sum is needed.  Same math as bwd2_kernel.
// --------------------------------------------------------------------------
#ifndef FAL_BWD_PIPE
#define FAL_BWD_PIPE 1
#endif
constexpr int kPipeBN = 128;    // keys per workgroup
// dK/dV hand-off in LDS after the loop: per wave, dV then dK*scale, 16 pieces of 512
// bytes each, kKvOStr apart so the row-wise reads of the epilogue spread over the banks
constexpr int kKvOStr = 528;
constexpr int kKvOPart = 16 * kKvOStr;
constexpr int kKvOWave = 2 * kKvOPart;
constexpr int kPipeBM = 64;     // query rows per item

template <class T, bool CAUSAL>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
bwd_kv_pipe_kernel(BwdParams p) {
  using V8 = vec8<T>;
  using TL = SwizzledTile<128>;
  constexpr int CPR = TL::CPR;
  // 4 slots of (Q tile, dO tile) and 4 slots of (64 Ls, 64 Dn) values
  __shared__ __attribute__((aligned(1024))) char smem[4 * 32768 + 4 * 512];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int ws = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  // work item: one or two 128-key tiles of one (batch, KV head); causal tiles are
  // paired (kt, n-1-kt) so every workgroup has the same number of items
  const int nkt = cdiv(p.Nk, kPipeBN);
  const int total = gridDim.x;
  int id = blockIdx.x;
  if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
  const int nk_items = CAUSAL ? (nkt + 1) / 2 : nkt;
  const int kit = id % nk_items;
  const int bh = id / nk_items;
  const int b = bh / p.Hkv, hkv = bh % p.Hkv;
  const int kt_b = (CAUSAL && nkt - 1 - kit != kit) ? nkt - 1 - kit : -1;
  const int G = p.Hq / p.Hkv;
  const int nq = p.Nq, nk = p.Nk;
  const int nqt = cdiv(nq, kPipeBM);

  typedef __attribute__((address_space(3))) char lds_t;
  const uint32_t lds0 = (uint32_t)(uintptr_t)((lds_t*)smem);
  // per-lane LDS addresses: fragment (row l32, chunk 2t+hh) and transposed reads
  // (rows hf*8 + hh*4 + i/4 of a 16-row step, 32-column block db) of a slot's tiles
  uint32_t p_qa[8], p_ta[2][4];
#pragma unroll
  for (int t = 0; t < 8; ++t) p_qa[t] = lds0 + 2 * TL::offset(l32, 2 * t + hh);
  {
    const int i = lane & 15;
    const int rl = hh * 4 + (i >> 2);
    const int cl = 2 * ((lane >> 4) & 1) + ((lane >> 1) & 1);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int db = 0; db < 4; ++db) p_ta[hf][db] = lds0 + 2 * (TL::offset(hf * 8 + rl, db * 4 + cl) + 4 * (lane & 1));
  }
  const uint32_t p_la = lds0 + 131072 + 16 * hh;
  // copy offsets: load i of wave ws fills chunks [(4i + ws)*64, +64) of a tile
  int p_qo[4], p_do[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int pch = (i * 4 + ws) * 64 + lane;
    const int r = pch / CPR;
    const int cc = TL::logical_chunk(r, pch % CPR);
    p_qo[i] = (int)(r * p.q_ss + cc * 8) * 2;
    p_do[i] = (int)(r * p.do_ss + cc * 8) * 2;
  }
  const int p_lo4 = lane * 4, p_lo4b = 256 + lane * 4;
  const int p_lk = l32 - 4 * hh;
  const uint32_t p_olds = lds0 + ws * kKvOWave + lane * 8;
  const uint32_t p_lbase = __builtin_amdgcn_readfirstlane(lds0 + ws * 1024);
  const uint32_t p_ldbase = __builtin_amdgcn_readfirstlane(lds0 + 131072);
  const float p_c = p.scale_log2;
  const float p_negc = p.scale_log2 > 0.f ? -INFINITY : INFINITY;   // c * negc = -inf
  const float p_scale = p.scale;
  const uint32_t p_qrb = (uint32_t)(p.q_ss * 2), p_drb = (uint32_t)(p.do_ss * 2);
  const int p_nq = nq, p_nqt = nqt;
  const int64_t qstep = (int64_t)kPipeBM * p.q_ss * 2, dstep = (int64_t)kPipeBM * p.do_ss * 2;

  // K and V of this wave's 32 keys of key tile kt (B operands), buffer loads: keys past
  // the end read as zeros.  The second tile's are loaded right after the first tile's
  // loop, so their latency overlaps that tile's epilogue.
  V8 kreg[8], vreg[8];
  auto load_kv = [&](int kt) {
    // one resource per key tile: its rows inside the sequence, offsets from its first row
    const int n0 = kt * kPipeBN;
    const int64_t rows = min(max((int64_t)p.Nk - n0, (int64_t)0), (int64_t)kPipeBN);
    const __amdgpu_buffer_rsrc_t krs =
        make_rsrc((const T*)p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh + (int64_t)n0 * p.k_ss,
                  (uint32_t)(rows * p.k_ss * 2));
    const __amdgpu_buffer_rsrc_t vrs =
        make_rsrc((const T*)p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh + (int64_t)n0 * p.v_ss,
                  (uint32_t)(rows * p.v_ss * 2));
    const int r = ws * 32 + l32;
    const int ko = (int)(r * p.k_ss * 2) + hh * 16, vo = (int)(r * p.v_ss * 2) + hh * 16;
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      kreg[t] = __builtin_bit_cast(V8, __builtin_amdgcn_raw_buffer_load_b128(krs, ko + t * 32, 0, 0));
      vreg[t] = __builtin_bit_cast(V8, __builtin_amdgcn_raw_buffer_load_b128(vrs, vo + t * 32, 0, 0));
    }
  };
  load_kv(kit);
  for (int tile_i = 0; tile_i < 2; ++tile_i) {
    const int kt = tile_i == 0 ? kit : kt_b;
    if (kt < 0) break;
    const int n0 = kt * kPipeBN;
    const int kw0 = n0 + ws * 32;
    const int qt0 = CAUSAL ? n0 / kPipeBM : 0;
    const int ntq = max(nqt - qt0, 0);
    const int nitems = G * ntq;
    __syncthreads();   // the previous tile's epilogue readers are done with the LDS
    if (nitems > 0) {
      const int hq0 = hkv * G;
      const uint64_t qb = (uint64_t)(uintptr_t)((const T*)p.q + (int64_t)b * p.q_sb + (int64_t)hq0 * p.q_sh +
                                                (int64_t)qt0 * kPipeBM * p.q_ss);
      const uint64_t dob = (uint64_t)(uintptr_t)((const T*)p.dout + (int64_t)b * p.do_sb +
                                                 (int64_t)hq0 * p.do_sh + (int64_t)qt0 * kPipeBM * p.do_ss);
      const uint64_t lb = (uint64_t)(uintptr_t)(p.lsd + (((int64_t)b * p.Hq + hq0) * nqt + qt0) * 2 * kPipeBM);
      const int64_t qwrap = p.q_sh * 2 - (int64_t)(ntq - 1) * qstep;
      const int64_t dwrap = p.do_sh * 2 - (int64_t)(ntq - 1) * dstep;
      const uint32_t p_qb_lo = (uint32_t)qb, p_qb_hi = (uint32_t)(qb >> 32) & 0xffffu;
      const uint32_t p_db_lo = (uint32_t)dob, p_db_hi = (uint32_t)(dob >> 32) & 0xffffu;
      const uint32_t p_lb_lo = (uint32_t)lb, p_lb_hi = (uint32_t)(lb >> 32) & 0xffffu;
      const uint32_t p_qs_lo = (uint32_t)qstep, p_qs_hi = (uint32_t)((uint64_t)qstep >> 32);
      const uint32_t p_qw_lo = (uint32_t)qwrap, p_qw_hi = (uint32_t)((uint64_t)qwrap >> 32);
      const uint32_t p_ds_lo = (uint32_t)dstep, p_ds_hi = (uint32_t)((uint64_t)dstep >> 32);
      const uint32_t p_dw_lo = (uint32_t)dwrap, p_dw_hi = (uint32_t)((uint64_t)dwrap >> 32);
      const uint32_t p_ldw = (uint32_t)(1 + qt0) * 2 * kPipeBM * 4;   // last tile of a head -> first of the next
      const int p_qt0 = qt0, p_nitems = nitems;
      const int p_kw0 = CAUSAL ? kw0 : -(1 << 30);
      if constexpr (std::is_same<T, half_t>::value)
        asm volatile(FAL_BWDP_ASM_F16 : FAL_BWDP_OUTS : FAL_BWDP_INS : FAL_BWDP_CLOBBERS);
      else
        asm volatile(FAL_BWDP_ASM_BF16 : FAL_BWDP_OUTS : FAL_BWDP_INS : FAL_BWDP_CLOBBERS);
    }
    if (tile_i == 0 && kt_b >= 0) load_kv(kt_b);
    // dV then dK*scale of this wave's keys: piece pc = db*4 + g4 of lane (hh, l32) holds
    // columns 8*pc + hh*4 .. +3 of key kw0 + l32, at which*kKvOPart + pc*kKvOStr + lane*8.
    // Written back row-wise: each 16-byte store instruction covers 4 whole 256-byte rows.
    {
      const char* wb = smem + ws * kKvOWave;
      const int cch = lane & 15;
      // buffer resources over this wave's keys inside the sequence: stores past the end
      // are dropped (no branch, no 64-bit address per store)
      const int nkw = max(min(nk - kw0, 32), 0);
      const __amdgpu_buffer_rsrc_t rs[2] = {
          make_rsrc((T*)p.dv + (int64_t)b * p.dv_sb + (int64_t)hkv * p.dv_sh + (int64_t)kw0 * p.dv_ss,
                    (uint32_t)((int64_t)nkw * p.dv_ss * 2)),
          make_rsrc((T*)p.dk + (int64_t)b * p.dk_sb + (int64_t)hkv * p.dk_sh + (int64_t)kw0 * p.dk_ss,
                    (uint32_t)((int64_t)nkw * p.dk_ss * 2))};
      const int vo[2] = {((lane >> 4) * (int)p.dv_ss + cch * 8) * 2, ((lane >> 4) * (int)p.dk_ss + cch * 8) * 2};
      const int rstep[2] = {(int)p.dv_ss * 8, (int)p.dk_ss * 8};   // 4 rows, in bytes
#pragma unroll
      for (int which = 0; which < 2; ++which) {
        u32x4 x[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
          const int r = jj * 4 + (lane >> 4);
          const char* src = wb + which * kKvOPart + cch * kKvOStr;
          const uint2 lo = *reinterpret_cast<const uint2*>(src + r * 8);
          const uint2 hi = *reinterpret_cast<const uint2*>(src + (32 + r) * 8);
          x[jj] = nitems > 0 ? u32x4{lo.x, lo.y, hi.x, hi.y} : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) buffer_store16(rs[which], vo[which] + jj * rstep[which], x[jj]);
      }
    }
  }
}

// --------------------------------------------------------------------------
// Query-outer dQ kernel for head_dim 32, 64, 96 and 128 (the KV-outer kernel above then
// produces only dK/dV).  Same structure as the forward kernel: a workgroup owns
// 32*NW query rows of one query head, each wave 32 rows whose Q and dO slices stay
// in VGPRs as the B operands of S^T = K Q^T and dP^T = V dO^T; K/V tiles of BN keys
// are staged in swizzled LDS by direct buffer loads, double-buffered.  Per tile:
// P^T = exp2(S^T * scale*log2e - L*log2e), dS^T = P^T (dP^T - D), and
// dQ^T += K^T dS^T with dS^T taken straight from the accumulator as the B operand
// and K^T read transposed from the K tile.  dQ is written once, in fp16, scaled:
// no fp32 accumulator and no atomics.
// --------------------------------------------------------------------------
#ifndef FAL_BWD_DQ_PAIR
#define FAL_BWD_DQ_PAIR 1
#endif
// pipelined dQ loop's hand-off in LDS: 16 blocks of 1 KB per wave, kDqOStr apart (row-wise
// reads of the epilogue spread over the banks)
constexpr int kDqOStr = 1040;
constexpr int kDqOWave = 16 * kDqOStr;
#ifndef FAL_BWD_DQ_WPE
#define FAL_BWD_DQ_WPE 2
#endif
#ifndef FAL_BWD_DQ_PIPE
#define FAL_BWD_DQ_PIPE 1   // batched head_dim 128: software-pipelined key-tile loop (fal_dq_pipe.inc)
#endif
template <class T, int D, int NW, int BN, bool CAUSAL, bool PIPE = false>
__global__ void __launch_bounds__(NW * 64)
__attribute__((amdgpu_waves_per_eu(PIPE ? 1 : FAL_BWD_DQ_WPE, PIPE ? 1 : 8)))
bwd_dq_kernel(BwdParams p) {
  using V8 = vec8<T>;
  using V4 = vec4<T>;
  using TL = SwizzledTile<D>;
  constexpr int BM = NW * 32;
  constexpr int KS = D / 16;
  constexpr int NKB = BN / 32;
  constexpr int DB = D / 32;
  constexpr int CPR = TL::CPR;
  constexpr int PART = BN * CPR * 8;
  constexpr int IPT = BN * CPR / (NW * 64);
  static_assert(BN * CPR % (NW * 64) == 0, "tile must split evenly over the waves");
  // PIPE (batched, head_dim 128): the key-tile loop is the software-pipelined asm block
  // of fal_dq_pipe.inc at one wave per SIMD, with a ring of 4 K/V tiles
  static_assert(!PIPE || (D == 128 && NW == 4 && BN == 64), "the pipelined loop is written for this shape");

  __shared__ __attribute__((aligned(1024))) T smem[(PIPE ? 4 : 2) * 2 * PART];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int l32 = lane & 31;
  const int hh = lane >> 5;

  int b, hq, qt_a, qt_b = -1, q_off, k_off, nq, nk;
  if (p.cu_q) {
    // 1-D grid: (work item, KV head) groups dealt round-robin to the 8 XCDs in list
    // order, the query heads of a group back to back on one XCD (they read the same
    // K/V); the grid is padded to a multiple of 8 groups
    const int g = p.Hq / p.Hkv;
    const int k8 = blockIdx.x >> 3;
    const int grp = (k8 / g) * 8 + (blockIdx.x & 7);
    const int item = grp / p.Hkv;
    if (item >= p.n_qitems) return;
    const int2 wk = p.qwork[item];
    if (wk.x < 0) return;
    hq = (grp % p.Hkv) * g + k8 % g;
    b = 0;
    qt_a = wk.y;
    seg_bounds(p.cu_q, wk.x, p.total_q, q_off, nq);
    seg_bounds(p.cu_k, wk.x, p.total_k, k_off, nk);
  } else {
    // heads of one KV head and the query tiles of a head are dealt to one XCD together
    const int total = gridDim.x;
    int id = blockIdx.x;
    if ((total & 7) == 0) id = (id & 7) * (total >> 3) + (id >> 3);
    // causal: a workgroup takes query tiles t and nqt-1-t, so all do equal work
    const int nqt = cdiv(p.Nq, BM);
    const int nitems = (CAUSAL && FAL_BWD_DQ_PAIR) ? (nqt + 1) / 2 : nqt;
    const int g = p.Hq / p.Hkv;
    const int hg = id % g;
    int rest = id / g;
    const int t = rest % nitems;
    rest /= nitems;
    qt_a = CAUSAL ? (nqt - 1 - t) : t;
    if (CAUSAL && FAL_BWD_DQ_PAIR && t != nqt - 1 - t) qt_b = t;
    b = rest / p.Hkv;
    hq = (rest % p.Hkv) * g + hg;
    q_off = 0;
    k_off = 0;
    nq = p.Nq;
    nk = p.Nk;
  }
  const int hkv = hq / (p.Hq / p.Hkv);
  for (int pass = 0; pass < 2; ++pass) {
  const int qt = pass == 0 ? qt_a : qt_b;
  if (qt < 0) break;
  if (pass) __syncthreads();   // the previous tile's LDS readers are done
  const int m0 = qt * BM;
  if (m0 >= nq) continue;

  const T* qbase = (const T*)p.q + (int64_t)b * p.q_sb + (int64_t)hq * p.q_sh + (int64_t)q_off * p.q_ss;
  const T* dobase = (const T*)p.dout + (int64_t)b * p.do_sb + (int64_t)hq * p.do_sh + (int64_t)q_off * p.do_ss;
  const T* kbase = (const T*)p.k + (int64_t)b * p.k_sb + (int64_t)hkv * p.k_sh + (int64_t)k_off * p.k_ss;
  const T* vbase = (const T*)p.v + (int64_t)b * p.v_sb + (int64_t)hkv * p.v_sh + (int64_t)k_off * p.v_ss;
  const int64_t lrow = (int64_t)b * p.l_sb + (int64_t)hq * p.l_sh + (int64_t)q_off * p.l_ss;

  // Q and dO slices of this wave (B operands: n = query row, k = head dim), the row's
  // log-sum-exp (log2 domain) and D = rowsum(dO * O).  The two lanes of a row hold one
  // half of the head dim each.  D is also stored for the dK/dV kernel, which runs after
  // this one.
  const int row = m0 + w * 32 + l32;
  V8 qreg[KS], doreg[KS];
  float lrow2 = INFINITY, dpart = 0.f;
  if (row < nq) {
    const T* orow = (const T*)p.o + (int64_t)b * p.o_sb + (int64_t)hq * p.o_sh + (int64_t)(q_off + row) * p.o_ss;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      qreg[t] = ld8(qbase + (int64_t)row * p.q_ss + t * 16 + hh * 8);
      doreg[t] = ld8(dobase + (int64_t)row * p.do_ss + t * 16 + hh * 8);
      const V8 ov = ld8(orow + t * 16 + hh * 8);
      dpart = dot8(doreg[t], ov, dpart);
    }
    const float L = p.lse[lrow + (int64_t)row * p.l_ss];
    lrow2 = (L == -INFINITY) ? INFINITY : L * kLog2e;
  } else {
#pragma unroll
    for (int t = 0; t < KS; ++t) qreg[t] = doreg[t] = zero8<T>();
  }
  const float drow = pair_sum(dpart);
  if (hh == 0 && row < nq) p.delta[lrow + (int64_t)row * p.l_ss] = drow;
  const float c = p.scale_log2;
  if (p.lsd && hh == 0) {
    // tile-major copy for bwd_kv_pipe_kernel, 64 rows per tile: -L*log2(e)/c, then -D.
    // Rows past the end (up to the tile boundary) and rows without keys get the value
    // whose exponent c * x is -inf, and -D = 0.
    const int nt64 = cdiv(nq, kPipeBM);
    if (row < nt64 * kPipeBM) {
      float* t = p.lsd + (((int64_t)b * p.Hq + hq) * nt64 + row / kPipeBM) * 2 * kPipeBM + row % kPipeBM;
      const bool live = row < nq && lrow2 != INFINITY;
      t[0] = live ? -lrow2 / c : (c > 0.f ? -INFINITY : INFINITY);
      t[kPipeBM] = row < nq ? -drow : 0.f;
    }
  }

  const int kend = CAUSAL ? min(nk, m0 + BM) : nk;
  const int ntiles = cdiv(kend, BN);
  const int nfull = CAUSAL ? min(nk / BN, (m0 + 1) / BN) : nk / BN;

  const int ws = __builtin_amdgcn_readfirstlane(w);
  int kvo[IPT], vvo[IPT];
#pragma unroll
  for (int i = 0; i < IPT; ++i) {
    const int I = i * NW + ws;
    const int pch = I * 64 + lane;
    const int r = pch / CPR;
    const int cc = TL::logical_chunk(r, pch % CPR);
    kvo[i] = (int)(r * p.k_ss + cc * 8) * 2;   // from the tile's first row
    vvo[i] = (int)(r * p.v_ss + cc * 8) * 2;
  }
  int kaddr[KS];   // fragment (row l32, chunk 2t+hh) of 32-key block 0
#pragma unroll
  for (int t = 0; t < KS; ++t) kaddr[t] = TL::offset(l32, 2 * t + hh);
  int taddr[2][DB];   // transposed reads: rows hf*8 + hh*4 + i/4 of each 16-key step
  {
    const int i = lane & 15;
    const int rl = hh * 4 + (i >> 2);
    const int cl = 2 * ((lane >> 4) & 1) + ((lane >> 1) & 1);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int db = 0; db < DB; ++db) taddr[hf][db] = TL::offset(hf * 8 + rl, db * 4 + cl) + 4 * (lane & 1);
  }

  if constexpr (PIPE) {
    // The whole key-tile loop: dQ^T += K^T dS^T of tile j-1, the gradient of tile j and
    // S^T, dP^T of tile j+1 overlap inside the wave; the masking of the diagonal and
    // last tiles is done inside.  dQ^T comes back through this wave's LDS blocks.
    typedef __attribute__((address_space(3))) T lds_t;
    const uint32_t lds0 = (uint32_t)(uintptr_t)((lds_t*)smem);
    uint32_t p_ka[KS], p_ta[2][DB];
#pragma unroll
    for (int t = 0; t < KS; ++t) p_ka[t] = lds0 + 2 * kaddr[t];
#pragma unroll
    for (int hf = 0; hf < 2; ++hf)
#pragma unroll
      for (int db = 0; db < DB; ++db) p_ta[hf][db] = lds0 + 2 * taddr[hf][db];
    const uint32_t p_lbase = __builtin_amdgcn_readfirstlane(lds0 + ws * 64 * 16);
    const uint32_t p_olds = lds0 + ws * kDqOWave + lane * 16;
    const int p_row = CAUSAL ? row : 0x3fffffff;
    const int p_hh4 = hh * 4;
    const float p_nl = -lrow2, p_dl = drow;
    const float p_c = c, p_negc = c > 0.f ? -INFINITY : INFINITY;   // c * negc = -inf
    const int64_t rows_left = max((int64_t)nk, (int64_t)0);
    const uint64_t ka0 = (uint64_t)(uintptr_t)kbase, va0 = (uint64_t)(uintptr_t)vbase;
    const uint32_t pk_rs[4] = {(uint32_t)ka0, (uint32_t)(ka0 >> 32) & 0xffffu,
                               (uint32_t)min(rows_left * p.k_ss * 2, (int64_t)0x7fffffff), 0x00020000u};
    const uint32_t pv_rs[4] = {(uint32_t)va0, (uint32_t)(va0 >> 32) & 0xffffu,
                               (uint32_t)min(rows_left * p.v_ss * 2, (int64_t)0x7fffffff), 0x00020000u};
    const uint32_t p_ktb = (uint32_t)(BN * p.k_ss * 2), p_vtb = (uint32_t)(BN * p.v_ss * 2);
    const uint32_t p_krb = (uint32_t)(p.k_ss * 2), p_vrb = (uint32_t)(p.v_ss * 2);
    const int p_rows = (int)min(rows_left, (int64_t)0x7fffffff);
    // tiles of this wave: [0, jl]; causal waves stop at their diagonal tile, waves whose
    // rows are all past the end have none
    const int wrow0 = m0 + ws * 32;
    int jl = CAUSAL ? min(ntiles - 1, (wrow0 + 31) / BN) : ntiles - 1;
    if (wrow0 >= nq) jl = -1;
    const int p_jl = __builtin_amdgcn_readfirstlane(jl);
    const int p_jend = ntiles, p_nk = nk;
    const int p_wrow = CAUSAL ? wrow0 : 0x3fffffff;
    if (ntiles > 0) {
      if constexpr (std::is_same<T, half_t>::value)
        asm volatile(FAL_DQP_ASM_F16 : FAL_DQP_OUTS : FAL_DQP_INS : FAL_DQP_CLOBBERS);
      else
        asm volatile(FAL_DQP_ASM_BF16 : FAL_DQP_OUTS : FAL_DQP_INS : FAL_DQP_CLOBBERS);
    }
    {
      // dQ^T block g = db*4 + g4 of lane (hh, l32) holds columns 8g + hh*4 .. +3 of row
      // m0 + ws*32 + l32 at ws*kDqOWave + lane*16 + g*kDqOStr; written back row-wise,
      // each 16-byte store instruction covering 4 whole rows
      const char* wb = (const char*)smem + ws * kDqOWave;
      const int cch = lane & 15;
      // a buffer resource over this wave's rows inside the sequence: stores past the end
      // are dropped (no branch, no 64-bit address per store)
      const int wr0 = m0 + ws * 32;
      const __amdgpu_buffer_rsrc_t dqrs =
          make_rsrc((T*)p.dq + (int64_t)b * p.dq_sb + (int64_t)hq * p.dq_sh + (int64_t)(q_off + wr0) * p.dq_ss,
                    (uint32_t)((int64_t)max(min(nq - wr0, 32), 0) * p.dq_ss * 2));
      const int dvo = ((lane >> 4) * (int)p.dq_ss + cch * 8) * 2;
      f32x4 a0[8], a1[8];
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        const int r = jj * 4 + (lane >> 4);
        a0[jj] = a1[jj] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (ntiles > 0) {
          a0[jj] = *reinterpret_cast<const f32x4*>(wb + r * 16 + cch * kDqOStr);
          a1[jj] = *reinterpret_cast<const f32x4*>(wb + (32 + r) * 16 + cch * kDqOStr);
        }
      }
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) {
        V8 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          h[e] = (T)(a0[jj][e] * p.scale);
          h[4 + e] = (T)(a1[jj][e] * p.scale);
        }
        buffer_store16(dqrs, dvo + jj * 4 * (int)p.dq_ss * 2, __builtin_bit_cast(u32x4, h));
      }
    }
    continue;
  }

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

  f32x16 dqacc[DB];
#pragma unroll
  for (int i = 0; i < DB; ++i) dqacc[i] = zero_f16();

  auto tile_body = [&](auto masked, int j, int buf) {
    constexpr bool MASK = decltype(masked)::value;
    const int n0 = j * BN;
    const T* ks = smem + buf * 2 * PART;
    const T* vs = ks + PART;
    // S^T = K Q^T and dP^T = V dO^T; fragments read one k-step ahead of their MFMAs
    f32x16 sacc[NKB], pacc[NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) sacc[kb] = pacc[kb] = zero_f16();
    V8 kf[2][NKB], vf[2][NKB];
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      kf[0][kb] = ld8(ks + kaddr[0] + kb * 32 * CPR * 8);
      vf[0][kb] = ld8(vs + kaddr[0] + kb * 32 * CPR * 8);
    }
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      if (t + 1 < KS) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
          kf[(t + 1) & 1][kb] = ld8(ks + kaddr[t + 1] + kb * 32 * CPR * 8);
          vf[(t + 1) & 1][kb] = ld8(vs + kaddr[t + 1] + kb * 32 * CPR * 8);
        }
        __builtin_amdgcn_sched_group_barrier(0x100, 2 * NKB, 0);
      }
#pragma unroll
      for (int kb = 0; kb < NKB; ++kb) {
        sacc[kb] = mfma32(kf[t & 1][kb], qreg[t], sacc[kb]);
        pacc[kb] = mfma32(vf[t & 1][kb], doreg[t], pacc[kb]);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * NKB, 0);
    }
    // P^T and dS^T; element i: key n0 + kb*32 + (i/4)*8 + hh*4 + i%4, query `row`
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float pv = fast_exp2(fmaf(sacc[kb][i], c, -lrow2));
        if (MASK) {
          const int key = n0 + kb * 32 + (i >> 2) * 8 + hh * 4 + (i & 3);
          if (key >= nk || (CAUSAL && key > row)) pv = 0.f;
        }
        pacc[kb][i] = pv * (pacc[kb][i] - drow);
      }
    // dQ^T += K^T dS^T
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        const V8 sb = cvt8t<T>(pacc[kb], t2);
        const int kofs = (kb * 2 + t2) * 16 * CPR * 8;
#pragma unroll
        for (int db = 0; db < DB; ++db) {
          const V4 lo = lds_tr(ks + taddr[0][db] + kofs);
          const V4 hi = lds_tr(ks + taddr[1][db] + kofs);
          dqacc[db] = mfma32(join8(lo, hi), sb, dqacc[db]);
        }
      }
  };
  auto step = [&](auto masked, int j, int buf) {
    wait_vmcnt0();
    __syncthreads();
    if (j + 1 < ntiles) load_tile(j + 1, buf ^ 1);
    tile_body(masked, j, buf);
  };

  if (ntiles > 0) load_tile(0, 0);
  int j = 0;
  for (; j + 1 < nfull; j += 2) {
    step(std::false_type{}, j, 0);
    step(std::false_type{}, j + 1, 1);
  }
  if (j < nfull) {
    step(std::false_type{}, j, 0);
    ++j;
  }
  const int wrow_hi = m0 + w * 32 + 31;
  for (; j < ntiles; ++j) {
    wait_vmcnt0();
    __syncthreads();
    if (j + 1 < ntiles) load_tile(j + 1, (j + 1) & 1);
    if (!CAUSAL || j * BN <= wrow_hi) tile_body(std::true_type{}, j, j & 1);
  }

  if (row < nq) {
    T* dqrow = (T*)p.dq + (int64_t)b * p.dq_sb + (int64_t)hq * p.dq_sh + (int64_t)(q_off + row) * p.dq_ss;
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
      for (int g4 = 0; g4 < 4; ++g4) {
        V4 h;
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = (T)(dqacc[db][g4 * 4 + e] * p.scale);
        *reinterpret_cast<V4*>(dqrow + db * 32 + g4 * 8 + hh * 4) = h;
      }
  }
  }
}

// --------------------------------------------------------------------------
// Launchers
// --------------------------------------------------------------------------
constexpr int kBwdNW = 4;

// head dims on the split path (dQ kernel + dK/dV kernel); 256 keeps the atomic kernel,
// whose dK/dV accumulators would not fit the split kernel's registers
constexpr bool split_d(int d) { return d == 32 || d == 64 || d == 96 || d == 128; }
// head dims whose KV-outer kernel also forms dQ = dS K (fp32 atomics into an accumulator,
// five products instead of the split form's seven)
#ifndef FAL_BWD_FUSED
#define FAL_BWD_FUSED 0
#endif
constexpr bool fused_d(int d) { return FAL_BWD_FUSED && (d == 64 || d == 128); }

int bwd_block_n(int d) {
  return split_d(d) ? FAL_BWD2_NW * 16 : kBwdNW * 32;
}

bool bwd_pipe(int d) { return FAL_BWD_PIPE && d == 128; }

template <class T, int D>
static hipError_t launch_bwd_t(const BwdParams& p, int causal, dim3 grid, hipStream_t st) {
  if constexpr (D == 128) {
    if (!p.cu_q && p.lsd) {
      const int nkt = cdiv(p.Nk, kPipeBN);
      grid.x = (unsigned)((causal ? (nkt + 1) / 2 : nkt) * p.B * p.Hkv);
      if (causal)
        hipLaunchKernelGGL((bwd_kv_pipe_kernel<T, true>), grid, dim3(256), 0, st, p);
      else
        hipLaunchKernelGGL((bwd_kv_pipe_kernel<T, false>), grid, dim3(256), 0, st, p);
      return hipGetLastError();
    }
  }
  if constexpr (split_d(D)) {
    constexpr bool kFused = fused_d(D);
    // batched causal: one workgroup per pair of key tiles
    if (!p.cu_q && causal) grid.x = (unsigned)((p.n_ktiles + 1) / 2) * p.B * p.Hkv;
    if (causal)
      hipLaunchKernelGGL((bwd2_kernel<T, D, true, kFused>), grid, dim3(FAL_BWD2_NW * 64), 0, st, p);
    else
      hipLaunchKernelGGL((bwd2_kernel<T, D, false, kFused>), grid, dim3(FAL_BWD2_NW * 64), 0, st, p);
  } else {
    if (causal)
      hipLaunchKernelGGL((bwd_kernel<T, D, kBwdNW, 32, true>), grid, dim3(kBwdNW * 64), 0, st, p);
    else
      hipLaunchKernelGGL((bwd_kernel<T, D, kBwdNW, 32, false>), grid, dim3(kBwdNW * 64), 0, st, p);
  }
  return hipGetLastError();
}
template <int D>
static hipError_t launch_bwd_d(const BwdParams& p, int causal, dim3 grid, hipStream_t st) {
  return p.bf16 ? launch_bwd_t<bf16_t, D>(p, causal, grid, st) : launch_bwd_t<half_t, D>(p, causal, grid, st);
}

#ifndef FAL_BWD_DQ_BN
#define FAL_BWD_DQ_BN 64
#endif
constexpr int kDqNW = 4;

bool bwd_split_dq(int d) { return split_d(d) && !fused_d(d); }
int bwd_dq_block_m(int d) {
  (void)d;
  return kDqNW * 32;
}

template <class T, int D>
static hipError_t launch_bwd_dq_t(const BwdParams& p, int causal, dim3 grid, hipStream_t st) {
  if (!p.cu_q && causal && FAL_BWD_DQ_PAIR)
    grid.x = (unsigned)((cdiv(p.Nq, kDqNW * 32) + 1) / 2) * p.B * p.Hq;
  if constexpr (D == 128) {
    if (!p.cu_q && FAL_BWD_DQ_PIPE) {
      if (causal)
        hipLaunchKernelGGL((bwd_dq_kernel<T, D, kDqNW, 64, true, true>), grid, dim3(kDqNW * 64), 0, st, p);
      else
        hipLaunchKernelGGL((bwd_dq_kernel<T, D, kDqNW, 64, false, true>), grid, dim3(kDqNW * 64), 0, st, p);
      return hipGetLastError();
    }
  }
  if (causal)
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, kDqNW, FAL_BWD_DQ_BN, true>), grid, dim3(kDqNW * 64), 0, st, p);
  else
    hipLaunchKernelGGL((bwd_dq_kernel<T, D, kDqNW, FAL_BWD_DQ_BN, false>), grid, dim3(kDqNW * 64), 0, st, p);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_bwd_dq_d(const BwdParams& p, int causal, dim3 grid, hipStream_t st) {
  return p.bf16 ? launch_bwd_dq_t<bf16_t, D>(p, causal, grid, st) : launch_bwd_dq_t<half_t, D>(p, causal, grid, st);
}

hipError_t launch_bwd_dq(const BwdParams& p, int d, int causal, dim3 grid, hipStream_t st) {
  switch (d) {
    case 32: return launch_bwd_dq_d<32>(p, causal, grid, st);
    case 64: return launch_bwd_dq_d<64>(p, causal, grid, st);
    case 96: return launch_bwd_dq_d<96>(p, causal, grid, st);
    case 128: return launch_bwd_dq_d<128>(p, causal, grid, st);
    default: return hipErrorInvalidValue;
  }
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

template <class T, int D, bool PRE>
static hipError_t launch_rowwise_t(const BwdParams& p, int batched, hipStream_t st) {
  const int rows = batched ? p.B * p.Hq * p.Nq : p.total_q * p.Hq;
  if (rows == 0) return hipSuccess;
  constexpr int RPB = 256 / row_group<D>();
  dim3 grid(cdiv(rows, RPB));
  if (PRE)
    hipLaunchKernelGGL((bwd_pre_kernel<T, D>), grid, dim3(256), 0, st, p, rows, batched);
  else
    hipLaunchKernelGGL((bwd_post_kernel<T, D>), grid, dim3(256), 0, st, p, rows, batched);
  return hipGetLastError();
}

template <int D, bool PRE>
static hipError_t launch_rowwise(const BwdParams& p, int batched, hipStream_t st) {
  return p.bf16 ? launch_rowwise_t<bf16_t, D, PRE>(p, batched, st) : launch_rowwise_t<half_t, D, PRE>(p, batched, st);
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

// C-ABI entry points of libfal_hip.so (declared in include/fal_api.h).
//
// This layer replaces the reference's pybind11 binding (csrc/flash_attn_legacy.cpp):
// it validates shapes, strides and alignment, lays out the caller-provided
// workspace, fills the kernel parameter blocks and enqueues the kernels on the
// caller's stream.  It never allocates device memory and never synchronises.
#include <atomic>
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "fal_kernels.h"
#include "../../include/fal_api.h"

using namespace fal;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() {
  g_err.clear();
  return FAL_OK;
}

bool head_dim_ok(int64_t d) { return d == 32 || d == 64 || d == 96 || d == 128 || d == 256; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// A strided operand: 16-byte aligned base and every used stride a multiple of 8
// elements, so each 8-element row chunk is one aligned 16-byte access.
int check_operand(const char* name, const void* p, const int64_t* st, bool use_batch) {
  if (!p) return fail(FAL_ERR_INVALID, "%s: null pointer", name);
  if (!st) return fail(FAL_ERR_INVALID, "%s: null strides", name);
  if (!aligned16(p)) return fail(FAL_ERR_INVALID, "%s: base pointer must be 16-byte aligned", name);
  for (int i = use_batch ? 0 : 1; i < 3; ++i)
    if (st[i] % 8 != 0 || st[i] < 0)
      return fail(FAL_ERR_INVALID, "%s: stride[%d]=%lld must be a non-negative multiple of 8", name, i,
                  (long long)st[i]);
  // kernels address a tile of up to 256 rows with 32-bit byte offsets
  if (st[2] >= (int64_t(1) << 22))
    return fail(FAL_ERR_UNSUPPORTED, "%s: sequence stride %lld elements is too large (limit 4194304)", name,
                (long long)st[2]);
  return FAL_OK;
}

int launch_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(FAL_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// softmax_scale * log2(e) with its magnitude kept away from 0, so masked scores
// (+-inf) never meet a zero factor.
float signed_scale_log2(float scale) {
  const float a = scale * kLog2e;
  if (std::fabs(a) >= 1e-30f) return a;
  return scale < 0.f ? -1e-30f : 1e-30f;
}

float scale_log2(float scale) {
  // |scale| * log2(e); clamped away from 0 so masked scores (-inf) stay -inf.
  const float a = std::fabs(scale) * kLog2e;
  return a < 1e-30f ? 1e-30f : a;
}

bool dims_ok(int64_t x) { return x >= 0 && x <= 0x7fffffff; }

}  // namespace

extern "C" {

const char* fal_last_error(void) { return g_err.c_str(); }

const char* fal_version(void) { return "0.5.0+gfx950"; }

int fal_device_supported(int device) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
size_t fal_fwd_workspace_size(int64_t batch, int64_t heads_q, int64_t seqlen_q, int64_t seqlen_k, int64_t head_dim,
                              int is_causal) {
  if (!head_dim_ok(head_dim) || batch <= 0 || heads_q <= 0 || !dims_ok(seqlen_q) || !dims_ok(seqlen_k)) return 0;
  int kchunk, nsplit;
  return fwd_split_plan(batch, heads_q, seqlen_q, seqlen_k, (int)head_dim, is_causal != 0, &kchunk, &nsplit);
}

#ifndef FAL_FWD_PERSIST
#define FAL_FWD_PERSIST 1
#endif
// Compute units of the current device (cached per device; 0 if the query fails).
// Entries are atomics: concurrent first calls on one device may both query it and store
// the same value.
static int device_cu_count() {
  static std::atomic<int> cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return 0;
  if (dev < 64) {
    const int c = cached[dev].load(std::memory_order_relaxed);
    if (c > 0) return c;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
  if (dev < 64) cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

static int fal_fwd_impl(const void* q, const void* k, const void* v, void* o, float* lse, int64_t batch,
            int64_t heads_q, int64_t heads_kv, int64_t seqlen_q, int64_t seqlen_k, int64_t head_dim,
            const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
            const int64_t* o_strides, float softmax_scale, int is_causal, void* workspace, size_t workspace_bytes,
            void* stream, int bf16) {
  if (!head_dim_ok(head_dim))
    return fail(FAL_ERR_UNSUPPORTED, "head_dim must be 32, 64, 96, 128, or 256, got %lld", (long long)head_dim);
  if (batch < 0 || heads_q <= 0 || heads_kv <= 0 || !dims_ok(seqlen_q) || !dims_ok(seqlen_k))
    return fail(FAL_ERR_INVALID, "invalid sizes");
  if (heads_q % heads_kv != 0)
    return fail(FAL_ERR_INVALID, "num_heads_q (%lld) must be divisible by num_heads_kv (%lld)",
                (long long)heads_q, (long long)heads_kv);
  int rc;
  if ((rc = check_operand("q", q, q_strides, true)) || (rc = check_operand("k", k, k_strides, true)) ||
      (rc = check_operand("v", v, v_strides, true)) || (rc = check_operand("o", o, o_strides, true)))
    return rc;
  if (!lse) return fail(FAL_ERR_INVALID, "lse: null pointer");
  if (batch == 0 || seqlen_q == 0) return ok();

  FwdParams p{};
  p.bf16 = bf16;
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.lse = lse;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.l_sb = heads_q * seqlen_q; p.l_sh = seqlen_q; p.l_ss = 1;
  p.B = (int)batch; p.Hq = (int)heads_q; p.Hkv = (int)heads_kv;
  p.Nq = (int)seqlen_q; p.Nk = (int)seqlen_k;
  p.scale_log2 = signed_scale_log2(softmax_scale);
  const int bm = fwd_block_m((int)head_dim);
  p.n_qtiles = cdiv((int)seqlen_q, bm);
  // small grids split the key range (partials in the workspace, merged by a second kernel)
  const size_t need = fwd_split_plan(batch, heads_q, seqlen_q, seqlen_k, (int)head_dim, is_causal != 0, &p.kchunk,
                                     &p.nsplit);
  if (need && (!workspace || workspace_bytes < need))
    return fail(FAL_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
  if (p.kchunk) {
    p.part_o = static_cast<float*>(workspace);
    p.part_ml = p.part_o + (size_t)batch * heads_q * p.nsplit * seqlen_q * head_dim;
  }
  int64_t nblocks = (int64_t)p.n_qtiles * batch * heads_q * p.nsplit;
  if (!p.kchunk && fwd_gqa4_ok((int)head_dim, heads_q, heads_kv)) {
    p.gqa4 = 1;
    p.n_qtiles = cdiv((int)seqlen_q, 64);
    nblocks = (int64_t)p.n_qtiles * batch * (heads_q / 4);
  }
  // pipelined kernel with at least two items per CU: one persistent workgroup per CU
  // walks pairs of query tiles
  if (!p.kchunk && fwd_pipe_ok((int)head_dim)) {
    const int ncu = device_cu_count();
    if (FAL_FWD_PERSIST && ncu > 0 && nblocks >= 2 * (int64_t)ncu) {
      p.persist = 1;
      const int64_t pairs = (int64_t)(p.n_qtiles + 1) / 2 * batch * (heads_q / (p.gqa4 ? 4 : 1));
      nblocks = std::min<int64_t>(pairs, ncu);
    }
  }
  if (nblocks > 0x7fffffff) return fail(FAL_ERR_INVALID, "problem too large for one launch");
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipError_t e = launch_fwd(p, (int)head_dim, is_causal != 0, dim3((unsigned)nblocks), st);
  if (e == hipSuccess && p.kchunk) e = launch_fwd_combine(p, (int)head_dim, is_causal != 0, st);
  return launch_status(e, "fal_fwd");
}
int fal_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t batch,
            int64_t heads_q, int64_t heads_kv, int64_t seqlen_q, int64_t seqlen_k, int64_t head_dim,
            const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
            const int64_t* o_strides, float softmax_scale, int is_causal, void* workspace,
            size_t workspace_bytes, void* stream) {
  return fal_fwd_impl(q, k, v, o, lse, batch, heads_q, heads_kv, seqlen_q, seqlen_k, head_dim, q_strides,
                      k_strides, v_strides, o_strides, softmax_scale, is_causal, workspace, workspace_bytes,
                      stream, 0);
}
int fal_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse, int64_t batch,
            int64_t heads_q, int64_t heads_kv, int64_t seqlen_q, int64_t seqlen_k, int64_t head_dim,
            const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
            const int64_t* o_strides, float softmax_scale, int is_causal, void* workspace,
            size_t workspace_bytes, void* stream) {
  return fal_fwd_impl(q, k, v, o, lse, batch, heads_q, heads_kv, seqlen_q, seqlen_k, head_dim, q_strides,
                      k_strides, v_strides, o_strides, softmax_scale, is_causal, workspace, workspace_bytes,
                      stream, 1);
}

#ifndef FAL_FWD_VARLEN_GQA4
#define FAL_FWD_VARLEN_GQA4 1   // varlen head_dim 128, Hq/Hkv a multiple of 4: the four-heads pipelined layout
#endif
size_t fal_fwd_varlen_workspace_size(int64_t num_seqs, int64_t total_q, int64_t max_seqlen_q, int64_t head_dim) {
  (void)max_seqlen_q;
  // small problems: the kernel derives its work items itself
  if (num_seqs <= kVarlenSmallSeqs && total_q <= kVarlenSmallTokens) return 0;
  // (head_dim 128 may run 64-row items: the four-heads layout, which the heads decide)
  const int bm = head_dim == 128 && FAL_FWD_VARLEN_GQA4 ? 64 : fwd_block_m_varlen(head_dim_ok(head_dim) ? (int)head_dim : 128);
  const int64_t cap = (total_q + bm - 1) / bm + num_seqs;
  return align256((size_t)cap * sizeof(int2));
}

#ifndef FAL_BWD_VARLEN_ORDER
#define FAL_BWD_VARLEN_ORDER 3   // KV-outer list: 3 grouped by sequence, 0 by tile index over all sequences
#endif
#ifndef FAL_BWD_DQ_VARLEN_ORDER
#define FAL_BWD_DQ_VARLEN_ORDER 2
#endif
#ifndef FAL_FWD_VARLEN_PAIR
#define FAL_FWD_VARLEN_PAIR 1   // four-heads varlen with a work list: pairs of query tiles per workgroup
#endif
#ifndef FAL_FWD_VARLEN_ORDER
#define FAL_FWD_VARLEN_ORDER 2   // 2: grouped by sequence; 1: heaviest tile index first over all sequences
#endif
static int fal_fwd_varlen_impl(const void* q, const void* k, const void* v, void* o, float* lse,
                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t num_seqs, int64_t total_q,
                   int64_t total_k, int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t max_seqlen_q,
                   int64_t max_seqlen_k, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* o_strides, float softmax_scale, int is_causal,
                   void* workspace, size_t workspace_bytes, void* stream, int bf16) {
  (void)max_seqlen_k;
  if (!head_dim_ok(head_dim))
    return fail(FAL_ERR_UNSUPPORTED, "head_dim must be 32, 64, 96, 128, or 256, got %lld", (long long)head_dim);
  if (num_seqs < 0 || heads_q <= 0 || heads_kv <= 0 || !dims_ok(total_q) || !dims_ok(total_k) ||
      max_seqlen_q < 0)
    return fail(FAL_ERR_INVALID, "invalid sizes");
  if (heads_q % heads_kv != 0)
    return fail(FAL_ERR_INVALID, "H_q (%lld) must be divisible by H_kv (%lld)", (long long)heads_q,
                (long long)heads_kv);
  if (!cu_seqlens_q || !cu_seqlens_k) return fail(FAL_ERR_INVALID, "cu_seqlens: null pointer");
  int rc;
  if ((rc = check_operand("q", q, q_strides, false)) || (rc = check_operand("k", k, k_strides, false)) ||
      (rc = check_operand("v", v, v_strides, false)) || (rc = check_operand("o", o, o_strides, false)))
    return rc;
  if (!lse) return fail(FAL_ERR_INVALID, "lse: null pointer");
  const size_t need = fal_fwd_varlen_workspace_size(num_seqs, total_q, max_seqlen_q, head_dim);
  if (need && (!workspace || workspace_bytes < need))
    return fail(FAL_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
  if (num_seqs == 0 || total_q == 0) return ok();

  // head_dim 128 with Hq/Hkv a multiple of 4: the pipelined kernel's four-heads layout
  // (64 rows of four query heads per workgroup) over the work list
  const bool gqa4 = FAL_FWD_VARLEN_GQA4 && fwd_gqa4_ok((int)head_dim, heads_q, heads_kv);
  const int bm = gqa4 ? 64 : fwd_block_m_varlen((int)head_dim);
  const int cap = (int)((total_q + bm - 1) / bm + num_seqs);
  // with a work list, the four-heads layout takes pairs of query tiles of a sequence
  // (ceil(nt/2) list entries per sequence: at most half the tiles plus one each)
  const bool vpair = gqa4 && FAL_FWD_VARLEN_PAIR && need > 0;
  const int items = vpair ? (int)((total_q + bm - 1) / bm / 2 + num_seqs + 1) : cap;
  hipStream_t st = static_cast<hipStream_t>(stream);
  int2* work = nullptr;
  if (need) {
    // grouped by sequence (see varlen_schedule_kernel): K/V locality in each XCD's L2;
    // smaller batches derive the same order inside the forward kernel
    work = static_cast<int2*>(workspace);
    int nb = cdiv((int)(max_seqlen_q > 0 ? max_seqlen_q : 1), bm);
    nb = nb < 1 ? 1 : (nb > 8192 ? 8192 : nb);
    hipError_t e = launch_varlen_schedule(cu_seqlens_q, (int)num_seqs, (int)total_q, bm, nb,
                                          vpair ? 4 : FAL_FWD_VARLEN_ORDER, work, cap, st);
    if (e != hipSuccess) return launch_status(e, "fal_fwd_varlen schedule");
  }

  FwdParams p{};
  p.bf16 = bf16;
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<half_t*>(o);
  p.lse = lse;
  p.q_sh = q_strides[1]; p.q_ss = q_strides[2];
  p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sh = o_strides[1]; p.o_ss = o_strides[2];
  p.l_sb = 0; p.l_sh = 1; p.l_ss = heads_q;
  p.B = 1; p.Hq = (int)heads_q; p.Hkv = (int)heads_kv;
  p.scale_log2 = signed_scale_log2(softmax_scale);
  p.cu_q = cu_seqlens_q;
  p.total_q = (int)total_q;
  p.total_k = (int)total_k;
  p.cu_k = cu_seqlens_k;
  p.work = work;
  p.num_seqs = (int)num_seqs;
  p.n_qtiles = items;   // an upper bound on the list entries (the list holds `cap` slots)
  const int64_t groups8 = ((int64_t)items * heads_kv + 7) / 8 * 8;
  p.gqa4 = gqa4 ? 1 : 0;
  p.persist = vpair ? 1 : 0;   // each workgroup walks its pair's two items
  const int64_t nblocks = groups8 * (heads_q / heads_kv / (gqa4 ? 4 : 1));
  if (nblocks > 0x7fffffff) return fail(FAL_ERR_INVALID, "problem too large for one launch");
  return launch_status(launch_fwd(p, (int)head_dim, is_causal != 0, dim3((unsigned)nblocks), st),
                       "fal_fwd_varlen");
}
int fal_fwd_varlen(const void* q, const void* k, const void* v, void* o, float* lse,
                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t num_seqs, int64_t total_q,
                   int64_t total_k, int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t max_seqlen_q,
                   int64_t max_seqlen_k, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* o_strides, float softmax_scale, int is_causal,
                   void* workspace, size_t workspace_bytes, void* stream) {
  return fal_fwd_varlen_impl(q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k, num_seqs, total_q, total_k, heads_q,
                             heads_kv, head_dim, max_seqlen_q, max_seqlen_k, q_strides, k_strides, v_strides,
                             o_strides, softmax_scale, is_causal, workspace, workspace_bytes, stream, 0);
}
int fal_fwd_varlen_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t num_seqs, int64_t total_q,
                   int64_t total_k, int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t max_seqlen_q,
                   int64_t max_seqlen_k, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* o_strides, float softmax_scale, int is_causal,
                   void* workspace, size_t workspace_bytes, void* stream) {
  return fal_fwd_varlen_impl(q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k, num_seqs, total_q, total_k, heads_q,
                             heads_kv, head_dim, max_seqlen_q, max_seqlen_k, q_strides, k_strides, v_strides,
                             o_strides, softmax_scale, is_causal, workspace, workspace_bytes, stream, 1);
}

// ---------------------------------------------------------------------------
// Backward
// ---------------------------------------------------------------------------
// Backward workspace: delta [rows] fp32, plus, for head dims without the query-outer
// dQ kernel, the fp32 dQ accumulator [rows, d] in front of it.
static size_t bwd_acc_bytes(size_t rows, int64_t head_dim) {
  return bwd_split_dq(head_dim_ok(head_dim) ? (int)head_dim : 0) ? 0 : align256(rows * head_dim * sizeof(float));
}

// Batched head_dim 128 also holds the lsd array: per (batch, query head, 64-row tile)
// 64 values of -L*log2(e)/c and 64 of -D.
static size_t bwd_lsd_bytes(int64_t batch, int64_t heads_q, int64_t seqlen_q, int64_t head_dim) {
  if (!head_dim_ok(head_dim) || !bwd_pipe((int)head_dim)) return 0;
  return align256((size_t)batch * heads_q * ((seqlen_q + 63) / 64) * 128 * sizeof(float));
}

size_t fal_bwd_workspace_size(int64_t batch, int64_t heads_q, int64_t seqlen_q, int64_t head_dim) {
  const size_t rows = (size_t)batch * heads_q * seqlen_q;
  return bwd_acc_bytes(rows, head_dim) + align256(rows * sizeof(float)) +
         bwd_lsd_bytes(batch, heads_q, seqlen_q, head_dim);
}

static int fill_bwd_common(BwdParams& p, const void* dout, const void* q, const void* k, const void* v,
                           const void* o, const float* lse, void* dq, void* dk, void* dv,
                           const int64_t* do_s, const int64_t* q_s, const int64_t* k_s, const int64_t* v_s,
                           const int64_t* o_s, const int64_t* dq_s, const int64_t* dk_s, const int64_t* dv_s,
                           bool batched) {
  int rc;
  if ((rc = check_operand("dout", dout, do_s, batched)) || (rc = check_operand("q", q, q_s, batched)) ||
      (rc = check_operand("k", k, k_s, batched)) || (rc = check_operand("v", v, v_s, batched)) ||
      (rc = check_operand("o", o, o_s, batched)) || (rc = check_operand("dq", dq, dq_s, batched)) ||
      (rc = check_operand("dk", dk, dk_s, batched)) || (rc = check_operand("dv", dv, dv_s, batched)))
    return rc;
  if (!lse) return fail(FAL_ERR_INVALID, "lse: null pointer");
  p.dout = static_cast<const half_t*>(dout);
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k);
  p.v = static_cast<const half_t*>(v);
  p.o = static_cast<const half_t*>(o);
  p.lse = lse;
  p.dq = static_cast<half_t*>(dq);
  p.dk = static_cast<half_t*>(dk);
  p.dv = static_cast<half_t*>(dv);
  p.do_sb = batched ? do_s[0] : 0; p.do_sh = do_s[1]; p.do_ss = do_s[2];
  p.q_sb = batched ? q_s[0] : 0; p.q_sh = q_s[1]; p.q_ss = q_s[2];
  p.k_sb = batched ? k_s[0] : 0; p.k_sh = k_s[1]; p.k_ss = k_s[2];
  p.v_sb = batched ? v_s[0] : 0; p.v_sh = v_s[1]; p.v_ss = v_s[2];
  p.o_sb = batched ? o_s[0] : 0; p.o_sh = o_s[1]; p.o_ss = o_s[2];
  p.dq_sb = batched ? dq_s[0] : 0; p.dq_sh = dq_s[1]; p.dq_ss = dq_s[2];
  p.dk_sb = batched ? dk_s[0] : 0; p.dk_sh = dk_s[1]; p.dk_ss = dk_s[2];
  p.dv_sb = batched ? dv_s[0] : 0; p.dv_sh = dv_s[1]; p.dv_ss = dv_s[2];
  return FAL_OK;
}

static int run_bwd(BwdParams& p, int d, int causal, dim3 grid, dim3 dq_grid, bool batched, hipStream_t st) {
  hipError_t e;
  if (bwd_split_dq(d)) {
    // dQ kernel first: it also computes D = rowsum(dO * O), which the dK/dV kernel
    // reads, so no preprocessing launch is needed
    if (dq_grid.x > 0 && dq_grid.y > 0) {
      e = launch_bwd_dq(p, d, causal, dq_grid, st);
      if (e != hipSuccess) return launch_status(e, "bwd dq");
    }
    if (grid.x > 0 && grid.y > 0) return launch_status(launch_bwd(p, d, causal, grid, st), "bwd main");
    return ok();
  }
  e = launch_bwd_pre(p, d, batched ? 1 : 0, st);
  if (e != hipSuccess) return launch_status(e, "bwd preprocess");
  if (grid.x > 0 && grid.y > 0) {
    e = launch_bwd(p, d, causal, grid, st);
    if (e != hipSuccess) return launch_status(e, "bwd main");
  }
  e = launch_bwd_post(p, d, st);
  return launch_status(e, "bwd dq cast");
}

static int fal_bwd_impl(const void* dout, const void* q, const void* k, const void* v, const void* o, const float* lse,
            void* dq, void* dk, void* dv, int64_t batch, int64_t heads_q, int64_t heads_kv, int64_t seqlen_q,
            int64_t seqlen_k, int64_t head_dim, const int64_t* do_strides, const int64_t* q_strides,
            const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
            const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
            float softmax_scale, int is_causal, void* workspace, size_t workspace_bytes, void* stream, int bf16) {
  if (!head_dim_ok(head_dim))
    return fail(FAL_ERR_UNSUPPORTED, "head_dim must be 32, 64, 96, 128, or 256, got %lld", (long long)head_dim);
  if (batch < 0 || heads_q <= 0 || heads_kv <= 0 || !dims_ok(seqlen_q) || !dims_ok(seqlen_k))
    return fail(FAL_ERR_INVALID, "invalid sizes");
  if (heads_q % heads_kv != 0) return fail(FAL_ERR_INVALID, "H_q must be divisible by H_kv for GQA");
  BwdParams p{};
  p.bf16 = bf16;
  int rc = fill_bwd_common(p, dout, q, k, v, o, lse, dq, dk, dv, do_strides, q_strides, k_strides, v_strides,
                           o_strides, dq_strides, dk_strides, dv_strides, true);
  if (rc) return rc;
  const size_t need = fal_bwd_workspace_size(batch, heads_q, seqlen_q, head_dim);
  if (!workspace || workspace_bytes < need)
    return fail(FAL_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
  if (batch == 0 || (seqlen_k == 0 && seqlen_q == 0)) return ok();
  const size_t rows = (size_t)batch * heads_q * seqlen_q;
  const size_t acc = bwd_acc_bytes(rows, head_dim);
  p.dq_acc = acc ? static_cast<float*>(workspace) : nullptr;
  p.delta = reinterpret_cast<float*>(static_cast<char*>(workspace) + acc);
  if (bwd_lsd_bytes(batch, heads_q, seqlen_q, head_dim))
    p.lsd = reinterpret_cast<float*>(static_cast<char*>(workspace) + acc + align256(rows * sizeof(float)));
  p.dqa_sb = heads_q * seqlen_q * head_dim; p.dqa_sh = seqlen_q * head_dim; p.dqa_ss = head_dim;
  p.l_sb = heads_q * seqlen_q; p.l_sh = seqlen_q; p.l_ss = 1;
  p.B = (int)batch; p.Hq = (int)heads_q; p.Hkv = (int)heads_kv;
  p.Nq = (int)seqlen_q; p.Nk = (int)seqlen_k;
  p.scale = softmax_scale;
  p.scale_log2 = signed_scale_log2(softmax_scale);
  const int bn = bwd_block_n((int)head_dim);
  p.n_ktiles = cdiv((int)seqlen_k, bn);
  const int64_t nblocks = (int64_t)p.n_ktiles * batch * heads_kv;
  const int64_t dq_blocks = (int64_t)cdiv((int)seqlen_q, bwd_dq_block_m((int)head_dim)) * batch * heads_q;
  if (nblocks > 0x7fffffff || dq_blocks > 0x7fffffff)
    return fail(FAL_ERR_INVALID, "problem too large for one launch");
  return run_bwd(p, (int)head_dim, is_causal != 0, dim3((unsigned)nblocks), dim3((unsigned)dq_blocks), true,
                 static_cast<hipStream_t>(stream));
}
int fal_bwd(const void* dout, const void* q, const void* k, const void* v, const void* o, const float* lse,
            void* dq, void* dk, void* dv, int64_t batch, int64_t heads_q, int64_t heads_kv, int64_t seqlen_q,
            int64_t seqlen_k, int64_t head_dim, const int64_t* do_strides, const int64_t* q_strides,
            const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
            const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
            float softmax_scale, int is_causal, void* workspace, size_t workspace_bytes, void* stream) {
  return fal_bwd_impl(dout, q, k, v, o, lse, dq, dk, dv, batch, heads_q, heads_kv, seqlen_q, seqlen_k,
                      head_dim, do_strides, q_strides, k_strides, v_strides, o_strides, dq_strides,
                      dk_strides, dv_strides, softmax_scale, is_causal, workspace, workspace_bytes, stream,
                      0);
}
int fal_bwd_bf16(const void* dout, const void* q, const void* k, const void* v, const void* o, const float* lse,
            void* dq, void* dk, void* dv, int64_t batch, int64_t heads_q, int64_t heads_kv, int64_t seqlen_q,
            int64_t seqlen_k, int64_t head_dim, const int64_t* do_strides, const int64_t* q_strides,
            const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
            const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
            float softmax_scale, int is_causal, void* workspace, size_t workspace_bytes, void* stream) {
  return fal_bwd_impl(dout, q, k, v, o, lse, dq, dk, dv, batch, heads_q, heads_kv, seqlen_q, seqlen_k,
                      head_dim, do_strides, q_strides, k_strides, v_strides, o_strides, dq_strides,
                      dk_strides, dv_strides, softmax_scale, is_causal, workspace, workspace_bytes, stream,
                      1);
}

size_t fal_bwd_varlen_workspace_size(int64_t num_seqs, int64_t total_q, int64_t total_k, int64_t heads_q,
                                     int64_t head_dim) {
  const size_t rows = (size_t)total_q * heads_q;
  const int d = head_dim_ok(head_dim) ? (int)head_dim : 128;
  const int bn = bwd_block_n(d);
  const size_t cap = (size_t)((total_k + bn - 1) / bn + num_seqs);
  size_t bytes = bwd_acc_bytes(rows, head_dim) + align256(rows * sizeof(float)) + align256(cap * sizeof(int2));
  if (bwd_split_dq(d)) {
    const int bm = bwd_dq_block_m(d);
    bytes += align256((size_t)((total_q + bm - 1) / bm + num_seqs) * sizeof(int2));
  }
  return bytes;
}

static int fal_bwd_varlen_impl(const void* dout, const void* q, const void* k, const void* v, const void* o, const float* lse,
                   void* dq, void* dk, void* dv, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                   int64_t num_seqs, int64_t total_q, int64_t total_k, int64_t heads_q, int64_t heads_kv,
                   int64_t head_dim, int64_t max_seqlen_q, int64_t max_seqlen_k, const int64_t* do_strides,
                   const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                   const int64_t* o_strides, const int64_t* dq_strides, const int64_t* dk_strides,
                   const int64_t* dv_strides, float softmax_scale, int is_causal, void* workspace,
                   size_t workspace_bytes, void* stream, int bf16) {
  if (!head_dim_ok(head_dim))
    return fail(FAL_ERR_UNSUPPORTED, "head_dim must be 32, 64, 96, 128, or 256, got %lld", (long long)head_dim);
  if (num_seqs < 0 || heads_q <= 0 || heads_kv <= 0 || !dims_ok(total_q) || !dims_ok(total_k) ||
      max_seqlen_k < 0)
    return fail(FAL_ERR_INVALID, "invalid sizes");
  if (heads_q % heads_kv != 0) return fail(FAL_ERR_INVALID, "H_q must be divisible by H_kv for GQA");
  if (!cu_seqlens_q || !cu_seqlens_k) return fail(FAL_ERR_INVALID, "cu_seqlens: null pointer");
  BwdParams p{};
  p.bf16 = bf16;
  int rc = fill_bwd_common(p, dout, q, k, v, o, lse, dq, dk, dv, do_strides, q_strides, k_strides, v_strides,
                           o_strides, dq_strides, dk_strides, dv_strides, false);
  if (rc) return rc;
  const size_t need = fal_bwd_varlen_workspace_size(num_seqs, total_q, total_k, heads_q, head_dim);
  if (!workspace || workspace_bytes < need)
    return fail(FAL_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (total_q == 0 && total_k == 0) return ok();
  const size_t rows = (size_t)total_q * heads_q;
  char* ws = static_cast<char*>(workspace);
  const size_t acc = bwd_acc_bytes(rows, head_dim);
  p.dq_acc = acc ? reinterpret_cast<float*>(ws) : nullptr;
  ws += acc;
  p.delta = reinterpret_cast<float*>(ws);
  ws += align256(rows * sizeof(float));
  int2* work = reinterpret_cast<int2*>(ws);
  p.dqa_sb = 0; p.dqa_sh = head_dim; p.dqa_ss = heads_q * head_dim;
  p.l_sb = 0; p.l_sh = 1; p.l_ss = heads_q;
  p.B = 1; p.Hq = (int)heads_q; p.Hkv = (int)heads_kv;
  p.total_q = (int)total_q;
  p.total_k = (int)total_k;
  p.scale = softmax_scale;
  p.scale_log2 = signed_scale_log2(softmax_scale);
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.work = work;
  const int bn = bwd_block_n((int)head_dim);
  const int cap = (int)((total_k + bn - 1) / bn + num_seqs);
  int nb = cdiv((int)(max_seqlen_k > 0 ? max_seqlen_k : 1), bn);
  nb = nb < 1 ? 1 : (nb > 8192 ? 8192 : nb);
  // Every key row of every segment is covered by exactly one work item, which writes
  // its dK/dV rows (zeros when the segment has no query rows).  The schedule kernel
  // writes zeros to the rows outside all segments (dK/dV here; dQ in the query-tile
  // schedule below, or the d 256 accumulator, zeroed for every row).
  // key tiles grouped by sequence, the tile with the most query rows first
  const ZeroRows zkv{dk, dv, dk_strides[2], dk_strides[1], dv_strides[2], dv_strides[1], (int)heads_kv,
                     (int)head_dim};
  hipError_t e = launch_varlen_schedule(cu_seqlens_k, (int)num_seqs, (int)total_k, bn, nb, FAL_BWD_VARLEN_ORDER,
                                        work, cap, st, &zkv);
  if (e != hipSuccess) return launch_status(e, "fal_bwd_varlen schedule");
  dim3 dq_grid(0, 0);
  if (bwd_split_dq((int)head_dim)) {
    // query tiles for the dQ kernel, grouped by sequence (as the forward's list)
    const int bm = bwd_dq_block_m((int)head_dim);
    const int capq = (int)((total_q + bm - 1) / bm + num_seqs);
    int2* qwork = work + align256((size_t)cap * sizeof(int2)) / sizeof(int2);
    int nbq = cdiv((int)(max_seqlen_q > 0 ? max_seqlen_q : 1), bm);
    nbq = nbq < 1 ? 1 : (nbq > 8192 ? 8192 : nbq);
    const ZeroRows zq{dq, nullptr, dq_strides[2], dq_strides[1], 0, 0, (int)heads_q, (int)head_dim};
    e = launch_varlen_schedule(cu_seqlens_q, (int)num_seqs, (int)total_q, bm, nbq, FAL_BWD_DQ_VARLEN_ORDER, qwork,
                               capq, st, &zq);
    if (e != hipSuccess) return launch_status(e, "fal_bwd_varlen dq schedule");
    p.qwork = qwork;
    p.n_qitems = capq;
    const int64_t groups8 = ((int64_t)capq * heads_kv + 7) / 8 * 8;
    const int64_t nblocks = groups8 * (heads_q / heads_kv);
    if (nblocks > 0x7fffffff) return fail(FAL_ERR_INVALID, "problem too large for one launch");
    dq_grid = dim3((unsigned)nblocks);
  }
  if ((int64_t)cap * heads_kv > 0x7fffffff) return fail(FAL_ERR_INVALID, "problem too large for one launch");
  return run_bwd(p, (int)head_dim, is_causal != 0, dim3((unsigned)(cap * heads_kv)), dq_grid, false, st);
}
int fal_bwd_varlen(const void* dout, const void* q, const void* k, const void* v, const void* o, const float* lse,
                   void* dq, void* dk, void* dv, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                   int64_t num_seqs, int64_t total_q, int64_t total_k, int64_t heads_q, int64_t heads_kv,
                   int64_t head_dim, int64_t max_seqlen_q, int64_t max_seqlen_k, const int64_t* do_strides,
                   const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                   const int64_t* o_strides, const int64_t* dq_strides, const int64_t* dk_strides,
                   const int64_t* dv_strides, float softmax_scale, int is_causal, void* workspace,
                   size_t workspace_bytes, void* stream) {
  return fal_bwd_varlen_impl(dout, q, k, v, o, lse, dq, dk, dv, cu_seqlens_q, cu_seqlens_k, num_seqs, total_q,
                             total_k, heads_q, heads_kv, head_dim, max_seqlen_q, max_seqlen_k, do_strides,
                             q_strides, k_strides, v_strides, o_strides, dq_strides, dk_strides, dv_strides,
                             softmax_scale, is_causal, workspace, workspace_bytes, stream, 0);
}
int fal_bwd_varlen_bf16(const void* dout, const void* q, const void* k, const void* v, const void* o, const float* lse,
                   void* dq, void* dk, void* dv, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                   int64_t num_seqs, int64_t total_q, int64_t total_k, int64_t heads_q, int64_t heads_kv,
                   int64_t head_dim, int64_t max_seqlen_q, int64_t max_seqlen_k, const int64_t* do_strides,
                   const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                   const int64_t* o_strides, const int64_t* dq_strides, const int64_t* dk_strides,
                   const int64_t* dv_strides, float softmax_scale, int is_causal, void* workspace,
                   size_t workspace_bytes, void* stream) {
  return fal_bwd_varlen_impl(dout, q, k, v, o, lse, dq, dk, dv, cu_seqlens_q, cu_seqlens_k, num_seqs, total_q,
                             total_k, heads_q, heads_kv, head_dim, max_seqlen_q, max_seqlen_k, do_strides,
                             q_strides, k_strides, v_strides, o_strides, dq_strides, dk_strides, dv_strides,
                             softmax_scale, is_causal, workspace, workspace_bytes, stream, 1);
}

// ---------------------------------------------------------------------------
// Decode
// ---------------------------------------------------------------------------
size_t fal_decode_workspace_size(int64_t batch, int64_t heads_q, int64_t heads_kv, int64_t max_seqlen_k,
                                 int64_t head_dim) {
  const int d = head_dim_ok(head_dim) ? (int)head_dim : 128;
  const int chunk = decode_chunk(d, (int)batch, (int)(heads_kv > 0 ? heads_kv : 1),
                                 (int)(max_seqlen_k > 0 ? max_seqlen_k : 1));
  const int64_t ms = (max_seqlen_k + chunk - 1) / chunk < 1 ? 1 : (max_seqlen_k + chunk - 1) / chunk;
  const size_t parts = (size_t)batch * heads_q * ms;
  return align256(parts * head_dim * sizeof(float)) + align256(parts * sizeof(float)) +
         align256((size_t)batch * ms * sizeof(int2));
}

static int fal_decode_impl(const void* q, const void* k_cache, const void* v_cache, const int32_t* cache_seqlens,
               const float* mask_bias, int64_t mask_stride, void* o, float* lse, int64_t batch, int64_t heads_q,
               int64_t heads_kv, int64_t head_dim, int64_t max_seqlen_k, const int64_t* q_strides,
               const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
               float softmax_scale, void* workspace, size_t workspace_bytes, void* stream, int bf16) {
  if (!head_dim_ok(head_dim))
    return fail(FAL_ERR_UNSUPPORTED, "head_dim must be 32, 64, 96, 128, or 256, got %lld", (long long)head_dim);
  if (batch < 0 || heads_q <= 0 || heads_kv <= 0 || !dims_ok(max_seqlen_k))
    return fail(FAL_ERR_INVALID, "invalid sizes");
  if (heads_q % heads_kv != 0) return fail(FAL_ERR_INVALID, "H_q must be divisible by H_kv");
  if (heads_q / heads_kv > 32)
    return fail(FAL_ERR_UNSUPPORTED, "decode supports at most 32 query heads per KV head, got %lld",
                (long long)(heads_q / heads_kv));
  if (!cache_seqlens) return fail(FAL_ERR_INVALID, "cache_seqlens: null pointer");
  int rc;
  if ((rc = check_operand("q", q, q_strides, true)) || (rc = check_operand("k_cache", k_cache, k_strides, true)) ||
      (rc = check_operand("v_cache", v_cache, v_strides, true)) || (rc = check_operand("o", o, o_strides, true)))
    return rc;
  const size_t need = fal_decode_workspace_size(batch, heads_q, heads_kv, max_seqlen_k, head_dim);
  if (!workspace || workspace_bytes < need)
    return fail(FAL_ERR_WORKSPACE, "workspace needs %zu bytes, got %zu", need, workspace_bytes);
  if (batch == 0) return ok();
  DecodeParams p{};
  p.bf16 = bf16;
  p.q = static_cast<const half_t*>(q);
  p.k = static_cast<const half_t*>(k_cache);
  p.v = static_cast<const half_t*>(v_cache);
  p.seqlens = cache_seqlens;
  p.bias = mask_bias;
  p.bias_sb = mask_stride;
  p.o = static_cast<half_t*>(o);
  p.lse = lse;
  p.q_sb = q_strides[0]; p.q_sh = q_strides[1];
  p.k_sb = k_strides[0]; p.k_sh = k_strides[1]; p.k_ss = k_strides[2];
  p.v_sb = v_strides[0]; p.v_sh = v_strides[1]; p.v_ss = v_strides[2];
  p.o_sb = o_strides[0]; p.o_sh = o_strides[1];
  p.B = (int)batch; p.Hq = (int)heads_q; p.Hkv = (int)heads_kv;
  p.max_seqlen = (int)max_seqlen_k;
  p.chunk = decode_chunk((int)head_dim, (int)batch, (int)heads_kv, (int)(max_seqlen_k > 0 ? max_seqlen_k : 1));
  p.max_splits = cdiv((int)(max_seqlen_k > 0 ? max_seqlen_k : 1), p.chunk);
  const size_t parts = (size_t)batch * heads_q * p.max_splits;
  p.part_o = static_cast<float*>(workspace);
  p.part_m = reinterpret_cast<float*>(static_cast<char*>(workspace) + align256(parts * head_dim * sizeof(float)));
  p.work = reinterpret_cast<const int2*>(static_cast<char*>(workspace) + align256(parts * head_dim * sizeof(float)) +
                                         align256(parts * sizeof(float)));
  p.scale_log2 = scale_log2(softmax_scale);
  p.negate_q = softmax_scale < 0.f;
  if ((int64_t)batch * p.max_splits * heads_kv * ((heads_q / heads_kv + 15) / 16) > 0x7fffffff)
    return fail(FAL_ERR_INVALID, "batch too large for one launch");
  return launch_status(launch_decode(p, (int)head_dim, static_cast<hipStream_t>(stream)), "fal_decode");
}
int fal_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* cache_seqlens,
               const float* mask_bias, int64_t mask_stride, void* o, float* lse, int64_t batch, int64_t heads_q,
               int64_t heads_kv, int64_t head_dim, int64_t max_seqlen_k, const int64_t* q_strides,
               const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
               float softmax_scale, void* workspace, size_t workspace_bytes, void* stream) {
  return fal_decode_impl(q, k_cache, v_cache, cache_seqlens, mask_bias, mask_stride, o, lse, batch, heads_q,
                         heads_kv, head_dim, max_seqlen_k, q_strides, k_strides, v_strides, o_strides,
                         softmax_scale, workspace, workspace_bytes, stream, 0);
}
int fal_decode_bf16(const void* q, const void* k_cache, const void* v_cache, const int32_t* cache_seqlens,
               const float* mask_bias, int64_t mask_stride, void* o, float* lse, int64_t batch, int64_t heads_q,
               int64_t heads_kv, int64_t head_dim, int64_t max_seqlen_k, const int64_t* q_strides,
               const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
               float softmax_scale, void* workspace, size_t workspace_bytes, void* stream) {
  return fal_decode_impl(q, k_cache, v_cache, cache_seqlens, mask_bias, mask_stride, o, lse, batch, heads_q,
                         heads_kv, head_dim, max_seqlen_k, q_strides, k_strides, v_strides, o_strides,
                         softmax_scale, workspace, workspace_bytes, stream, 1);
}

// ---------------------------------------------------------------------------
// Decode without allocation: the workspace is a fixed device array of this file
// ---------------------------------------------------------------------------
}  // extern "C"

namespace {

// Workspace of fal_decode_noalloc: partial outputs, partial LSEs and the work list of
// one decode call.  Each GPU that runs the entry point holds its own copy until the
// process ends; every call on that GPU shares it.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];   // device address of `scratch` on each device, once resolved

// The device address of this device's `scratch` (the host-side symbol is only a handle).
int scratch_for_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FAL_ERR_LAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(FAL_ERR_UNSUPPORTED, "device index %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(FAL_ERR_LAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FAL_OK;
}

}  // namespace

extern "C" {

int fal_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, const int32_t* cache_seqlens,
                       const float* mask_bias, int64_t mask_stride, void* o, float* lse, int64_t batch,
                       int64_t heads_q, int64_t heads_kv, int64_t head_dim, int64_t max_seqlen_k,
                       const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                       const int64_t* o_strides, float softmax_scale, void* stream) {
  if (!head_dim_ok(head_dim))
    return fail(FAL_ERR_UNSUPPORTED, "head_dim must be 32, 64, 96, 128, or 256, got %lld", (long long)head_dim);
  if (batch < 0 || heads_q <= 0 || heads_kv <= 0 || !dims_ok(max_seqlen_k))
    return fail(FAL_ERR_INVALID, "invalid sizes");
  const size_t need = fal_decode_workspace_size(batch, heads_q, heads_kv, max_seqlen_k, head_dim);
  if (need > kNoAllocScratchBytes)
    return fail(FAL_ERR_WORKSPACE,
                "fal_decode_noalloc: this call needs %zu bytes of workspace, above the fixed %zu-byte "
                "device array (use fal_decode with a caller workspace)",
                need, kNoAllocScratchBytes);
  void* ws = nullptr;
  int rc = scratch_for_current_device(&ws);
  if (rc) return rc;
  return fal_decode_impl(q, k_cache, v_cache, cache_seqlens, mask_bias, mask_stride, o, lse, batch, heads_q,
                         heads_kv, head_dim, max_seqlen_k, q_strides, k_strides, v_strides, o_strides,
                         softmax_scale, ws, kNoAllocScratchBytes, stream, 0);
}

}  // extern "C"

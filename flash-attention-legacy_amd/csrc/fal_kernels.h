// Kernel parameter blocks and launcher declarations shared by the kernel
// translation units and the C-ABI layer.  Strides are in elements and 64-bit
// (the reference's int32 strides, csrc/include/flash_attn_common.h:25-147,
// overflow above 2^31 elements); the last dimension is always unit-stride.
#pragma once

#include "fal_common.h"

namespace fal {

// Forward.  Batched mode (cu_q == nullptr): tensors are [B, H, N, d] addressed
// by (b, h, n) strides.  Varlen mode: b is 0, the "seq" stride is the token
// stride of the packed [total, H, d] tensor and cu_q/cu_k give the segments;
// `work` is the (sequence, query-tile) list built by varlen_schedule_kernel.
struct FwdParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  float* lse;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t l_sb, l_sh, l_ss;
  int B, Hq, Hkv, Nq, Nk;
  int n_qtiles;
  int total_q, total_k;   // varlen: rows of the packed Q and K/V (segments are clamped to them)
  float scale_log2;   // softmax_scale * log2(e), signed, |.| >= 1e-30
  const int* cu_q;
  const int* cu_k;
  const int2* work;   // varlen work list; null: each workgroup derives its item from cu_q
  int num_seqs;       // varlen: segments in cu_q / cu_k (used when work is null)
  int bf16;           // element type of every fp16/bf16 tensor: 0 fp16, 1 bf16
  // Batched split-KV (grids too small to fill the GPU): each query tile's key tiles
  // are cut into splits of `kchunk` tiles, one workgroup each; the workgroups write
  // unnormalised partial outputs and their (max, sum), and fwd_combine_kernel merges
  // them.  kchunk = 0: one workgroup covers the whole key range and writes O and L.
  int kchunk;
  int nsplit;         // splits per query tile (grid = B * Hq * n_qtiles * nsplit)
  float* part_o;      // [B * Hq * nsplit, Nq, d] fp32
  float* part_ml;     // [B * Hq * nsplit, Nq, 2]: log2-domain max m and sum l (true sum 2^m * l)
  // Batched head_dim-128 pipelined kernel with Hq/Hkv a multiple of 4: the four waves of
  // a workgroup take the same 64 query rows of four query heads that share one KV head
  // (n_qtiles counts 64-row tiles, the grid B * Hq/4 * n_qtiles), so under a causal mask
  // every wave stops at the same diagonal tile.
  int gqa4;
  // pipelined kernel: persistent grid (one workgroup per CU walking pairs of query tiles)
  int persist;
};

// Backward.  Same addressing as FwdParams, plus dO (do_*), the fp32 dQ
// accumulator (dqa_*, same layout as Q but float), dK/dV outputs and the
// per-row delta = rowsum(dO * O) (same layout as lse).
struct BwdParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  const half_t* o;
  const half_t* dout;
  const float* lse;
  float* delta;
  float* dq_acc;
  half_t* dq;
  half_t* dk;
  half_t* dv;
  int64_t q_sb, q_sh, q_ss;
  int64_t k_sb, k_sh, k_ss;
  int64_t v_sb, v_sh, v_ss;
  int64_t o_sb, o_sh, o_ss;
  int64_t do_sb, do_sh, do_ss;
  int64_t l_sb, l_sh, l_ss;
  int64_t dqa_sb, dqa_sh, dqa_ss;
  int64_t dq_sb, dq_sh, dq_ss;
  int64_t dk_sb, dk_sh, dk_ss;
  int64_t dv_sb, dv_sh, dv_ss;
  int B, Hq, Hkv, Nq, Nk;
  int n_ktiles;
  float scale;        // softmax_scale (signed)
  float scale_log2;   // softmax_scale * log2(e) (signed)
  const int* cu_q;
  const int* cu_k;
  const int2* work;   // (sequence, kv-tile) list in varlen mode
  const int2* qwork;  // (sequence, query-tile) list of the dQ kernel in varlen mode
  int n_qitems;       // capacity of qwork
  int total_q;        // varlen: rows of the packed Q (row-wise kernels)
  int total_k;        // varlen: rows of the packed K/V
  int bf16;           // element type of every fp16/bf16 tensor: 0 fp16, 1 bf16
  float* lsd;         // batched head_dim 128: per 64-row tile, -L*log2(e)/c then -D (null: unused)
};

// KV-cache decode (one query token per sequence).
struct DecodeParams {
  const half_t* q;          // [B, Hq, d] via (q_sb, q_sh)
  const half_t* k;          // cache rows via (k_sb, k_ss, k_sh)
  const half_t* v;
  const int* seqlens;       // [B] valid cache rows
  const float* bias;        // optional additive mask [B, bias_sb]
  half_t* o;                // [B, Hq, d] via (o_sb, o_sh)
  float* lse;               // optional [B, Hq] natural-log LSE
  float* part_o;            // [B, Hq, max_splits, d] fp32 partial outputs
  float* part_m;            // [B, Hq, max_splits] partial log2-domain LSE
  const int2* work;         // [B * max_splits] (sequence, split) items, longest first
  int64_t q_sb, q_sh;
  int64_t k_sb, k_ss, k_sh;
  int64_t v_sb, v_ss, v_sh;
  int64_t o_sb, o_sh;
  int64_t bias_sb;
  int B, Hq, Hkv, max_splits, chunk;
  int max_seqlen;           // cache rows; cache_seqlens are clamped to it
  float scale_log2;
  int negate_q;
  int bf16;           // element type of every fp16/bf16 tensor: 0 fp16, 1 bf16
};

hipError_t launch_fwd(const FwdParams& p, int d, int causal, dim3 grid, hipStream_t st);
int fwd_block_m(int d);
bool fwd_pipe_ok(int d);   // batched calls of this head dim run the pipelined tile loop
bool fwd_gqa4_ok(int d, int64_t heads_q, int64_t heads_kv);   // FwdParams::gqa4 applies
int fwd_block_m_varlen(int d);   // query rows per workgroup of a packed-sequence call
int fwd_block_n(int d);
// Split-KV plan for a batched forward: sets kchunk / nsplit (kchunk 0 = no split) and
// returns the workspace bytes the split needs (0 without a split).
size_t fwd_split_plan(int64_t B, int64_t Hq, int64_t Nq, int64_t Nk, int d, int causal, int* kchunk, int* nsplit);
hipError_t launch_fwd_combine(const FwdParams& p, int d, int causal, hipStream_t st);
// Rows of up to two packed [rows, heads, d] 16-bit tensors that the schedule kernel
// zeroes: those before the first segment and from the end of the last one on
// (the rows no segment covers when cu_seqlens is monotone).
struct ZeroRows {
  void* a;
  void* b;                            // optional
  int64_t a_row, a_head, b_row, b_head;   // element strides
  int heads, d;
};
// Small varlen forwards (at most this many sequences and query tokens) need no
// schedule kernel: each workgroup derives its (sequence, tile) item from cu_seqlens
// itself.  That saves a launch where launches dominate, and costs about 1% on large
// batches (C4: 874 against 882 TFLOP/s), which keep the list.
#ifndef FAL_VARLEN_SMALL_SEQS
#define FAL_VARLEN_SMALL_SEQS 64
#endif
#ifndef FAL_VARLEN_SMALL_TOKENS
#define FAL_VARLEN_SMALL_TOKENS 16384
#endif
constexpr int kVarlenSmallSeqs = FAL_VARLEN_SMALL_SEQS;
constexpr int kVarlenSmallTokens = FAL_VARLEN_SMALL_TOKENS;
hipError_t launch_varlen_schedule(const int* cu, int num_seqs, int rows, int tile, int nbuckets, int descending,
                                  int2* work, int capacity, hipStream_t st, const ZeroRows* zero = nullptr);

int bwd_block_n(int d);
hipError_t launch_bwd(const BwdParams& p, int d, int causal, dim3 grid, hipStream_t st);
hipError_t launch_bwd_pre(const BwdParams& p, int d, int rows_batched, hipStream_t st);
hipError_t launch_bwd_post(const BwdParams& p, int d, hipStream_t st);
// head dims whose dQ comes from the query-outer kernel (no fp32 accumulator)
bool bwd_split_dq(int d);
int bwd_dq_block_m(int d);
// batched head_dim d uses bwd_kv_pipe_kernel (workspace holds the lsd array)
bool bwd_pipe(int d);
hipError_t launch_bwd_dq(const BwdParams& p, int d, int causal, dim3 grid, hipStream_t st);

int decode_chunk(int d, int B, int Hkv, int max_seqlen);

hipError_t launch_decode(const DecodeParams& p, int d, hipStream_t st);

}  // namespace fal

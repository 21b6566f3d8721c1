/*
 * fal_api.h -- C ABI of libfal_hip.so, the gfx950 (MI355X) attention library
 * behind the flash_attn_legacy Python package.
 *
 * It replaces the reference's pybind11 extension `flash_attn_legacy_cuda`
 * (csrc/flash_attn_legacy.cpp:294-310).  Differences of form, not of meaning:
 *   - plain device pointers, sizes and element strides instead of torch::Tensor;
 *   - the caller allocates every output and workspace (the *_workspace_size
 *     functions say how much); the library never allocates or frees memory;
 *   - errors are returned as a status code; fal_last_error() gives the message
 *     (the reference raises through TORCH_CHECK / FLASH_ATTN_CHECK_CUDA,
 *     csrc/flash_attn_legacy.cpp:48-60, csrc/include/flash_attn_common.h:297-305).
 *
 * Conventions
 *   - fp16 data (IEEE binary16; the *_bf16 entry points take bfloat16), fp32
 *     log-sum-exp, int32 sequence offsets.
 *   - `*_strides` point at three int64 element strides (batch, head, seq) of a
 *     tensor whose last (head_dim) dimension is contiguous.  Packed (varlen)
 *     tensors use (unused, head, token).  Base pointers must be 16-byte aligned
 *     and every stride a multiple of 8 elements.
 *   - head_dim is one of 32, 64, 96, 128, 256 (reference: flash_attn.py:34,
 *     flash_attn_legacy.cpp:56-57).
 *   - `stream` is a hipStream_t (NULL = default stream).  All work is enqueued
 *     asynchronously on it.
 *   - Functions are reentrant; they keep no state between calls apart from the
 *     thread-local error message.
 */
#ifndef FAL_API_H
#define FAL_API_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum fal_status {
  FAL_OK = 0,
  FAL_ERR_INVALID = 1,      /* bad argument (shape, stride, alignment, null pointer) */
  FAL_ERR_UNSUPPORTED = 2,  /* head_dim or device not supported */
  FAL_ERR_LAUNCH = 3,       /* HIP launch / runtime error */
  FAL_ERR_WORKSPACE = 4     /* workspace missing or too small */
};

/* Message for the last failing call on this thread ("" if none). */
const char* fal_last_error(void);

/* Library version string, e.g. "0.5.0+gfx950". */
const char* fal_version(void);

/* 1 if `device` is a gfx950 GPU this library was built for, else 0. */
int fal_device_supported(int device);

/*
 * Forward attention, batched layout.
 * Replaces flash_attn_forward (csrc/flash_attn_legacy.cpp:42-98).
 *   q [B, Hq, Nq, d]; k, v [B, Hkv, Nk, d]; o [B, Hq, Nq, d] (fp16);
 *   lse [B, Hq, Nq] fp32, contiguous, natural-log log-sum-exp of the scaled scores.
 * Hq % Hkv == 0 (query head h uses KV head h / (Hq/Hkv)).  The reference requires
 * Nq == Nk (flash_attn_legacy.cpp:58); Nq != Nk is accepted here with the same
 * top-left causal alignment (key j is visible to query i iff j <= i).
 */
/* workspace: fal_fwd_workspace_size bytes.  It is 0 (workspace may be NULL) unless the
 * grid is smaller than the GPU (fewer than 256 query tiles of 128 rows over batch and
 * heads, with long key ranges): such calls split each query tile's key range over
 * several workgroups, keep their partial outputs in the workspace and merge them in a
 * second kernel (a "split-KV" forward).  The results are the same up to fp32 rounding. */
size_t fal_fwd_workspace_size(int64_t batch, int64_t heads_q, int64_t seqlen_q, int64_t seqlen_k,
                              int64_t head_dim, int is_causal);
int fal_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
            int64_t batch, int64_t heads_q, int64_t heads_kv,
            int64_t seqlen_q, int64_t seqlen_k, int64_t head_dim,
            const int64_t* q_strides, const int64_t* k_strides,
            const int64_t* v_strides, const int64_t* o_strides,
            float softmax_scale, int is_causal,
            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Forward attention over packed variable-length sequences.
 * Replaces flash_attn_forward_varlen (csrc/flash_attn_legacy.cpp:193-290).
 *   q [total_q, Hq, d]; k, v [total_k, Hkv, d]; o [total_q, Hq, d];
 *   lse [total_q, Hq] fp32 contiguous;
 *   cu_seqlens_q / cu_seqlens_k: device int32 [num_seqs + 1] prefix offsets.
 * max_seqlen_q bounds the longest query segment (used to size the on-device
 * tile schedule).  No host synchronisation: the (sequence, tile) work list is
 * built on the device in `workspace` (fal_fwd_varlen_workspace_size bytes).  For
 * small problems (up to 64 sequences and 16384 query tokens) the size is 0,
 * `workspace` may be null, and each workgroup derives its item from cu_seqlens_q.
 */
size_t fal_fwd_varlen_workspace_size(int64_t num_seqs, int64_t total_q, int64_t max_seqlen_q,
                                     int64_t head_dim);
int fal_fwd_varlen(const void* q, const void* k, const void* v, void* o, float* lse,
                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t num_seqs,
                   int64_t total_q, int64_t total_k, int64_t heads_q, int64_t heads_kv,
                   int64_t head_dim, int64_t max_seqlen_q, int64_t max_seqlen_k,
                   const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* o_strides,
                   float softmax_scale, int is_causal,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward attention, batched layout.
 * Replaces flash_attn_backward (csrc/flash_attn_legacy.cpp:105-186) and the
 * kernels it launches (precompute_D, flash_attn_bwd_*_launch).
 *   dout, q, o [B, Hq, Nq, d]; k, v [B, Hkv, Nk, d]; lse [B, Hq, Nq] from fal_fwd.
 *   Outputs dq [B, Hq, Nq, d], dk / dv [B, Hkv, Nk, d] (fp16), fully overwritten.
 * workspace: fal_bwd_workspace_size bytes: the row deltas D, plus an fp32 dQ
 * accumulator for head_dim 256 (the other head dims write dQ from their own kernel).
 * All gradients are bitwise deterministic, except dQ at head_dim 256: it is
 * accumulated with fp32 atomics, so its low bits can vary run to run (as in the
 * reference, flash_attn_bwd.cu:618).
 */
size_t fal_bwd_workspace_size(int64_t batch, int64_t heads_q, int64_t seqlen_q, int64_t head_dim);
int fal_bwd(const void* dout, const void* q, const void* k, const void* v, const void* o,
            const float* lse, void* dq, void* dk, void* dv,
            int64_t batch, int64_t heads_q, int64_t heads_kv,
            int64_t seqlen_q, int64_t seqlen_k, int64_t head_dim,
            const int64_t* do_strides, const int64_t* q_strides, const int64_t* k_strides,
            const int64_t* v_strides, const int64_t* o_strides,
            const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
            float softmax_scale, int is_causal,
            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward attention over packed variable-length sequences, one launch for all
 * sequences.  Replaces the per-sequence Python loop of
 * FlashAttnVarlenFunc.backward (flash_attn_legacy/flash_attn.py:133-157), which
 * calls the batched backward once per sequence with host syncs in between.
 *   Layouts as fal_fwd_varlen; lse [total_q, Hq] from fal_fwd_varlen.
 */
size_t fal_bwd_varlen_workspace_size(int64_t num_seqs, int64_t total_q, int64_t total_k,
                                     int64_t heads_q, int64_t head_dim);
int fal_bwd_varlen(const void* dout, const void* q, const void* k, const void* v, const void* o,
                   const float* lse, void* dq, void* dk, void* dv,
                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t num_seqs,
                   int64_t total_q, int64_t total_k, int64_t heads_q, int64_t heads_kv,
                   int64_t head_dim, int64_t max_seqlen_q, int64_t max_seqlen_k,
                   const int64_t* do_strides, const int64_t* q_strides, const int64_t* k_strides,
                   const int64_t* v_strides, const int64_t* o_strides,
                   const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
                   float softmax_scale, int is_causal,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * KV-cache decode: one query token per sequence attends to the first
 * cache_seqlens[b] rows of its cache, with no causal mask.
 * Replaces the eager decode branch of flash_attn_legacy_forward
 * (flash_attn_legacy/integrations.py:77-98), which has no kernel in the reference.
 *   q [B, Hq, d] via q_strides (batch, head, -); o likewise;
 *   k_cache / v_cache rows addressed by strides (batch, head, seq) -- both the
 *   [B, S, Hkv, d] and the [B, Hkv, S, d] cache layouts work;
 *   cache_seqlens: device int32 [B], each in [0, max_seqlen_k];
 *   mask_bias: optional fp32 additive mask, row b at mask_bias + b*mask_stride
 *   (entries 0..cache_seqlens[b]-1 are read); NULL for none;
 *   lse: optional fp32 [B, Hq] natural-log LSE (NULL to skip).
 * Split-K: each sequence is cut into ceil(len / chunk) splits, chunk chosen from
 * (batch, heads_kv, max_seqlen_k); a second kernel merges them by log-sum-exp.
 */
size_t fal_decode_workspace_size(int64_t batch, int64_t heads_q, int64_t heads_kv,
                                 int64_t max_seqlen_k, int64_t head_dim);
int fal_decode(const void* q, const void* k_cache, const void* v_cache,
               const int32_t* cache_seqlens, const float* mask_bias, int64_t mask_stride,
               void* o, float* lse,
               int64_t batch, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
               int64_t max_seqlen_k,
               const int64_t* q_strides, const int64_t* k_strides,
               const int64_t* v_strides, const int64_t* o_strides,
               float softmax_scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * bf16 (bfloat16) forms of the five compute entry points: the same arguments,
 * shapes, strides, workspace sizes and status codes, with every fp16 tensor
 * (q, k, v, o, dout, dq, dk, dv, the caches) in bf16 instead; log-sum-exp, D and
 * mask bias stay fp32.  Products accumulate in fp32 (bf16 MFMA); P and dS are
 * rounded to bf16 for their second product, and the softmax scale is applied to
 * the fp32 scores.  No counterpart in the reference, which is fp16 only (its HF
 * integration casts bf16 models to fp16, integrations.py:65-67): this serves
 * bf16 models without that cast and its overflow risk.
 */
int fal_fwd_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                 int64_t batch, int64_t heads_q, int64_t heads_kv,
                 int64_t seqlen_q, int64_t seqlen_k, int64_t head_dim,
                 const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides,
                 float softmax_scale, int is_causal,
                 void* workspace, size_t workspace_bytes, void* stream);
int fal_fwd_varlen_bf16(const void* q, const void* k, const void* v, void* o, float* lse,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t num_seqs,
                        int64_t total_q, int64_t total_k, int64_t heads_q, int64_t heads_kv,
                        int64_t head_dim, int64_t max_seqlen_q, int64_t max_seqlen_k,
                        const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides,
                        float softmax_scale, int is_causal,
                        void* workspace, size_t workspace_bytes, void* stream);
int fal_bwd_bf16(const void* dout, const void* q, const void* k, const void* v, const void* o,
                 const float* lse, void* dq, void* dk, void* dv,
                 int64_t batch, int64_t heads_q, int64_t heads_kv,
                 int64_t seqlen_q, int64_t seqlen_k, int64_t head_dim,
                 const int64_t* do_strides, const int64_t* q_strides, const int64_t* k_strides,
                 const int64_t* v_strides, const int64_t* o_strides,
                 const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
                 float softmax_scale, int is_causal,
                 void* workspace, size_t workspace_bytes, void* stream);
int fal_bwd_varlen_bf16(const void* dout, const void* q, const void* k, const void* v, const void* o,
                        const float* lse, void* dq, void* dk, void* dv,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t num_seqs,
                        int64_t total_q, int64_t total_k, int64_t heads_q, int64_t heads_kv,
                        int64_t head_dim, int64_t max_seqlen_q, int64_t max_seqlen_k,
                        const int64_t* do_strides, const int64_t* q_strides, const int64_t* k_strides,
                        const int64_t* v_strides, const int64_t* o_strides,
                        const int64_t* dq_strides, const int64_t* dk_strides, const int64_t* dv_strides,
                        float softmax_scale, int is_causal,
                        void* workspace, size_t workspace_bytes, void* stream);
int fal_decode_bf16(const void* q, const void* k_cache, const void* v_cache,
                    const int32_t* cache_seqlens, const float* mask_bias, int64_t mask_stride,
                    void* o, float* lse,
                    int64_t batch, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                    int64_t max_seqlen_k,
                    const int64_t* q_strides, const int64_t* k_strides,
                    const int64_t* v_strides, const int64_t* o_strides,
                    float softmax_scale, void* workspace, size_t workspace_bytes, void* stream);

/*
 * fal_decode without a workspace argument and without any allocation.
 * No counterpart in the reference.  It serves callers that cannot allocate device
 * memory: code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Arguments, results and status codes are those of fal_decode (fp16),
 * minus workspace / workspace_bytes.
 *   - The workspace is a fixed 16 MiB device array inside the library (one copy per
 *     GPU, held until the process ends).  A call whose fal_decode_workspace_size
 *     exceeds 16 MiB fails with FAL_ERR_WORKSPACE (e.g. batch 32, 32 query heads,
 *     d 128 allows caches up to 32768 rows per sequence at the default split size).
 *   - Every call on one GPU shares that array: calls that overlap in time on one GPU
 *     (different streams or threads) race and give wrong results.  Serialise them.
 *   - The first call on each device looks up the array's device address; no
 *     allocation, free or memset happens in any call.
 */
int fal_decode_noalloc(const void* q, const void* k_cache, const void* v_cache,
                       const int32_t* cache_seqlens, const float* mask_bias, int64_t mask_stride,
                       void* o, float* lse,
                       int64_t batch, int64_t heads_q, int64_t heads_kv, int64_t head_dim,
                       int64_t max_seqlen_k,
                       const int64_t* q_strides, const int64_t* k_strides,
                       const int64_t* v_strides, const int64_t* o_strides,
                       float softmax_scale, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FAL_API_H */

"""
Flash Attention Legacy -- PyTorch autograd interface, MI355X (gfx950) build.

Same public API as the reference package (flash_attn_legacy/flash_attn.py): MHA,
GQA and MQA through ``flash_attention``, packed sequences through
``flash_attn_varlen_func``, and the ``FlashAttention`` / ``FlashMultiHeadAttention``
modules.  The compute runs in hand-written HIP kernels for gfx950 behind the C ABI
of ``libfal_hip.so`` (see ``hip_ext``).  New here: ``flash_attn_with_kvcache`` for
KV-cache decode, and a single-launch varlen backward.
"""

import math
from typing import Optional

import torch
import torch.nn as nn
from torch.autograd import Function

from . import hip_ext as _ext

_HEAD_DIMS = (32, 64, 96, 128, 256)
# float16 as in the reference; bfloat16 runs natively as well (bf16 MFMA, fp32 accumulation)
_DTYPES = (torch.float16, torch.bfloat16)


class FlashAttentionFunc(Function):
    """Autograd function for Flash Attention v2 (reference flash_attn.py:22-56).
    GQA: Q [B, H_q, N, d], K/V [B, H_kv, N, d] with H_q % H_kv == 0."""

    @staticmethod
    def forward(ctx, q, k, v, softmax_scale, is_causal):
        assert q.dtype in _DTYPES, f"Q must be float16 or bfloat16, got {q.dtype}"
        assert k.dtype == q.dtype and v.dtype == q.dtype
        assert q.is_cuda and q.dim() == 4
        d = q.shape[-1]
        assert d in _HEAD_DIMS, f"head_dim must be 32, 64, 96, 128, or 256, got {d}"

        H_q, H_kv = q.shape[1], k.shape[1]
        assert H_q % H_kv == 0, f"H_q ({H_q}) must be divisible by H_kv ({H_kv})"

        o, lse = _ext.forward(q, k, v, softmax_scale, is_causal)

        ctx.save_for_backward(q, k, v, o, lse)
        ctx.softmax_scale = softmax_scale
        ctx.is_causal = is_causal
        return o

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, o, lse = ctx.saved_tensors
        dq, dk, dv = _ext.backward(grad_output, q, k, v, o, lse, ctx.softmax_scale, ctx.is_causal)
        return dq, dk, dv, None, None


def flash_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    softmax_scale: Optional[float] = None,
    is_causal: bool = False,
) -> torch.Tensor:
    """
    Flash Attention v2 on MI355X.

    Supports MHA, GQA, and MQA:
      - MHA: Q [B, H, N, d], K [B, H, N, d], V [B, H, N, d]
      - GQA: Q [B, H_q, N, d], K/V [B, H_kv, N, d], H_q divisible by H_kv
      - MQA: GQA with H_kv = 1

    Args:
        q: Query [B, H_q, N, d] float16 or bfloat16
        k: Key   [B, H_kv, N, d], same dtype
        v: Value [B, H_kv, N, d], same dtype
        softmax_scale: default 1/sqrt(d)
        is_causal: causal mask (top-left aligned: key j visible to query i iff j <= i)

    Returns:
        [B, H_q, N, d], dtype of q
    """
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    return FlashAttentionFunc.apply(q, k, v, softmax_scale, is_causal)


class FlashAttnVarlenFunc(Function):
    """Autograd function for packed variable-length attention (reference
    flash_attn.py:90-159).  Forward and backward are each one launch over all
    sequences; the reference's backward loops over sequences in Python."""

    @staticmethod
    def forward(ctx, q, k, v, cu_seqlens_q, cu_seqlens_k,
                max_seqlen_q, max_seqlen_k, softmax_scale, is_causal):
        assert q.dtype in _DTYPES, f"Q must be float16 or bfloat16, got {q.dtype}"
        assert k.dtype == q.dtype and v.dtype == q.dtype
        assert q.is_cuda and q.dim() == 3
        d = q.shape[-1]
        assert d in _HEAD_DIMS, f"head_dim must be 32, 64, 96, 128, or 256, got {d}"

        cu_seqlens_q = cu_seqlens_q.contiguous().to(torch.int32)
        cu_seqlens_k = cu_seqlens_k.contiguous().to(torch.int32)

        o, lse = _ext.forward_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k,
                                     max_seqlen_q, max_seqlen_k, softmax_scale, is_causal)

        ctx.save_for_backward(q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k)
        ctx.max_seqlen_q = max_seqlen_q
        ctx.max_seqlen_k = max_seqlen_k
        ctx.softmax_scale = softmax_scale
        ctx.is_causal = is_causal
        return o

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k = ctx.saved_tensors
        dq, dk, dv = _ext.backward_varlen(grad_output, q, k, v, o, lse, cu_seqlens_q, cu_seqlens_k,
                                          ctx.max_seqlen_q, ctx.max_seqlen_k,
                                          ctx.softmax_scale, ctx.is_causal)
        return dq, dk, dv, None, None, None, None, None, None


def flash_attn_varlen_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: Optional[float] = None,
    causal: bool = False,
) -> torch.Tensor:
    """
    Variable-length Flash Attention for packed sequences.

    Sequences are concatenated along the token dimension and ``cu_seqlens`` marks
    the boundaries, so no compute or memory is spent on padding.  Causal masking
    uses per-sequence (local) indices.

    Args:
        q: [total_q, num_heads, head_dim] float16 or bfloat16
        k: [total_k, num_heads_k, head_dim] float16
        v: [total_k, num_heads_k, head_dim] float16
        cu_seqlens_q: [batch_size + 1] int32 cumulative sequence lengths for Q
        cu_seqlens_k: [batch_size + 1] int32 cumulative sequence lengths for K/V
        max_seqlen_q: max sequence length in Q
        max_seqlen_k: max sequence length in K/V
        softmax_scale: default 1/sqrt(head_dim)
        causal: apply causal mask

    Returns:
        [total_q, num_heads, head_dim], dtype of q
    """
    assert q.dim() == 3, f"q must be [total, heads, d], got shape {q.shape}"
    assert k.dim() == 3, f"k must be [total, heads_k, d], got shape {k.shape}"
    assert v.dim() == 3, f"v must be [total, heads_k, d], got shape {v.shape}"
    assert q.dtype in _DTYPES, f"Q must be float16 or bfloat16, got {q.dtype}"

    d = q.shape[-1]
    assert d in _HEAD_DIMS, f"head_dim must be 32, 64, 96, 128, or 256, got {d}"

    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)

    return FlashAttnVarlenFunc.apply(
        q, k, v, cu_seqlens_q, cu_seqlens_k,
        max_seqlen_q, max_seqlen_k, softmax_scale, causal,
    )


def flash_attn_with_kvcache(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    cache_seqlens,
    softmax_scale: Optional[float] = None,
    return_softmax_lse: bool = False,
    cache_layout: str = "bshd",
):
    """
    KV-cache decode: each sequence's single new query token attends to the first
    ``cache_seqlens[b]`` rows of its cache (no causal mask), split-K on the GPU.

    The reference has no decode kernel; it computes this step with eager PyTorch
    (reference integrations.py:77-98).  Results match that formula.

    Args:
        q: [B, 1, H_q, d] float16 or bfloat16 (or [B, H_q, d])
        k_cache, v_cache: [B, S_max, H_kv, d] float16 (``cache_layout="bshd"``) or
            [B, H_kv, S_max, d] (``"bhsd"``, the HF layout)
        cache_seqlens: int32 tensor [B] (or an int for all sequences)
        softmax_scale: default 1/sqrt(d)
        return_softmax_lse: also return the natural-log LSE [B, H_q] fp32

    Returns:
        [B, 1, H_q, d] float16 (same rank as ``q``), and the LSE if requested.
    """
    squeeze = q.dim() == 3
    q3 = q if squeeze else q.reshape(q.shape[0], q.shape[2], q.shape[3]) if q.shape[1] == 1 else None
    assert q3 is not None, "flash_attn_with_kvcache supports one query token per sequence"
    assert q.dtype in _DTYPES, f"q must be float16 or bfloat16, got {q.dtype}"
    d = q3.shape[-1]
    assert d in _HEAD_DIMS, f"head_dim must be 32, 64, 96, 128, or 256, got {d}"
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(d)
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((q3.shape[0],), cache_seqlens, dtype=torch.int32, device=q.device)
    res = _ext.decode(q3, k_cache, v_cache, cache_seqlens, softmax_scale,
                      cache_layout=cache_layout, return_lse=return_softmax_lse)
    o, lse = res if return_softmax_lse else (res, None)
    if not squeeze:
        o = o.unsqueeze(1)
    return (o, lse) if return_softmax_lse else o


class FlashAttention(nn.Module):
    """Drop-in Flash Attention module. Supports GQA/MQA (reference flash_attn.py:223-235)."""

    def __init__(self, head_dim: int = 64, causal: bool = False,
                 softmax_scale: Optional[float] = None):
        super().__init__()
        assert head_dim in _HEAD_DIMS
        self.head_dim = head_dim
        self.causal = causal
        self.softmax_scale = softmax_scale or (1.0 / math.sqrt(head_dim))

    def forward(self, q, k, v):
        return flash_attention(q, k, v, self.softmax_scale, self.causal)


class FlashMultiHeadAttention(nn.Module):
    """
    Multi-head attention with the Flash Attention backend (reference flash_attn.py:238-312).
    Supports standard MHA, GQA, and MQA.

    Args:
        embed_dim: Total embedding dimension
        num_heads: Number of query heads (H_q)
        num_kv_heads: Number of KV heads (H_kv). Default = num_heads (standard MHA).
        causal: Apply causal mask
        bias: Use bias in linear projections
        dropout: Dropout rate (applied post-attention)
    """

    def __init__(self, embed_dim: int, num_heads: int, num_kv_heads: Optional[int] = None,
                 causal: bool = False, bias: bool = True, dropout: float = 0.0):
        super().__init__()
        if num_kv_heads is None:
            num_kv_heads = num_heads

        assert embed_dim % num_heads == 0
        assert num_heads % num_kv_heads == 0, (
            f"num_heads ({num_heads}) must be divisible by num_kv_heads ({num_kv_heads})"
        )

        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = embed_dim // num_heads
        assert self.head_dim in _HEAD_DIMS, f"head_dim={self.head_dim}, must be 32, 64, 96, 128, or 256"

        self.causal = causal
        self.scale = 1.0 / math.sqrt(self.head_dim)

        self.q_proj = nn.Linear(embed_dim, num_heads * self.head_dim, bias=bias)
        self.k_proj = nn.Linear(embed_dim, num_kv_heads * self.head_dim, bias=bias)
        self.v_proj = nn.Linear(embed_dim, num_kv_heads * self.head_dim, bias=bias)
        self.out_proj = nn.Linear(embed_dim, embed_dim, bias=bias)
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    def forward(self, x: torch.Tensor, key_value: Optional[torch.Tensor] = None):
        """x: [B, N, embed_dim]; key_value: optional [B, N_kv, embed_dim] for cross-attention.
        Returns [B, N, embed_dim]."""
        B, N, _ = x.shape
        kv = key_value if key_value is not None else x

        # [B, N, H, d] views transposed to [B, H, N, d]: the kernels take the strides
        # directly, so no copy is made here.
        q = self.q_proj(x).view(B, N, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(kv).view(B, -1, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(kv).view(B, -1, self.num_kv_heads, self.head_dim).transpose(1, 2)

        orig_dtype = q.dtype
        if q.dtype not in _DTYPES:
            q, k, v = q.half(), k.half(), v.half()

        out = flash_attention(q, k, v, self.scale, self.causal)

        if orig_dtype != out.dtype:
            out = out.to(orig_dtype)

        out = out.transpose(1, 2).contiguous().view(B, N, self.embed_dim)
        return self.dropout(self.out_proj(out))

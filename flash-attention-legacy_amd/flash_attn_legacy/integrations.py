"""
HuggingFace Transformers integration for flash_attn_legacy (MI355X build).

Registers "flash_attn_legacy" as an attention implementation, so models load with

    model = AutoModelForCausalLM.from_pretrained(
        "meta-llama/Llama-2-7b-hf",
        attn_implementation="flash_attn_legacy",
        torch_dtype=torch.float16,
        device_map="cuda",
    )

Same registration and prefill behaviour as the reference (integrations.py:24-161).
Decode steps (one new query token against a longer KV cache) go to the split-K
decode kernel instead of the reference's eager matmul/softmax/matmul; the result
is the same formula (integrations.py:77-98).
"""

import math
from typing import Optional

import torch
import torch.nn as nn

_HEAD_DIMS = (32, 64, 96, 128, 256)


def _mask_to_bias(attention_mask: torch.Tensor, batch: int, kv_len: int):
    """Reduce an HF attention mask to one additive fp32 row per sequence [B, kv_len]
    for a single-token query, or None when the mask varies over heads.  Boolean masks
    mean True = attend (transformers' convention); float masks are additive."""
    m = attention_mask
    if m.dim() == 2:                       # [B, kv] padding mask (1 = keep)
        m = m[:, None, None, :]
    if m.dim() != 4 or m.shape[1] != 1:
        return None
    row = m[:, 0, -1, :kv_len]
    if row.shape[0] != batch:
        if row.shape[0] != 1:
            return None
        row = row.expand(batch, -1)
    if row.dtype == torch.bool:
        return torch.zeros(row.shape, dtype=torch.float32, device=row.device).masked_fill_(~row, float("-inf"))
    if not row.is_floating_point():       # integer padding mask, 1 = keep
        return torch.zeros(row.shape, dtype=torch.float32, device=row.device).masked_fill_(row == 0, float("-inf"))
    return row.float()


def _padded_prefill(query, key, value, keep, scaling, is_causal):
    """Prefill of a padded batch: the tokens that ``keep`` [B, N] (bool, True = real
    token) marks are packed into one varlen batch, attended with the varlen kernel
    (causal within each sequence's own tokens), and scattered back; padded query rows
    are zero.  This is what FlashAttention-2's HF path computes for a 2-D padding mask."""
    from .flash_attn import flash_attn_varlen_func
    B, H_q, N, d = query.shape
    H_kv = key.shape[1]
    flat = keep.reshape(-1)
    idx = flat.nonzero().squeeze(1)
    seqlens = keep.sum(1, dtype=torch.int32)
    cu = torch.nn.functional.pad(torch.cumsum(seqlens, 0, dtype=torch.int32), (1, 0))
    max_len = int(seqlens.max())
    pack = lambda t, h: t.transpose(1, 2).reshape(B * N, h, d).index_select(0, idx)
    o = flash_attn_varlen_func(pack(query, H_q), pack(key, H_kv), pack(value, H_kv), cu, cu, max_len, max_len,
                               softmax_scale=scaling, causal=is_causal)
    out = o.new_zeros((B * N, H_q, d)).index_copy(0, idx, o)
    return out.view(B, N, H_q, d).transpose(1, 2)


def _eager(query, key, value, attention_mask, scaling, is_causal):
    """The reference's eager branch (integrations.py:80-98), used only for inputs outside
    the kernels' contract (unsupported head_dim, per-head masks, masked multi-token
    queries against a longer cache).  A 2-D padding mask [B, kv] (True or 1 = keep)
    applies to every query row."""
    q_len, kv_len = query.shape[2], key.shape[2]
    if attention_mask is not None and attention_mask.dim() == 2:
        attention_mask = attention_mask[:, None, None, -kv_len:].bool()
    H_q, H_kv = query.shape[1], key.shape[1]
    if H_kv != H_q:
        rep = H_q // H_kv
        key = key.repeat_interleave(rep, dim=1)
        value = value.repeat_interleave(rep, dim=1)
    s = torch.matmul(query, key.transpose(-2, -1)) * scaling
    if attention_mask is not None:
        if attention_mask.dtype == torch.bool:
            s = s.masked_fill(~attention_mask[..., :kv_len], float("-inf"))
        else:
            s = s + attention_mask[..., :kv_len]
    if is_causal and q_len > 1:
        causal_mask = torch.triu(
            torch.full((q_len, kv_len), float("-inf"), device=query.device, dtype=query.dtype),
            diagonal=1,
        )
        s = s + causal_mask
    return torch.matmul(torch.softmax(s, dim=-1), value)


def flash_attn_legacy_forward(
    module: nn.Module,
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    attention_mask: Optional[torch.Tensor],
    dropout: float = 0.0,
    scaling: Optional[float] = None,
    **kwargs,
):
    """Attention function for transformers' AttentionInterface (reference integrations.py:24-103).

    * prefill (q_len == kv_len): flash kernel.  A 2-D padding mask (what transformers
      passes for this implementation, once ``register`` has given it FlashAttention-2's
      mask function) takes the varlen kernel over the unpadded tokens; a 4-D mask is
      not applied, as in the reference (causality comes from ``is_causal``);
    * decode (q_len == 1 < kv_len): split-K decode kernel over the [B, H_kv, S, d]
      cache, with the mask's last row as an additive bias;
    * q_len != kv_len > 1 without a mask: forward kernel with top-left causal
      alignment, which is what the reference's eager branch computes;
    * anything else: the reference's eager formula.

    Returns (attn_output [B, N, H, d], None).
    """
    from .flash_attn import flash_attention
    from . import hip_ext

    B, H_q, q_len, d = query.shape
    kv_len = key.shape[2]

    if scaling is None:
        scaling = 1.0 / math.sqrt(d)

    # Causal flag: kwargs override, then module.is_causal, then (no mask and q_len > 1).
    if "is_causal" in kwargs:
        is_causal = kwargs["is_causal"]
    elif hasattr(module, "is_causal"):
        is_causal = module.is_causal
    elif attention_mask is None and q_len > 1:
        is_causal = True
    else:
        is_causal = False

    in_dtype = query.dtype
    # fp16 and bf16 run natively; other dtypes are cast to fp16 as in the reference
    # (integrations.py:65-67)
    half = lambda t: t if t.dtype in (torch.float16, torch.bfloat16) else t.half()
    attn_output = None

    if d in _HEAD_DIMS and q_len == kv_len and attention_mask is not None and attention_mask.dim() == 2:
        keep = attention_mask[:, -kv_len:].bool()
        if bool(keep.all()):
            attn_output = flash_attention(half(query), half(key), half(value),
                                          softmax_scale=scaling, is_causal=is_causal)
        else:
            attn_output = _padded_prefill(half(query), half(key), half(value), keep, scaling, is_causal)
    elif d in _HEAD_DIMS and q_len == kv_len:
        attn_output = flash_attention(half(query), half(key), half(value),
                                      softmax_scale=scaling, is_causal=is_causal)
    elif d in _HEAD_DIMS and q_len == 1 and H_q // key.shape[1] <= 32:
        bias = None if attention_mask is None else _mask_to_bias(attention_mask, B, kv_len)
        if attention_mask is None or bias is not None:
            seqlens = torch.full((B,), kv_len, dtype=torch.int32, device=query.device)
            o = hip_ext.decode(half(query)[:, :, 0, :], half(key), half(value), seqlens, scaling,
                               mask_bias=bias, cache_layout="bhsd")
            attn_output = o.unsqueeze(2)
    elif d in _HEAD_DIMS and attention_mask is None:
        attn_output = flash_attention(half(query), half(key), half(value),
                                      softmax_scale=scaling, is_causal=is_causal)

    if attn_output is None:
        attn_output = _eager(query, key, value, attention_mask, scaling, is_causal)
    elif attn_output.dtype != in_dtype:
        attn_output = attn_output.to(in_dtype)

    # [B, H, N, d] -> [B, N, H, d], the SDPA output layout
    attn_output = attn_output.transpose(1, 2).contiguous()
    return attn_output, None


def _config_head_dim_supported(config) -> bool:
    """Head dim of a model config (``head_dim``, else ``hidden_size // num_attention_heads``)
    is one the kernels support; unknown head dims count as supported (reference
    integrations.py:146-154)."""
    head_dim = getattr(config, "head_dim", None)
    if head_dim is None:
        hs = getattr(config, "hidden_size", None)
        nh = getattr(config, "num_attention_heads", None)
        if hs and nh:
            head_dim = hs // nh
    return head_dim is None or head_dim in _HEAD_DIMS


def register():
    """Register flash_attn_legacy in transformers' attention registry (reference
    integrations.py:106-161).

    1. ``ALL_ATTENTION_FUNCTIONS.register("flash_attn_legacy", flash_attn_legacy_forward)``,
       and FlashAttention-2's mask function for the same name, so that padded batches
       arrive with their 2-D padding mask (without it transformers passes no mask at
       all to an implementation it does not know, and padding is silently attended).
    2. Wrap ``PreTrainedModel._check_and_adjust_attn_implementation`` so this name skips
       transformers' flash-attention preload (any name containing "flash" triggers it),
       and falls back to "sdpa" for head dims the kernels do not support.

    Returns True if registration succeeded, False otherwise.
    """
    try:
        from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS, PreTrainedModel

        ALL_ATTENTION_FUNCTIONS.register("flash_attn_legacy", flash_attn_legacy_forward)
        try:
            from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, flash_attention_mask
            ALL_MASK_ATTENTION_FUNCTIONS.register("flash_attn_legacy", flash_attention_mask)
        except ImportError:   # older transformers build 4-D masks for every implementation
            pass

        original_check = PreTrainedModel._check_and_adjust_attn_implementation
        if getattr(original_check, "_flash_attn_legacy_patch", False):
            return True

        def _patched_check(self, attn_implementation, is_init_check=False, allow_all_kernels=False):
            if attn_implementation == "flash_attn_legacy":
                if not _config_head_dim_supported(self.config):
                    return original_check(self, "sdpa", is_init_check, allow_all_kernels)
                return "flash_attn_legacy"
            return original_check(self, attn_implementation, is_init_check, allow_all_kernels)

        _patched_check._flash_attn_legacy_patch = True
        PreTrainedModel._check_and_adjust_attn_implementation = _patched_check
        return True
    except (ImportError, AttributeError):
        return False

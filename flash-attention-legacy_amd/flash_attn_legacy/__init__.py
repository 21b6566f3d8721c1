"""
Flash Attention Legacy -- Flash Attention v2 for AMD Instinct MI355X (gfx950)
==============================================================================

Drop-in for the ``flash_attn_legacy`` package: same functions, modules and
HuggingFace registration, computed by hand-written HIP kernels for CDNA4.

Supports MHA, GQA (grouped-query) and MQA (multi-query) attention; packed
variable-length sequences; KV-cache decode.

Head dimensions: 32, 64, 96, 128, 256

Quick start:
    >>> import torch
    >>> from flash_attn_legacy import flash_attention
    >>> q = torch.randn(2, 8, 1024, 64, device='cuda', dtype=torch.float16)
    >>> k = torch.randn(2, 8, 1024, 64, device='cuda', dtype=torch.float16)
    >>> v = torch.randn(2, 8, 1024, 64, device='cuda', dtype=torch.float16)
    >>> out = flash_attention(q, k, v, is_causal=True)
"""

__version__ = "0.5.0"

from .flash_attn import (
    flash_attention,
    flash_attn_varlen_func,
    flash_attn_with_kvcache,
    FlashAttention,
    FlashMultiHeadAttention,
)

from .utils import (
    check_gpu_compatibility,
    get_device_info,
)

from .integrations import register

__all__ = [
    "flash_attention",
    "flash_attn_varlen_func",
    "flash_attn_with_kvcache",
    "FlashAttention",
    "FlashMultiHeadAttention",
    "check_gpu_compatibility",
    "get_device_info",
    "register",
]

# Auto-register with HuggingFace transformers if available
register()

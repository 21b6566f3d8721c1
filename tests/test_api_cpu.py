"""Python layer on a CPU-only host: the public API surface of the reference package
(flash_attn_legacy/__init__.py:31-51), its argument checks (flash_attn.py:29-37,
100-103,206-212), module construction (flash_attn.py:223-312) and the HuggingFace
registration (integrations.py:106-161).  No kernel runs here."""

import math

import pytest
import torch


def test_public_api_surface():
    import flash_attn_legacy as fal
    for name in ("flash_attention", "flash_attn_varlen_func", "FlashAttention", "FlashMultiHeadAttention",
                 "check_gpu_compatibility", "get_device_info", "register", "flash_attn_with_kvcache"):
        assert hasattr(fal, name), name
    assert fal.__version__ == "0.5.0"


def test_forward_argument_checks():
    from flash_attn_legacy import flash_attention
    q = torch.zeros(1, 2, 8, 64)
    with pytest.raises(AssertionError, match="float16"):
        flash_attention(q, q, q)
    qh = q.half()
    with pytest.raises(AssertionError):          # not on a GPU
        flash_attention(qh, qh, qh)


def test_varlen_argument_checks():
    from flash_attn_legacy import flash_attn_varlen_func
    cu = torch.tensor([0, 8], dtype=torch.int32)
    with pytest.raises(AssertionError, match=r"q must be \[total, heads, d\]"):
        flash_attn_varlen_func(torch.zeros(1, 8, 2, 64).half(), torch.zeros(8, 2, 64).half(),
                               torch.zeros(8, 2, 64).half(), cu, cu, 8, 8)
    with pytest.raises(AssertionError, match="head_dim must be"):
        x = torch.zeros(8, 2, 48).half()
        flash_attn_varlen_func(x, x, x, cu, cu, 8, 8)


def test_module_construction():
    from flash_attn_legacy import FlashAttention, FlashMultiHeadAttention
    m = FlashMultiHeadAttention(512, num_heads=8, num_kv_heads=2, causal=True)
    assert m.head_dim == 64 and m.num_kv_heads == 2
    assert abs(m.scale - 1 / 8) < 1e-12
    with pytest.raises(AssertionError):
        FlashMultiHeadAttention(512, num_heads=8, num_kv_heads=3)
    with pytest.raises(AssertionError):
        FlashMultiHeadAttention(480, num_heads=10)      # head_dim 48
    assert FlashAttention(head_dim=128).softmax_scale == pytest.approx(1 / math.sqrt(128))


def test_hf_registration():
    from transformers.modeling_utils import ALL_ATTENTION_FUNCTIONS, PreTrainedModel
    import flash_attn_legacy
    from flash_attn_legacy.integrations import flash_attn_legacy_forward
    assert flash_attn_legacy.register() is True
    assert ALL_ATTENTION_FUNCTIONS["flash_attn_legacy"] is flash_attn_legacy_forward
    assert getattr(PreTrainedModel._check_and_adjust_attn_implementation, "_flash_attn_legacy_patch", False)
    # padded batches reach the attention function with their 2-D padding mask
    from transformers.masking_utils import ALL_MASK_ATTENTION_FUNCTIONS, flash_attention_mask
    assert ALL_MASK_ATTENTION_FUNCTIONS["flash_attn_legacy"] is flash_attention_mask
    # idempotent: registering again does not wrap the check twice
    flash_attn_legacy.register()
    chk = PreTrainedModel._check_and_adjust_attn_implementation
    assert getattr(chk, "_flash_attn_legacy_patch", False)


def test_hf_head_dim_fallback_to_sdpa():
    from transformers import LlamaConfig
    from flash_attn_legacy.integrations import _config_head_dim_supported
    assert not _config_head_dim_supported(LlamaConfig(hidden_size=480, num_attention_heads=10))   # 48
    assert _config_head_dim_supported(LlamaConfig(hidden_size=512, num_attention_heads=8))        # 64
    assert _config_head_dim_supported(LlamaConfig(hidden_size=512, num_attention_heads=8, head_dim=128))


def test_mask_reduction_for_decode():
    from flash_attn_legacy.integrations import _mask_to_bias
    m = torch.zeros(2, 1, 1, 6)
    m[0, ..., :2] = float("-inf")
    b = _mask_to_bias(m, 2, 5)
    assert b.shape == (2, 5) and torch.isinf(b[0, :2]).all() and (b[1] == 0).all()
    bm = torch.ones(2, 1, 1, 5, dtype=torch.bool)
    bm[1, ..., 0] = False
    b = _mask_to_bias(bm, 2, 5)
    assert torch.isneginf(b[1, 0]) and (b[0] == 0).all()
    pad = torch.tensor([[1, 1, 0], [1, 1, 1]])
    b = _mask_to_bias(pad, 2, 3)
    assert torch.isneginf(b[0, 2]) and (b[1] == 0).all()
    assert _mask_to_bias(torch.zeros(2, 4, 1, 5), 2, 5) is None    # per-head mask: not reducible


def test_eager_fallback_takes_2d_padding_mask():
    """A 2-D padding mask in the eager branch equals the same mask as an additive 4-D
    row broadcast over heads and query rows (and keys it masks get zero weight)."""
    from flash_attn_legacy.integrations import _eager
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(2, 4, 3, 8, generator=g) for _ in range(3))
    pad = torch.tensor([[0, 1, 1, 1, 1], [1, 1, 1, 1, 1]])
    k5, v5 = torch.randn(2, 4, 5, 8, generator=g), torch.randn(2, 4, 5, 8, generator=g)
    add = torch.zeros(2, 1, 1, 5).masked_fill(pad[:, None, None, :] == 0, float("-inf"))
    a = _eager(q, k5, v5, pad, 0.3, False)
    b = _eager(q, k5, v5, add, 0.3, False)
    assert torch.allclose(a, b)
    v5b = v5.clone()
    v5b[0, :, 0] += 100.0           # the padded key's value must not matter
    assert torch.allclose(_eager(q, k5, v5b, pad, 0.3, False), a)


def test_utils_without_gpu():
    from flash_attn_legacy import check_gpu_compatibility, get_device_info
    if torch.cuda.is_available():
        pytest.skip("GPU host")
    assert check_gpu_compatibility(verbose=False) is False
    with pytest.raises(RuntimeError):
        get_device_info()


def test_bench_refuses_several_gpus():
    """bench.py measures one GPU; --gpus N > 1 exits with a message instead of running."""
    import os
    import subprocess
    import sys
    root = os.path.join(os.path.dirname(__file__), "..")
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)

"""Device detection on the MI355X, and the flash-vs-standard A/B of the reference's
tests/test_performance.py:88-184 (correctness, speed) and utils.py's benchmark helper.

The reference only asserts that flash attention is not catastrophically slower than
standard attention (speed-up > 0.2, test_performance.py:178-184); on gfx950 the fused
kernel is asserted to be faster from N = 1024 on.
"""

import math

import pytest
import torch

pytestmark = pytest.mark.gpu


def test_device_info_reports_gfx950():
    from flash_attn_legacy import check_gpu_compatibility, get_device_info
    info = get_device_info()
    assert info["gfx_arch"] == "gfx950"
    assert info["supported"] is True
    assert info["sm_version"] >= 30            # the reference's own check (test_flash_attn.py:473-474)
    assert info["multiprocessor_count"] == 256
    assert info["peak_fp16_tflops"] == 2500.0 and info["peak_hbm_gbs"] == 8000.0
    assert check_gpu_compatibility(verbose=False) is True


def _standard(q, k, v, scale, causal):
    s = (q.float() @ k.float().transpose(-1, -2)) * scale
    if causal:
        n = q.shape[-2]
        s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool, device=q.device), 1), float("-inf"))
    return torch.softmax(s, dim=-1).half() @ v


@pytest.mark.parametrize("N", [256, 1024, 2048])
@pytest.mark.parametrize("d", [64, 128])
def test_correctness_ab(N, d):
    from flash_attn_legacy import flash_attention
    g = torch.Generator().manual_seed(N + d)
    q, k, v = ((torch.randn(2, 8, N, d, generator=g) * 0.3).half().cuda() for _ in range(3))
    scale = 1.0 / math.sqrt(d)
    diff = (flash_attention(q, k, v, softmax_scale=scale, is_causal=True).float()
            - _standard(q, k, v, scale, True).float()).abs().max().item()
    assert diff < 2e-3


@pytest.mark.parametrize("N", [512, 1024, 2048, 4096])
def test_speed_ab(N):
    from flash_attn_legacy.utils import benchmark_flash_vs_standard
    r = benchmark_flash_vs_standard(batch_size=2, num_heads=8, seq_len=N, head_dim=64, is_causal=True,
                                    num_warmup=3, num_iters=10)
    print(r)
    assert r["max_abs_diff"] < 2e-2
    assert r["speedup"] > 0.2
    if N >= 1024:
        assert r["speedup"] > 1.0, r
        assert r["flash_mem_mb"] < r["std_mem_mb"], r
    assert 0 < r["flash_frac_peak"] < 1

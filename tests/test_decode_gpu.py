"""KV-cache split-K decode parity on the GPU.

The reference has no decode kernel; its decode step is the eager formula of
flash_attn_legacy/integrations.py:77-98, restated by oracle.attention.decode.
Cases: both cache layouts, GQA ratios, lengths that are not multiples of the
split chunk, length 0/1, an additive mask row, LSE, and the benchmark
configuration C5 (B=32, 32q/8kv, d=128, lengths U[1024, 32768]).
"""

import math

import numpy as np
import pytest
import torch

from helpers import FWD_ATOL, max_abs, np64, randn
from oracle import attention as orc

pytestmark = pytest.mark.gpu


def run(q, kc, vc, lens, scale, layout="bshd", bias=None, lse=False):
    from flash_attn_legacy import hip_ext
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    return hip_ext.decode(q, kc, vc, seq, scale, mask_bias=bias, cache_layout=layout, return_lse=lse)


def ref(q, kc, vc, lens, scale, layout="bshd", bias=None):
    k = kc if layout == "bshd" else kc.transpose(1, 2)
    v = vc if layout == "bshd" else vc.transpose(1, 2)
    o, lse = orc.decode(np64(q)[:, None], np64(k), np64(v), np.array(lens), scale,
                        None if bias is None else np64(bias))
    return torch.from_numpy(o[:, 0]), torch.from_numpy(lse)


@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("layout", ["bshd", "bhsd"])
def test_decode_head_dims_layouts(d, layout):
    B, hq, hkv, S = 3, 8, 2, 700
    lens = [700, 1, 333]
    q = randn((B, hq, d), seed=1)
    shape = (B, S, hkv, d) if layout == "bshd" else (B, hkv, S, d)
    kc, vc = randn(shape, seed=2), randn(shape, seed=3)
    scale = 1.0 / math.sqrt(d)
    o, lse = run(q, kc, vc, lens, scale, layout, lse=True)
    ro, rl = ref(q, kc, vc, lens, scale, layout)
    assert max_abs(o, ro) <= FWD_ATOL
    assert max_abs(lse, rl) <= 1e-3


@pytest.mark.parametrize("hq,hkv", [(8, 8), (32, 8), (32, 1), (12, 4)])
def test_decode_gqa_ratios(hq, hkv):
    B, S, d = 2, 1500, 128
    lens = [1500, 1029]
    q = randn((B, hq, d), seed=4)
    kc, vc = randn((B, S, hkv, d), seed=5), randn((B, S, hkv, d), seed=6)
    o = run(q, kc, vc, lens, 1.0 / math.sqrt(d))
    ro, _ = ref(q, kc, vc, lens, 1.0 / math.sqrt(d))
    assert max_abs(o, ro) <= FWD_ATOL


def test_decode_empty_and_single():
    B, hq, hkv, S, d = 3, 4, 2, 64, 64
    lens = [0, 1, 64]
    q = randn((B, hq, d), seed=7)
    kc, vc = randn((B, S, hkv, d), seed=8), randn((B, S, hkv, d), seed=9)
    o, lse = run(q, kc, vc, lens, 0.125, lse=True)
    assert torch.all(o[0] == 0) and torch.all(torch.isneginf(lse[0]))
    torch.testing.assert_close(o[1], vc[1, 0].repeat_interleave(2, dim=0), rtol=0, atol=1e-3)
    ro, _ = ref(q, kc, vc, lens, 0.125)
    assert max_abs(o[2], ro[2]) <= FWD_ATOL


def test_decode_mask_bias():
    B, hq, hkv, S, d = 2, 8, 2, 900, 128
    lens = [900, 517]
    q = randn((B, hq, d), seed=10)
    kc, vc = randn((B, S, hkv, d), seed=11), randn((B, S, hkv, d), seed=12)
    bias = torch.zeros(B, S, device="cuda")
    bias[0, :100] = float("-inf")          # left padding of sequence 0
    bias[1] = randn((S,), seed=13).float()
    o = run(q, kc, vc, lens, 1.0 / math.sqrt(d), bias=bias)
    ro, _ = ref(q, kc, vc, lens, 1.0 / math.sqrt(d), bias=bias)
    assert max_abs(o, ro) <= FWD_ATOL


def test_decode_matches_last_row_of_causal_prefill():
    """The decode step for token n equals row n of causal attention over n+1 tokens."""
    from flash_attn_legacy import flash_attention
    B, hq, hkv, n, d = 2, 8, 2, 777, 128
    q = randn((B, hq, n, d), seed=14)
    k, v = randn((B, hkv, n, d), seed=15), randn((B, hkv, n, d), seed=16)
    full = flash_attention(q, k, v, is_causal=True)
    o = run(q[:, :, -1].contiguous(), k, v, [n] * B, 1.0 / math.sqrt(d), layout="bhsd")
    assert max_abs(o, full[:, :, -1]) <= FWD_ATOL


def c5_inputs(seed=0):
    g = torch.Generator().manual_seed(seed)
    lens = [int(x) for x in torch.randint(1024, 32769, (32,), generator=g)]
    B, hq, hkv, d, S = 32, 32, 8, 128, max(lens)
    q = randn((B, 1, hq, d), seed=seed + 1)
    kc = randn((B, S, hkv, d), seed=seed + 2)
    vc = randn((B, S, hkv, d), seed=seed + 3)
    return lens, q, kc, vc


def test_config_c5():
    """C5 at full size through flash_attn_with_kvcache; 8 sequences against the fp32
    CPU formula and every output finite."""
    from flash_attn_legacy import flash_attn_with_kvcache
    from oracle.torch_ref import ref_decode
    lens, q, kc, vc = c5_inputs()
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    scale = 1.0 / math.sqrt(128)
    o = flash_attn_with_kvcache(q, kc, vc, seq, softmax_scale=scale)
    assert o.shape == q.shape and torch.isfinite(o).all()
    for b in (0, 5, 9, 13, 17, 21, 26, 31):
        r = ref_decode(q[b:b + 1].cpu(), kc[b:b + 1].cpu(), vc[b:b + 1].cpu(), [lens[b]], scale)
        assert max_abs(o[b:b + 1], r) <= FWD_ATOL, b


def test_decode_deterministic():
    """The split kernel merges its waves in a fixed order: repeated calls are bitwise equal."""
    from flash_attn_legacy import hip_ext
    seq = torch.tensor([1, 700, 3000, 129], dtype=torch.int32, device="cuda")
    q = randn((4, 16, 128), seed=8)
    kc, vc = randn((4, 3000, 4, 128), seed=9), randn((4, 3000, 4, 128), seed=10)
    o0, l0 = hip_ext.decode(q, kc, vc, seq, 0.088, return_lse=True)
    for _ in range(5):
        o, l = hip_ext.decode(q, kc, vc, seq, 0.088, return_lse=True)
        assert torch.equal(o, o0) and torch.equal(l, l0)


def test_cache_seqlens_beyond_capacity_are_clamped():
    """cache_seqlens above the cache capacity (or negative) behave as the lengths
    clamped to [0, S]: the kernels clamp on the device and never read past the cache
    or write past the workspace."""
    B, hq, hkv, S, d = 3, 8, 2, 64, 128
    q = randn((B, hq, d), seed=50)
    kc, vc = randn((B, S, hkv, d), seed=51), randn((B, S, hkv, d), seed=52)
    o_g, l_g = run(q, kc, vc, [S, 5, 0], 0.088, lse=True)
    o_b, l_b = run(q, kc, vc, [S + 1000, 5, -3], 0.088, lse=True)
    assert torch.equal(o_g, o_b) and torch.equal(l_g, l_b)


@pytest.mark.parametrize("B", [1, 63, 64, 65, 130])
def test_decode_batch_sizes_both_schedules(B):
    """Batches of up to 64 sequences derive their (sequence, split) items inside the
    split kernel; larger batches take the schedule kernel's list.  Both against the
    oracle, with lengths that give full splits, partial last splits and empty rows."""
    g = torch.Generator().manual_seed(B)
    hq, hkv, d = 8, 2, 64
    lens = [int(x) for x in torch.randint(0, 5000, (B,), generator=g)]
    lens[0] = 4096                       # an exact multiple of the split size
    if B > 2:
        lens[1], lens[2] = 0, 1
    S = max(lens)
    q = randn((B, hq, d), seed=70)
    kc, vc = randn((B, S, hkv, d), seed=71), randn((B, S, hkv, d), seed=72)
    o, lse = run(q, kc, vc, lens, 0.125, lse=True)
    ro, rl = ref(q, kc, vc, lens, 0.125)
    assert max_abs(o, ro) <= FWD_ATOL
    fin = torch.isfinite(rl)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert max_abs(lse.cpu()[fin], rl[fin]) <= 1e-3

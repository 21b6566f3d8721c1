"""Parity at large logits, rows outside every varlen segment, and argument checks.

* Large logits: q, k drawn at 4x and 5x N(0,1) with unit-scale V, so scores reach
  tens of units and the softmax is sharply peaked.  Every score is scaled in fp32
  (the reference scales the fp32 product, flash_attn_fwd_volta.cu:254-266), so the
  forward must stay within 2e-3 of the fp64 oracle and the gradients within 1e-2.
* Varlen backward: rows before the first segment and after the last one belong to
  no sequence; the reference's per-sequence loop leaves them at the zeros it
  starts from (flash_attn.py:125-131).  The library writes those zeros itself, so
  the test first fills the allocator's free blocks with NaN.
* Shape checks of backward / backward_varlen / decode raise RuntimeError before any
  launch (a mismatched tensor would otherwise be read out of bounds).
"""

import math

import numpy as np
import pytest
import torch

from helpers import FWD_ATOL, GRAD_RTOL, cu_from_lens, max_abs, np64, oracle_bwd, oracle_fwd, randn, rel_err
from oracle import attention as orc

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("mag", [4.0, 5.0])
def test_forward_large_logits_unit_v(d, causal, mag):
    from flash_attn_legacy import hip_ext
    B, H, N = 1, 4, 256
    q = randn((B, H, N, d), seed=101, scale=mag)
    k = randn((B, H, N, d), seed=102, scale=mag)
    v = randn((B, H, N, d), seed=103)
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, causal)
    ref_o, ref_l = oracle_fwd(q, k, v, scale, causal)
    err = max_abs(o, ref_o)
    assert err <= FWD_ATOL, f"max |O - O_ref| = {err:.3e}"
    assert max_abs(lse, ref_l) <= 1e-3


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("mag", [4.0, 5.0])
def test_backward_large_logits_unit_v(d, causal, mag):
    from flash_attn_legacy import hip_ext
    B, H, N = 1, 4, 256
    q = randn((B, H, N, d), seed=111, scale=mag)
    k = randn((B, H, N, d), seed=112, scale=mag)
    v = randn((B, H, N, d), seed=113)
    do = randn((B, H, N, d), seed=114)
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, causal)
    got = hip_ext.backward(do, q, k, v, o, lse, scale, causal)
    ref = oracle_bwd(q, k, v, do, scale, causal)
    for name, g, r in zip(("dq", "dk", "dv"), got, ref):
        e = rel_err(g, r)
        assert e <= GRAD_RTOL, f"{name} rel err {e:.3e}"


def _poison_allocator(nbytes: int, device="cuda"):
    """Fill a few free blocks of the caching allocator with NaN, so that a later
    torch.empty of a similar size is likely to return NaN-filled memory."""
    blocks = [torch.full((nbytes // 2 + 64 * i,), float("nan"), dtype=torch.float16, device=device)
              for i in range(6)]
    torch.cuda.synchronize()
    del blocks


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("lead,trail", [(0, 37), (19, 0), (8, 70)])
def test_varlen_backward_rows_outside_segments_are_zero(d, lead, trail):
    from flash_attn_legacy import hip_ext
    lens = [100, 150]
    total = lead + sum(lens) + trail
    hq, hkv = 4, 2
    q = randn((total, hq, d), seed=121, scale=0.5)
    k = randn((total, hkv, d), seed=122, scale=0.5)
    v = randn((total, hkv, d), seed=123)
    do = randn((total, hq, d), seed=124)
    cu = torch.tensor([lead, lead + lens[0], lead + sum(lens)], dtype=torch.int32, device="cuda")
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward_varlen(q, k, v, cu, cu, max(lens), max(lens), scale, True)
    _poison_allocator(total * hq * d * 2)
    dq, dk, dv = hip_ext.backward_varlen(do, q, k, v, o, lse, cu, cu, max(lens), max(lens), scale, True)
    for name, g in (("dq", dq), ("dk", dk), ("dv", dv)):
        outside = torch.cat([g[:lead], g[lead + sum(lens):]])
        assert torch.equal(outside, torch.zeros_like(outside)), f"{name}: rows outside segments not zero"
    ref = orc.varlen_bwd(np64(q), np64(k), np64(v), np64(do), cu.cpu().numpy(), cu.cpu().numpy(), scale, True)
    for name, g, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref):
        e = rel_err(g, torch.from_numpy(r))
        assert e <= GRAD_RTOL, f"{name} rel err {e:.3e}"


def test_varlen_backward_no_sequences_zero_everything():
    from flash_attn_legacy import hip_ext
    total, hq, hkv, d = 40, 2, 1, 64
    q, do = randn((total, hq, d), seed=131), randn((total, hq, d), seed=132)
    k, v = randn((total, hkv, d), seed=133), randn((total, hkv, d), seed=134)
    o = torch.zeros_like(q)
    lse = torch.full((total, hq), float("-inf"), dtype=torch.float32, device="cuda")
    cu = torch.zeros(1, dtype=torch.int32, device="cuda")
    _poison_allocator(total * hq * d * 2)
    for g in hip_ext.backward_varlen(do, q, k, v, o, lse, cu, cu, 0, 0, 0.125, False):
        assert torch.equal(g, torch.zeros_like(g))


def test_backward_shape_checks():
    from flash_attn_legacy import hip_ext
    B, H, N, d = 1, 2, 64, 64
    q, k, v, do = (randn((B, H, N, d), seed=s) for s in (141, 142, 143, 144))
    o, lse = hip_ext.forward(q, k, v, 0.125, False)
    with pytest.raises(RuntimeError):
        hip_ext.backward(do, q, k, v, o, lse[:, :, :32], 0.125, False)          # short L
    with pytest.raises(RuntimeError):
        hip_ext.backward(do, q, k, v, o, lse.double(), 0.125, False)            # L not fp32
    with pytest.raises(RuntimeError):
        hip_ext.backward(do, q, k, v[:, :, :32], o, lse, 0.125, False)          # V != K
    with pytest.raises(RuntimeError):
        hip_ext.backward(do, q, k[..., :32], v[..., :32], o, lse, 0.125, False)  # head dim
    with pytest.raises(RuntimeError):
        hip_ext.backward(do, q, k, v, o[:, :, :32], lse, 0.125, False)          # O != Q
    with pytest.raises(RuntimeError):
        hip_ext.backward(do, q, torch.cat([k, k]), torch.cat([v, v]), o, lse, 0.125, False)   # batch


def test_backward_varlen_checks():
    from flash_attn_legacy import hip_ext
    total, H, d = 96, 2, 64
    q, k, v, do = (randn((total, H, d), seed=s) for s in (151, 152, 153, 154))
    cu = cu_from_lens([40, 56])
    o, lse = hip_ext.forward_varlen(q, k, v, cu, cu, 56, 56, 0.125, True)
    with pytest.raises(RuntimeError):
        hip_ext.backward_varlen(do, q, k, v, o, lse, cu.long(), cu, 56, 56, 0.125, True)
    with pytest.raises(RuntimeError):
        hip_ext.backward_varlen(do, q, k, v, o, lse, cu, cu[:2], 56, 56, 0.125, True)
    with pytest.raises(RuntimeError):
        hip_ext.backward_varlen(do, q, k, v, o, lse[:10], cu, cu, 56, 56, 0.125, True)
    with pytest.raises(RuntimeError):
        hip_ext.backward_varlen(do, q, k, v[:50], o, lse, cu, cu, 56, 56, 0.125, True)


def test_decode_checks():
    from flash_attn_legacy import hip_ext
    B, Hq, Hkv, S, d = 4, 8, 2, 64, 64
    q = randn((B, Hq, d), seed=161)
    kc, vc = randn((B, S, Hkv, d), seed=162), randn((B, S, Hkv, d), seed=163)
    seq = torch.full((B,), S, dtype=torch.int32, device="cuda")
    hip_ext.decode(q, kc, vc, seq, 0.125)
    with pytest.raises(RuntimeError):
        hip_ext.decode(q, kc, vc, seq[:2], 0.125)
    with pytest.raises(RuntimeError):
        hip_ext.decode(q, kc, vc, seq, 0.125, mask_bias=torch.zeros((B, S - 1), device="cuda"))
    with pytest.raises(RuntimeError):
        hip_ext.decode(q, kc, vc, seq, 0.125, mask_bias=torch.zeros((B - 1, S), device="cuda"))
    with pytest.raises(RuntimeError):
        hip_ext.decode(q, kc, vc, seq, 0.125, mask_bias=torch.zeros((S,), device="cuda"))

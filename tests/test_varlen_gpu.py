"""Varlen (packed sequences) parity on the GPU, forward and backward.

Cases follow the reference's TestVarlen (tests/test_flash_attn.py:290-419): per-
sequence oracle, GQA, single sequence equal to the batched path, many short
sequences; plus the benchmark configuration C4 (16 lengths U[64, 4096], 32q/8kv
heads, d=128, causal) and empty / unequal q-k segments.
"""

import math

import numpy as np
import pytest
import torch

from helpers import FWD_ATOL, GRAD_RTOL, cu_from_lens, max_abs, np64, randn, rel_err
from oracle import attention as orc

pytestmark = pytest.mark.gpu


def varlen(q, k, v, cu_q, cu_k, mq, mk, scale, causal):
    from flash_attn_legacy import flash_attn_varlen_func
    return flash_attn_varlen_func(q, k, v, cu_q, cu_k, mq, mk, softmax_scale=scale, causal=causal)


def fwd_check(lens_q, lens_k, hq, hkv, d, causal, seed=0):
    tq, tk = sum(lens_q), sum(lens_k)
    q = randn((tq, hq, d), seed=seed)
    k = randn((tk, hkv, d), seed=seed + 1)
    v = randn((tk, hkv, d), seed=seed + 2)
    cu_q, cu_k = cu_from_lens(lens_q), cu_from_lens(lens_k)
    scale = 1.0 / math.sqrt(d)
    from flash_attn_legacy import hip_ext
    o, lse = hip_ext.forward_varlen(q, k, v, cu_q, cu_k, max(lens_q), max(lens_k), scale, causal)
    ref_o, ref_lse = orc.varlen_fwd(np64(q), np64(k), np64(v), cu_q.cpu().numpy(), cu_k.cpu().numpy(),
                                    scale, causal)
    assert o.shape == (tq, hq, d) and lse.shape == (tq, hq)
    assert max_abs(o, torch.from_numpy(ref_o)) <= FWD_ATOL
    fin = np.isfinite(ref_lse)
    assert np.array_equal(np.isfinite(lse.cpu().numpy()), fin)
    assert float(np.abs(lse.cpu().numpy()[fin] - ref_lse[fin]).max(initial=0)) <= 1e-3


@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_varlen_correctness(d, causal):
    fwd_check([32, 64, 48], [32, 64, 48], 4, 4, d, causal)


@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
def test_varlen_gqa(d):
    fwd_check([64, 32], [64, 32], 8, 2, d, True)


def test_varlen_single_sequence_matches_batched():
    from flash_attn_legacy import flash_attention
    H, N, d = 4, 128, 64
    q, k, v = (randn((N, H, d), seed=s, scale=0.3) for s in (1, 2, 3))
    cu = cu_from_lens([N])
    out_varlen = varlen(q, k, v, cu, cu, N, N, 1.0 / math.sqrt(d), True)
    qb, kb, vb = (t.permute(1, 0, 2).unsqueeze(0) for t in (q, k, v))
    out_batch = flash_attention(qb, kb, vb, softmax_scale=1.0 / math.sqrt(d), is_causal=True)
    torch.testing.assert_close(out_varlen, out_batch.squeeze(0).permute(1, 0, 2), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("causal", [False, True])
def test_many_short_and_empty_segments(causal):
    fwd_check([16, 8, 32, 4, 24, 0, 1, 300, 129], [16, 8, 32, 4, 24, 0, 1, 300, 129], 2, 1, 64, causal)


@pytest.mark.parametrize("causal", [False, True])
def test_unequal_q_k_segments(causal):
    fwd_check([10, 70, 130], [140, 33, 130], 4, 2, 128, causal)


@pytest.mark.parametrize("nseq", [63, 64, 65, 130])
@pytest.mark.parametrize("causal", [False, True])
def test_work_items_on_both_sides_of_64_sequences(nseq, causal):
    """Up to 64 sequences (and 16384 query tokens) each forward workgroup derives its
    (sequence, tile) item from cu_seqlens; more use the schedule kernel's list.  Lengths
    repeat (equal tile counts are ordered by index) and include empty segments and
    segments of several tiles."""
    g = torch.Generator().manual_seed(nseq)
    lens = [int(x) for x in torch.randint(0, 40, (nseq,), generator=g)]
    lens[::7] = [0] * len(lens[::7])
    lens[3] = 300
    lens[nseq // 2] = 257
    fwd_check(lens, lens, 2, 1, 64, causal, seed=nseq)


def bwd_check(lens_q, lens_k, hq, hkv, d, causal, seed=0):
    tq, tk = sum(lens_q), sum(lens_k)
    q = randn((tq, hq, d), seed=seed)
    k = randn((tk, hkv, d), seed=seed + 1)
    v = randn((tk, hkv, d), seed=seed + 2)
    do = randn((tq, hq, d), seed=seed + 3)
    cu_q, cu_k = cu_from_lens(lens_q), cu_from_lens(lens_k)
    scale = 1.0 / math.sqrt(d)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    varlen(qg, kg, vg, cu_q, cu_k, max(lens_q), max(lens_k), scale, causal).backward(do)
    ref = orc.varlen_bwd(np64(q), np64(k), np64(v), np64(do), cu_q.cpu().numpy(), cu_k.cpu().numpy(),
                         scale, causal)
    for name, g, r in zip(("dq", "dk", "dv"), (qg.grad, kg.grad, vg.grad), ref):
        e = rel_err(g, torch.from_numpy(r))
        assert e <= GRAD_RTOL, f"{name} rel err {e:.3e}"


@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_varlen_backward(d, causal):
    bwd_check([32, 64, 48, 1], [32, 64, 48, 1], 4, 2, d, causal)


def test_varlen_backward_unequal_segments():
    bwd_check([10, 70, 0, 130], [140, 33, 5, 130], 4, 2, 64, True)


def c4_lengths(seed=0):
    g = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(64, 4097, (16,), generator=g)]


def test_config_c4_forward():
    """C4 forward at full size; every sequence's heads of KV group 0 and 7 against the
    fp32 CPU formula."""
    from oracle.torch_ref import ref_attention
    lens = c4_lengths()
    tot, hq, hkv, d = sum(lens), 32, 8, 128
    q = randn((tot, hq, d), seed=0)
    k = randn((tot, hkv, d), seed=1)
    v = randn((tot, hkv, d), seed=2)
    cu = cu_from_lens(lens)
    scale = 1.0 / math.sqrt(d)
    o = varlen(q, k, v, cu, cu, max(lens), max(lens), scale, True)
    assert torch.isfinite(o).all()
    torch.set_num_threads(max(torch.get_num_threads(), 8))
    c = cu.cpu().tolist()
    for i in range(len(lens)):
        for g in (0, hkv - 1):
            hs = slice(g * 4, g * 4 + 4)
            qi = q[c[i]:c[i + 1], hs].permute(1, 0, 2)[None].cpu()
            ki = k[c[i]:c[i + 1], g:g + 1].permute(1, 0, 2)[None].cpu()
            vi = v[c[i]:c[i + 1], g:g + 1].permute(1, 0, 2)[None].cpu()
            ref = ref_attention(qi, ki, vi, scale, True)[0].permute(1, 0, 2)
            assert max_abs(o[c[i]:c[i + 1], hs], ref) <= FWD_ATOL, (i, g)


def _list_lengths(n, lo, hi, seed):
    g = torch.Generator().manual_seed(seed)
    return [int(x) for x in torch.randint(lo, hi + 1, (n,), generator=g)]


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("hq,hkv", [(8, 2), (16, 2)])
def test_four_heads_pair_walk(causal, hq, hkv):
    """Head dim 128 with Hq/Hkv a multiple of 4 and a work list (more than 64 sequences):
    each workgroup walks the query tiles nt-1-j and j of one sequence.  Lengths of 1,
    63, 64, 65 and 129 rows give tile counts of 1 (a lone tile), odd and even; O and L
    of every row against the float64 oracle."""
    lens = _list_lengths(66, 1, 400, seed=90) + [1, 63, 64, 65, 129]
    fwd_check(lens, lens, hq, hkv, 128, causal, seed=91)


@pytest.mark.parametrize("causal", [True, False])
def test_four_heads_pair_walk_unequal_segments(causal):
    """The pair walk with query and key segments of different lengths (top-left causal
    alignment within each sequence, empty query and key segments)."""
    lq = _list_lengths(70, 0, 300, seed=92)
    lk = [max(0, n + d) for n, d in zip(lq, _list_lengths(70, -40, 120, seed=93))]
    fwd_check(lq, lk, 8, 2, 128, causal, seed=94)


def test_config_c4_backward():
    """C4 lengths (16 sequences of U[64, 4096] tokens), 32/8 heads, d=128, causal: the
    native one-launch varlen backward against the per-sequence semantics of the
    reference's loop (flash_attn_legacy/flash_attn.py:133-157; dK/dV of a sequence come
    from its own rows only).  dQ, dK and dV of KV groups 0, 3 and 7 of every sequence
    against the CPU oracle's fp32 autograd, L and O from this library's forward."""
    from oracle.torch_ref import ref_backward
    lens = c4_lengths()
    tot, hq, hkv, d = sum(lens), 32, 8, 128
    q, k, v, do = (randn((tot, h, d), seed=s) for s, h in ((0, hq), (1, hkv), (2, hkv), (3, hq)))
    cu = cu_from_lens(lens)
    scale = 1.0 / math.sqrt(d)
    qg, kg, vg = (t.clone().requires_grad_(True) for t in (q, k, v))
    varlen(qg, kg, vg, cu, cu, max(lens), max(lens), scale, True).backward(do)
    dq, dk, dv = (t.grad.cpu() for t in (qg, kg, vg))
    for t in (dq, dk, dv):
        assert torch.isfinite(t).all()
    torch.set_num_threads(max(torch.get_num_threads(), 8))
    c = cu.cpu().tolist()
    sw = lambda x: x.permute(1, 0, 2)[None].cpu()
    for i in range(len(lens)):
        r = slice(c[i], c[i + 1])
        for g in (0, 3, hkv - 1):
            hs, gs = slice(g * 4, g * 4 + 4), slice(g, g + 1)
            ref = ref_backward(sw(q[r, hs]), sw(k[r, gs]), sw(v[r, gs]), sw(do[r, hs]), scale, True)
            for name, got, rg in zip(("dq", "dk", "dv"), (dq[r, hs], dk[r, gs], dv[r, gs]), ref):
                e = rel_err(got, rg[0].permute(1, 0, 2))
                assert e <= GRAD_RTOL, (name, i, g, e)


@pytest.mark.parametrize("d", [96, 128])
def test_malformed_cu_seqlens_are_clamped(d):
    """A cu_seqlens array past the packed tensor (last entry total + 50, a second
    entry beyond it too) behaves as the array clamped to [0, total]: the kernels
    clamp every segment on the device, so no row outside the tensor is touched.
    Forward and backward must equal the well-formed call bit for bit."""
    from flash_attn_legacy import hip_ext
    lens = [100, 157]
    total = sum(lens)
    q, k, v = randn((total, 4, d), seed=40), randn((total, 2, d), seed=41), randn((total, 2, d), seed=42)
    do = randn((total, 4, d), seed=43)
    good = cu_from_lens(lens)
    bad = torch.tensor([0, 100, total + 50], dtype=torch.int32, device="cuda")
    scale = 1.0 / math.sqrt(d)
    for causal in (False, True):
        o_g, l_g = hip_ext.forward_varlen(q, k, v, good, good, max(lens), max(lens), scale, causal)
        o_b, l_b = hip_ext.forward_varlen(q, k, v, bad, bad, 207, 207, scale, causal)
        assert torch.equal(o_g, o_b) and torch.equal(l_g, l_b)
        g_g = hip_ext.backward_varlen(do, q, k, v, o_g, l_g, good, good, max(lens), max(lens), scale, causal)
        g_b = hip_ext.backward_varlen(do, q, k, v, o_g, l_g, bad, bad, 207, 207, scale, causal)
        for a, b in zip(g_g, g_b):
            assert torch.equal(a, b)

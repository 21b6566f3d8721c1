"""Backward parity on the GPU: dQ/dK/dV from the HIP kernels against the oracle.

Cases follow the reference's TestBackwardMHA (tests/test_flash_attn.py:200-234),
TestBackwardGQA (:241-279) and TestLongSequences.test_long_seq_backward
(:519-541) with seeded inputs; the bound is the relative error
max|g - g_ref| / max|g_ref| <= 1e-2 per gradient against the fp64 oracle
(which recomputes P from the closed-form LSE, oracle/attention.py).
"""

import math

import numpy as np

import pytest
import torch

from helpers import GRAD_RTOL, np64, oracle_bwd, randn, rel_err

pytestmark = pytest.mark.gpu

HEAD_DIMS = [32, 64, 96, 128, 256]


def run_fa(q, k, v, do, scale, causal):
    from flash_attn_legacy import flash_attention
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    flash_attention(q, k, v, softmax_scale=scale, is_causal=causal).backward(do)
    return q.grad, k.grad, v.grad


def check(q, k, v, do, scale, causal):
    got = run_fa(q, k, v, do, scale, causal)
    ref = oracle_bwd(q, k, v, do, scale, causal)
    for name, g, r in zip(("dq", "dk", "dv"), got, ref):
        assert g.shape == r.shape, name
        e = rel_err(g, r)
        assert e <= GRAD_RTOL, f"{name} rel err {e:.3e}"


@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("causal", [False, True])
def test_gradient_flow(d, causal):
    q, k, v = (randn((1, 2, 64, d), seed=s) for s in (1, 2, 3))
    dq, dk, dv = run_fa(q, k, v, torch.ones_like(q), 1.0 / math.sqrt(d), causal)
    for g in (dq, dk, dv):
        assert g is not None and not torch.all(g == 0)


@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N", [32, 64, 128, 200])
def test_gradient_correctness(d, causal, N):
    q, k, v = (randn((1, 2, N, d), seed=s, scale=0.5) for s in (4, 5, 6))
    do = randn((1, 2, N, d), seed=7)
    check(q, k, v, do, 1.0 / math.sqrt(d), causal)


@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("hq,hkv", [(8, 2), (4, 1)])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa_gradients(d, hq, hkv, causal):
    N = 96
    q = randn((1, hq, N, d), seed=8)
    k, v = (randn((1, hkv, N, d), seed=s) for s in (9, 10))
    do = randn((1, hq, N, d), seed=11)
    check(q, k, v, do, 1.0 / math.sqrt(d), causal)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("N", [1024, 2048])
def test_long_seq_backward(d, N):
    q, k, v, do = (randn((1, 2, N, d), seed=s) for s in (12, 13, 14, 15))
    check(q, k, v, do, 1.0 / math.sqrt(d), True)


@pytest.mark.parametrize("nq,nk", [(64, 200), (200, 64)])
@pytest.mark.parametrize("causal", [False, True])
def test_unequal_lengths(nq, nk, causal):
    d = 64
    q = randn((2, 4, nq, d), seed=16)
    k, v = (randn((2, 2, nk, d), seed=s) for s in (17, 18))
    do = randn((2, 4, nq, d), seed=19)
    check(q, k, v, do, 0.125, causal)


def test_strided_grad_output():
    d, N = 64, 128
    q, k, v = (randn((2, 4, N, d), seed=s) for s in (20, 21, 22))
    do = randn((2, N, 4, d), seed=23).transpose(1, 2)
    check(q, k, v, do, 0.125, True)


def test_config_c3():
    """C3: B=2, H=16, N=2048, d=128, causal; all of dQ/dK/dV against the fp32
    CPU autograd of the closed form (the reference's ref_backward formula)."""
    from oracle.torch_ref import ref_backward
    B, H, N, d = 2, 16, 2048, 128
    q, k, v, do = (randn((B, H, N, d), seed=s) for s in (0, 1, 2, 3))
    got = run_fa(q, k, v, do, 1.0 / math.sqrt(d), True)
    torch.set_num_threads(max(torch.get_num_threads(), 8))
    for b in range(B):
        for h0 in range(0, H, 4):
            sl = (slice(b, b + 1), slice(h0, h0 + 4))
            ref = ref_backward(q[sl].cpu(), k[sl].cpu(), v[sl].cpu(), do[sl].cpu(), 1.0 / math.sqrt(d), True)
            for name, g, r in zip(("dq", "dk", "dv"), got, ref):
                e = rel_err(g[sl], r)
                assert e <= GRAD_RTOL, f"{name} b={b} h0={h0} rel err {e:.3e}"


@pytest.mark.parametrize("d", [32, 64, 96, 128])
def test_deterministic_gradients(d):
    """d 64/128 take the split backward (no atomics): repeated calls are bitwise equal."""
    from flash_attn_legacy import hip_ext
    q, k, v, do = (randn((2, 8, 300, d), seed=s) for s in (31, 32, 33, 34))
    o, lse = hip_ext.forward(q, k, v, 0.1, True)
    g0 = hip_ext.backward(do, q, k, v, o, lse, 0.1, True)
    for _ in range(3):
        g = hip_ext.backward(do, q, k, v, o, lse, 0.1, True)
        for a, b in zip(g, g0):
            assert torch.equal(a, b)


def test_long_sequence_sampled_gradients():
    """N = 16384, causal, 2 query heads per KV head: sampled rows of dQ against float64
    rows computed from that row alone (O, L, D, P, dP, dS over all its keys), and
    sampled rows of dK / dV against float64 sums over every query row that sees the key
    (those sums take each row's L and D from the kernel's forward L and O, whose sampled
    rows are themselves checked in test_fwd_gpu.py)."""
    from flash_attn_legacy import hip_ext
    Hq, Hkv, N, d = 2, 1, 16384, 128
    scale = 1.0 / math.sqrt(d)
    q = randn((1, Hq, N, d), seed=70)
    k, v = randn((1, Hkv, N, d), seed=71), randn((1, Hkv, N, d), seed=72)
    do = randn((1, Hq, N, d), seed=73)
    o, lse = hip_ext.forward(q, k, v, scale, True)
    dq, dk, dv = hip_ext.backward(do, q, k, v, o, lse, scale, True)
    qf, kf, vf, dof, of = (np64(t)[0] for t in (q, k, v, do, o))
    lf = lse[0].double().cpu().numpy()
    kk, vv = kf[0], vf[0]
    rows = [0, 5, 4095, 8191, 12000, N - 1]
    for h in range(Hq):
        ref = []
        for r in rows:
            s = kk[: r + 1] @ qf[h, r] * scale
            m = s.max()
            p = np.exp(s - m)
            L = m + np.log(p.sum())
            p = np.exp(s - L)
            orow = p @ vv[: r + 1]
            dp = vv[: r + 1] @ dof[h, r]
            ds = p * (dp - dof[h, r] @ orow)
            ref.append(scale * ds @ kk[: r + 1])
        assert rel_err(dq[0, h, rows], torch.from_numpy(np.stack(ref))) <= GRAD_RTOL, h
    keys = [0, 7, 4096, 10000, N - 2, N - 1]
    dk_ref, dv_ref = [], []
    for j in keys:
        gk, gv = np.zeros(d), np.zeros(d)
        for h in range(Hq):
            qq, gg = qf[h, j:], dof[h, j:]
            p = np.exp(qq @ kk[j] * scale - lf[h, j:])
            dp = gg @ vv[j]
            dd = np.einsum("rd,rd->r", gg, of[h, j:])
            gk += scale * (p * (dp - dd)) @ qq
            gv += p @ gg
        dk_ref.append(gk)
        dv_ref.append(gv)
    assert rel_err(dk[0, 0, keys], torch.from_numpy(np.stack(dk_ref))) <= GRAD_RTOL
    assert rel_err(dv[0, 0, keys], torch.from_numpy(np.stack(dv_ref))) <= GRAD_RTOL


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,Hq,Hkv,N", [(2, 16, 16, 4096), (1, 32, 8, 4160)])
def test_large_grid_every_head(B, Hq, Hkv, N, causal):
    """head_dim 128 backward on grids of several workgroups per CU (pipelined dQ and dK/dV
    kernels; an odd tile count leaves one query tile unpaired): every gradient of every
    head against the CPU oracle's fp32 autograd (tests/test_flash_attn.py:35-58)."""
    from oracle.torch_ref import ref_backward
    torch.set_num_threads(max(torch.get_num_threads(), 8))
    d = 128
    scale = 1.0 / math.sqrt(d)
    q, do = randn((B, Hq, N, d), seed=31), randn((B, Hq, N, d), seed=34)
    k, v = randn((B, Hkv, N, d), seed=32), randn((B, Hkv, N, d), seed=33)
    dq, dk, dv = run_fa(q, k, v, do, scale, causal)
    G = Hq // Hkv
    for b in range(B):
        for g in range(Hkv):
            hs = slice(g * G, (g + 1) * G)
            ref = ref_backward(q[b:b + 1, hs].cpu(), k[b:b + 1, g:g + 1].cpu(), v[b:b + 1, g:g + 1].cpu(),
                               do[b:b + 1, hs].cpu(), scale, causal)
            for name, got, r in zip(("dq", "dk", "dv"), (dq[b:b + 1, hs], dk[b:b + 1, g:g + 1],
                                                           dv[b:b + 1, g:g + 1]), ref):
                assert rel_err(got, r) <= GRAD_RTOL, (name, b, g)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,Hq,Hkv,N", [(2, 4, 4, 200), (2, 8, 2, 333), (1, 8, 2, 1000)])
def test_negative_scale_head_dim_128(B, Hq, Hkv, N, causal):
    """A negative softmax scale through the pipelined head-dim-128 backward (its
    accumulators start at -L*log2(e)/c with c of either sign, masked scores take the
    value whose product with c is -inf): MHA and GQA, row counts that are not a
    multiple of 64, against the float64 oracle."""
    d = 128
    q, do = randn((B, Hq, N, d), seed=81), randn((B, Hq, N, d), seed=84)
    k, v = randn((B, Hkv, N, d), seed=82), randn((B, Hkv, N, d), seed=83)
    check(q, k, v, do, -1.0 / math.sqrt(d), causal)

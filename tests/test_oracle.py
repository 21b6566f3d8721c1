"""Pins the CPU oracle (oracle/attention.py, oracle/torch_ref.py) -- CPU only.

The oracle is only trusted because each function is checked here against
something that is not a retyping of its own formula:

* float64 torch autograd of the closed form (an independent implementation, used
  for the forward, the backward and the GQA reduction);
* brute-force scalar Python loops on tiny inputs (forward and LSE);
* central finite differences of a scalar loss (backward);
* the closed forms the reference's tests rely on: N=1 gives O=V, Q=K=0 gives
  mean(V) (prefix means when causal), causal row 0 gives V[0], MQA equals
  broadcast K/V, single-segment varlen equals batched
  (reference tests/test_flash_attn.py:104-193,356-378,645-656);
* decode equals the last row of causal attention over the same prefix.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as orc
from oracle import torch_ref

RNG = np.random.default_rng(1234)


def rnd(*shape):
    return RNG.standard_normal(shape)


def torch_closed_form(q, k, v, scale, causal):
    """float64 torch: softmax(QK^T*scale + top-left mask) V with GQA by repeat."""
    q, k, v = (torch.as_tensor(x, dtype=torch.float64) for x in (q, k, v))
    rep = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(rep, dim=1)
    v = v.repeat_interleave(rep, dim=1)
    s = q @ k.transpose(-1, -2) * scale
    if causal:
        m = torch.ones(q.shape[2], k.shape[2], dtype=torch.bool).triu(1)
        s = s.masked_fill(m, float("-inf"))
    return torch.softmax(s, -1) @ v, torch.logsumexp(s, -1)


@pytest.mark.parametrize("hq,hkv", [(2, 2), (4, 2), (4, 1)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("nq,nk", [(7, 7), (5, 9), (9, 5), (1, 6)])
def test_forward_matches_torch_float64(hq, hkv, causal, nq, nk):
    q, k, v = rnd(2, hq, nq, 8), rnd(2, hkv, nk, 8), rnd(2, hkv, nk, 8)
    o, lse = orc.attention_fwd(q, k, v, 0.37, causal)
    ro, rl = torch_closed_form(q, k, v, 0.37, causal)
    np.testing.assert_allclose(o, ro.numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(lse, rl.numpy(), rtol=1e-12, atol=1e-12)


def test_forward_brute_force_loops():
    q, k, v = rnd(1, 2, 4, 3), rnd(1, 1, 5, 3), rnd(1, 1, 5, 3)
    scale = 0.8
    for causal in (False, True):
        o, lse = orc.attention_fwd(q, k, v, scale, causal)
        for h in range(2):
            for i in range(4):
                keys = [j for j in range(5) if not (causal and j > i)]
                s = [scale * sum(q[0, h, i, t] * k[0, 0, j, t] for t in range(3)) for j in keys]
                mx = max(s)
                e = [math.exp(x - mx) for x in s]
                den = sum(e)
                for t in range(3):
                    ref = sum(e[a] * v[0, 0, j, t] for a, j in enumerate(keys)) / den
                    assert abs(o[0, h, i, t] - ref) < 1e-12
                assert abs(lse[0, h, i] - (mx + math.log(den))) < 1e-12


def test_closed_forms():
    v = rnd(2, 3, 1, 8)
    o, _ = orc.attention_fwd(rnd(2, 3, 1, 8), rnd(2, 3, 1, 8), v, 0.3, False)
    np.testing.assert_allclose(o, v)                                   # N=1 -> O=V
    z = np.zeros((1, 2, 6, 4))
    v = rnd(1, 2, 6, 4)
    o, lse = orc.attention_fwd(z, z, v, 0.5, False)
    np.testing.assert_allclose(o, np.broadcast_to(v.mean(2, keepdims=True), o.shape))
    np.testing.assert_allclose(lse, np.full(lse.shape, math.log(6)))   # uniform -> log N
    o, _ = orc.attention_fwd(z, z, v, 0.5, True)
    prefix = np.cumsum(v, axis=2) / np.arange(1, 7)[None, None, :, None]
    np.testing.assert_allclose(o, prefix)                              # causal -> prefix means
    q, k = rnd(1, 2, 6, 4), rnd(1, 2, 6, 4)
    o, _ = orc.attention_fwd(q, k, v, 0.5, True)
    np.testing.assert_allclose(o[:, :, 0], v[:, :, 0])                 # causal row 0 = V[0]


def test_mqa_equals_broadcast():
    q, k, v = rnd(2, 4, 5, 8), rnd(2, 1, 5, 8), rnd(2, 1, 5, 8)
    a, _ = orc.attention_fwd(q, k, v, 0.4, True)
    b, _ = orc.attention_fwd(q, np.repeat(k, 4, 1), np.repeat(v, 4, 1), 0.4, True)
    np.testing.assert_allclose(a, b)


def test_empty_keys_give_zero_and_neg_inf():
    o, lse = orc.attention_fwd(rnd(1, 1, 3, 4), np.zeros((1, 1, 0, 4)), np.zeros((1, 1, 0, 4)), 1.0, False)
    assert np.all(o == 0) and np.all(np.isneginf(lse))


@pytest.mark.parametrize("hq,hkv", [(2, 2), (4, 2)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("nq,nk", [(6, 6), (4, 7)])
def test_backward_matches_torch_autograd(hq, hkv, causal, nq, nk):
    q, k, v, do = rnd(2, hq, nq, 8), rnd(2, hkv, nk, 8), rnd(2, hkv, nk, 8), rnd(2, hq, nq, 8)
    dq, dk, dv = orc.attention_bwd(q, k, v, do, 0.45, causal)
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    o, _ = torch_closed_form(qt, kt, vt, 0.45, causal)
    o.backward(torch.tensor(do))
    np.testing.assert_allclose(dq, qt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dk, kt.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dv, vt.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_backward_finite_differences():
    q, k, v, g = rnd(1, 2, 5, 3), rnd(1, 1, 5, 3), rnd(1, 1, 5, 3), rnd(1, 2, 5, 3)
    scale, causal, eps = 0.7, True, 1e-6
    grads = orc.attention_bwd(q, k, v, g, scale, causal)

    def loss(q_, k_, v_):
        o, _ = orc.attention_fwd(q_, k_, v_, scale, causal)
        return float((o * g).sum())

    for which, x in enumerate((q, k, v)):
        for idx in [(0, 0, 1, 2), (0, 0, 4, 0), (0, 0, 3, 1)]:
            if which > 0:
                idx = (0, 0) + idx[2:]
            xp, xm = x.copy(), x.copy()
            xp[idx] += eps
            xm[idx] -= eps
            args_p = [q, k, v]
            args_m = [q, k, v]
            args_p[which], args_m[which] = xp, xm
            fd = (loss(*args_p) - loss(*args_m)) / (2 * eps)
            assert abs(fd - grads[which][idx]) < 1e-6, (which, idx)


def test_varlen_forward_equals_per_segment_and_batched():
    lens = [3, 0, 5, 1]
    cu = np.concatenate([[0], np.cumsum(lens)])
    q, k, v = rnd(cu[-1], 4, 8), rnd(cu[-1], 2, 8), rnd(cu[-1], 2, 8)
    for causal in (False, True):
        o, lse = orc.varlen_fwd(q, k, v, cu, cu, 0.3, causal)
        for s, e in zip(cu[:-1], cu[1:]):
            if e == s:
                continue
            ro, rl = torch_closed_form(q[s:e].transpose(1, 0, 2)[None], k[s:e].transpose(1, 0, 2)[None],
                                       v[s:e].transpose(1, 0, 2)[None], 0.3, causal)
            np.testing.assert_allclose(o[s:e], ro.numpy()[0].transpose(1, 0, 2), atol=1e-12)
            np.testing.assert_allclose(lse[s:e], rl.numpy()[0].T, atol=1e-12)
    # single segment == batched
    cu1 = np.array([0, 9])
    q, k, v = rnd(9, 2, 4), rnd(9, 2, 4), rnd(9, 2, 4)
    a, _ = orc.varlen_fwd(q, k, v, cu1, cu1, 0.5, True)
    b, _ = orc.attention_fwd(q.transpose(1, 0, 2)[None], k.transpose(1, 0, 2)[None], v.transpose(1, 0, 2)[None],
                             0.5, True)
    np.testing.assert_allclose(a, b[0].transpose(1, 0, 2))


def test_varlen_backward_matches_packed_autograd():
    lens_q, lens_k = [3, 4, 2], [5, 4, 3]
    cq, ck = np.concatenate([[0], np.cumsum(lens_q)]), np.concatenate([[0], np.cumsum(lens_k)])
    q, k, v, do = rnd(cq[-1], 4, 8), rnd(ck[-1], 2, 8), rnd(ck[-1], 2, 8), rnd(cq[-1], 4, 8)
    dq, dk, dv = orc.varlen_bwd(q, k, v, do, cq, ck, 0.6, True)
    qt, kt, vt = (torch.tensor(x, requires_grad=True) for x in (q, k, v))
    outs = []
    for i in range(3):
        sl_q, sl_k = slice(cq[i], cq[i + 1]), slice(ck[i], ck[i + 1])
        o, _ = torch_closed_form(qt[sl_q].transpose(0, 1)[None], kt[sl_k].transpose(0, 1)[None],
                                 vt[sl_k].transpose(0, 1)[None], 0.6, True)
        outs.append(o[0].transpose(0, 1))
    torch.cat(outs).backward(torch.tensor(do))
    np.testing.assert_allclose(dq, qt.grad.numpy(), atol=1e-12)
    np.testing.assert_allclose(dk, kt.grad.numpy(), atol=1e-12)
    np.testing.assert_allclose(dv, vt.grad.numpy(), atol=1e-12)


def test_decode_is_last_row_of_causal_prefix_and_applies_bias():
    B, hq, hkv, S, d = 3, 4, 2, 9, 8
    lens = [9, 4, 1]
    kc, vc = rnd(B, S, hkv, d), rnd(B, S, hkv, d)
    q = rnd(B, 1, hq, d)
    o, lse = orc.decode(q, kc, vc, lens, 0.35)
    for b, n in enumerate(lens):
        ro, rl = torch_closed_form(q[b, 0][None, :, None], kc[b, :n].transpose(1, 0, 2)[None],
                                   vc[b, :n].transpose(1, 0, 2)[None], 0.35, False)
        np.testing.assert_allclose(o[b, 0], ro.numpy()[0, :, 0], atol=1e-12)
        np.testing.assert_allclose(lse[b], rl.numpy()[0, :, 0], atol=1e-12)
    bias = rnd(B, S)
    bias[0, :3] = -np.inf
    o2, _ = orc.decode(q, kc, vc, lens, 0.35, bias=bias)
    for b, n in enumerate(lens):
        qt = torch.tensor(q[b, 0])
        kt = torch.tensor(kc[b, :n]).repeat_interleave(2, dim=1)
        vt = torch.tensor(vc[b, :n]).repeat_interleave(2, dim=1)
        s = torch.einsum("hd,nhd->hn", qt, kt) * 0.35 + torch.tensor(bias[b, :n])
        ref = torch.einsum("hn,nhd->hd", torch.softmax(s, -1), vt)
        np.testing.assert_allclose(o2[b, 0], ref.numpy(), atol=1e-12)


def test_torch_fp32_reference_agrees_with_float64_oracle():
    q = torch.randn(1, 4, 33, 16, generator=torch.Generator().manual_seed(3))
    k = torch.randn(1, 2, 33, 16, generator=torch.Generator().manual_seed(4))
    v = torch.randn(1, 2, 33, 16, generator=torch.Generator().manual_seed(5))
    for causal in (False, True):
        a = torch_ref.ref_attention(q, k, v, 0.25, causal)
        b, _ = orc.attention_fwd(q.numpy(), k.numpy(), v.numpy(), 0.25, causal)
        np.testing.assert_allclose(a.numpy(), b, atol=1e-5)
        o2, l2 = torch_ref.ref_attention_lse(q, k, v, 0.25, causal)
        b2, lb = orc.attention_fwd(q.numpy(), k.numpy(), v.numpy(), 0.25, causal)
        np.testing.assert_allclose(o2.numpy(), b2, atol=1e-5)
        np.testing.assert_allclose(l2.numpy(), lb, atol=1e-5)
    # L is the natural-log logsumexp of the scaled scores; Nq > Nk leaves no causal row
    # without a key, Nq < Nk under a causal mask checks the top-left alignment
    q2 = torch.randn(1, 2, 9, 16, generator=torch.Generator().manual_seed(7))
    _, l3 = torch_ref.ref_attention_lse(q2, k[:, :, :5], v[:, :, :5], 0.25, True)
    s3 = torch.einsum("hqd,hkd->hqk", q2[0].double(), k[0, :, :5].double().repeat_interleave(1, 0)) * 0.25
    for r in range(9):
        ref = torch.logsumexp(s3[:, r, : min(r + 1, 5)], dim=-1)
        np.testing.assert_allclose(l3[0, :, r].numpy(), ref.numpy(), atol=1e-5)
    do = torch.randn(1, 4, 33, 16, generator=torch.Generator().manual_seed(6))
    ga = torch_ref.ref_backward(q, k, v, do, 0.25, True)
    gb = orc.attention_bwd(q.numpy(), k.numpy(), v.numpy(), do.numpy(), 0.25, True)
    for x, y in zip(ga, gb):
        np.testing.assert_allclose(x.numpy(), y, atol=1e-4)


def test_gqa_gradients_are_group_sums_of_mha_gradients():
    """GQA backward == MHA backward on K/V repeated per group, with dK/dV summed over
    the query heads of each group (the reference's in-block group loop,
    csrc/kernels/flash_attn_bwd.cu:496)."""
    hq, hkv, n, d = 6, 2, 7, 5
    q, k, v, do = rnd(1, hq, n, d), rnd(1, hkv, n, d), rnd(1, hkv, n, d), rnd(1, hq, n, d)
    g = hq // hkv
    dq, dk, dv = orc.attention_bwd(q, k, v, do, 0.4, True)
    mq, mk, mv = orc.attention_bwd(q, np.repeat(k, g, axis=1), np.repeat(v, g, axis=1), do, 0.4, True)
    np.testing.assert_allclose(dq, mq, atol=1e-12)
    np.testing.assert_allclose(dk, mk.reshape(1, hkv, g, n, d).sum(2), atol=1e-12)
    np.testing.assert_allclose(dv, mv.reshape(1, hkv, g, n, d).sum(2), atol=1e-12)


def test_decode_single_row_cache_returns_that_row():
    """A cache of length 1 gives O = V[0] and L = q.k*scale, whatever q is."""
    kc, vc, q = rnd(2, 5, 1, 4), rnd(2, 5, 1, 4), rnd(2, 1, 3, 4) * 10
    o, lse = orc.decode(q, kc, vc, [1, 1], 0.7)
    for b in range(2):
        np.testing.assert_allclose(o[b, 0], np.repeat(vc[b, 0], 3, axis=0), atol=1e-12)
        np.testing.assert_allclose(lse[b], q[b, 0] @ kc[b, 0, 0] * 0.7, atol=1e-12)

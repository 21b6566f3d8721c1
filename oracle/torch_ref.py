"""fp32 PyTorch attention on the host CPU -- the reference's own oracle formula.

TEST INFRASTRUCTURE ONLY (used by ``tests/`` and ``bench.py``'s ``cpu_baseline``
leg, never by the product).  Restates ``ref_attention`` / ``ref_backward`` of the
reference's ``tests/test_flash_attn.py:19-58`` on CPU tensors, plus the eager
decode branch of ``flash_attn_legacy/integrations.py:77-98``.  Pinned against the
float64 numpy oracle in ``tests/test_oracle.py``.
"""

from __future__ import annotations

import torch


def ref_attention(q, k, v, scale, is_causal=False):
    """fp32 ``softmax(QK^T*scale + top-left mask) V``; GQA by ``repeat_interleave``
    (``tests/test_flash_attn.py:19-32``).  Returns fp32 (no fp16 round-trip)."""
    h_q, h_kv = q.shape[1], k.shape[1]
    if h_kv < h_q:
        k = k.repeat_interleave(h_q // h_kv, dim=1)
        v = v.repeat_interleave(h_q // h_kv, dim=1)
    s = torch.matmul(q.float(), k.float().transpose(-2, -1)) * scale
    if is_causal:
        n_q, n_k = q.shape[-2], k.shape[-2]
        mask = torch.triu(torch.ones(n_q, n_k, dtype=torch.bool), diagonal=1)
        s.masked_fill_(mask, float("-inf"))
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v.float())


def ref_attention_lse(q, k, v, scale, is_causal=False):
    """:func:`ref_attention` plus the per-row log-sum-exp in natural log,
    ``L = m + ln(max(l, 1e-20))`` (``flash_attn_fwd_volta.cu:343``), -inf for rows with
    no key.  Returns fp32 (O, L)."""
    h_q, h_kv = q.shape[1], k.shape[1]
    if h_kv < h_q:
        k = k.repeat_interleave(h_q // h_kv, dim=1)
        v = v.repeat_interleave(h_q // h_kv, dim=1)
    s = torch.matmul(q.float(), k.float().transpose(-2, -1)) * scale
    if is_causal:
        n_q, n_k = q.shape[-2], k.shape[-2]
        mask = torch.triu(torch.ones(n_q, n_k, dtype=torch.bool), diagonal=1)
        s.masked_fill_(mask, float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))[..., None])
    return torch.matmul(p, v.float()), lse


def ref_backward(q, k, v, grad_out, scale, is_causal=False):
    """fp32 autograd of :func:`ref_attention`; dK/dV summed over GQA groups
    (``tests/test_flash_attn.py:35-58``).  Returns fp32 gradients."""
    h_q, h_kv = q.shape[1], k.shape[1]
    reps = h_q // h_kv
    q_f = q.float().detach().requires_grad_(True)
    k_f = k.float().detach().repeat_interleave(reps, dim=1).requires_grad_(True)
    v_f = v.float().detach().repeat_interleave(reps, dim=1).requires_grad_(True)
    s = torch.matmul(q_f, k_f.transpose(-2, -1)) * scale
    if is_causal:
        n = q.shape[-2]
        mask = torch.triu(torch.ones(n, k.shape[-2], dtype=torch.bool), diagonal=1)
        s.masked_fill_(mask, float("-inf"))
    o = torch.matmul(torch.softmax(s, dim=-1), v_f)
    o.backward(grad_out.float())
    b, _, n_k, d = k.shape
    dk = k_f.grad.view(b, h_kv, reps, n_k, d).sum(dim=2)
    dv = v_f.grad.view(b, h_kv, reps, n_k, d).sum(dim=2)
    return q_f.grad, dk, dv


def ref_decode(q, k_cache, v_cache, cache_seqlens, scale):
    """fp32 eager decode per batch element (``integrations.py:77-98``):
    q [B,1,Hq,d], caches [B,S,Hkv,d] -> O [B,1,Hq,d] fp32."""
    out = torch.empty(q.shape, dtype=torch.float32)
    for b in range(q.shape[0]):
        n = int(cache_seqlens[b])
        qi = q[b:b + 1].transpose(1, 2)                       # [1,Hq,1,d]
        ki = k_cache[b:b + 1, :n].transpose(1, 2)
        vi = v_cache[b:b + 1, :n].transpose(1, 2)
        out[b] = ref_attention(qi, ki, vi, scale, False).transpose(1, 2)[0]
    return out

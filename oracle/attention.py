"""CPU oracle for the attention hot path (forward, backward, varlen, KV-cache decode).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (the ``flash_attn_legacy``
package or the HIP library) imports this module; only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg use it, and
only as the checker.

It restates, in numpy, the algorithm the reference computes and tests against:

* forward   ``O = softmax(Q K^T * scale + causal_mask) V`` with the GQA head map
  ``kv_head = q_head // (H_q / H_kv)`` and a top-left aligned causal mask
  (``col > row`` masked)                      -- reference ``tests/test_flash_attn.py:19-32``,
  ``csrc/kernels/flash_attn_fwd_volta.cu:188,264-266``;
* log-sum-exp ``L = m + ln(max(l, 1e-20))`` in natural log, scale applied
  before the max; a row with no valid key gives ``O = 0, L = -inf``
                                              -- ``flash_attn_fwd_volta.cu:333,343``;
* backward  ``D = rowsum(dO * O)``, ``P = exp(S*scale - L)``,
  ``dV = P^T dO``, ``dP = dO V^T``, ``dS = P (dP - D) scale``,
  ``dQ = dS K``, ``dK = dS^T Q``, dK/dV summed over each GQA group
                                              -- ``tests/test_flash_attn.py:35-58``,
  ``csrc/kernels/flash_attn_bwd.cu:76-107,527-619``;
* varlen    one independent attention per ``cu_seqlens`` segment with local
  (per-sequence) causal indices; backward accumulates ``dk/dv +=`` per segment
                                              -- ``tests/test_flash_attn.py:293-308``,
  ``flash_attn_fwd_volta.cu:448-449``, ``flash_attn_legacy/flash_attn.py:133-157``;
* decode    ``q_len = 1`` attention over the first ``cache_seqlens[b]`` rows of a
  KV cache, no causal mask, optional additive mask row
                                              -- ``flash_attn_legacy/integrations.py:77-98``.

Every function is pinned by ``tests/test_oracle.py`` against independent
checks: float64 autograd of the closed form (torch), brute-force scalar loops
on tiny inputs, central finite differences for the gradients, and the closed
forms the reference's own tests use (N=1 gives O=V, Q=K=0 gives mean(V),
causal row 0 gives V[0], MQA equals broadcast K/V, single-segment varlen
equals batched).
"""

from __future__ import annotations

import numpy as np

NEG_INF = -np.inf


def _expand_kv(x: np.ndarray, h_q: int) -> np.ndarray:
    """Repeat KV heads so head ``h`` of the result is KV head ``h // (h_q // h_kv)``.

    Mirrors ``repeat_interleave(reps, dim=1)`` in ``tests/test_flash_attn.py:22-25``
    and the kernel's head map ``flash_attn_fwd_volta.cu:188``.
    """
    h_kv = x.shape[1]
    assert h_q % h_kv == 0, "H_q must be divisible by H_kv"
    return np.repeat(x, h_q // h_kv, axis=1)


def causal_mask(n_q: int, n_k: int) -> np.ndarray:
    """Boolean mask, True where masked: top-left aligned ``col > row``.

    ``flash_attn_fwd_volta.cu:264-265`` (batched) and ``:448-449`` (varlen, local indices).
    """
    rows = np.arange(n_q)[:, None]
    cols = np.arange(n_k)[None, :]
    return cols > rows


def attention_fwd(q, k, v, scale, causal=False, dtype=np.float64):
    """Forward attention.  q [B,Hq,Nq,d], k/v [B,Hkv,Nk,d] -> (O [B,Hq,Nq,d], L [B,Hq,Nq]).

    Restates ``ref_attention`` (``tests/test_flash_attn.py:19-32``) and the kernel's
    LSE (``flash_attn_fwd_volta.cu:343``); rows without any valid key return O=0 and
    L=-inf like the kernel's ``inv_sum = 0`` branch (``:333``).
    """
    q = np.asarray(q, dtype=dtype)
    h_q = q.shape[1]
    k = _expand_kv(np.asarray(k, dtype=dtype), h_q)
    v = _expand_kv(np.asarray(v, dtype=dtype), h_q)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * dtype(scale)
    if causal:
        s = np.where(causal_mask(q.shape[2], k.shape[2]), NEG_INF, s)
    m = s.max(axis=-1, keepdims=True) if s.shape[-1] > 0 else np.full(s.shape[:-1] + (1,), NEG_INF, dtype)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    p = np.exp(s - m_safe)
    l = p.sum(axis=-1, keepdims=True)
    inv = np.where(l > 0, 1.0 / np.where(l > 0, l, 1.0), 0.0)
    o = np.matmul(p * inv, v)
    with np.errstate(divide="ignore"):
        lse = (m + np.log(np.maximum(l, 1e-20)))[..., 0]
    lse = np.where(np.isfinite(m[..., 0]), lse, NEG_INF)
    return o.astype(dtype), lse.astype(dtype)


def attention_bwd(q, k, v, do, scale, causal=False, dtype=np.float64, o=None, lse=None):
    """Backward attention.  Returns (dQ [B,Hq,N,d], dK [B,Hkv,N,d], dV [B,Hkv,N,d]).

    Recomputes P from the saved log-sum-exp and uses ``D = rowsum(dO * O)`` as the
    reference kernel does (``flash_attn_bwd.cu:76-107,527-619``); when ``o``/``lse``
    are not given they come from :func:`attention_fwd`.  GQA gradients are summed
    over the query heads of each KV group (``tests/test_flash_attn.py:54-57``).
    """
    q = np.asarray(q, dtype=dtype)
    do = np.asarray(do, dtype=dtype)
    h_q, h_kv = q.shape[1], k.shape[1]
    if o is None or lse is None:
        o, lse = attention_fwd(q, k, v, scale, causal, dtype)
    o = np.asarray(o, dtype=dtype)
    lse = np.asarray(lse, dtype=dtype)
    ke = _expand_kv(np.asarray(k, dtype=dtype), h_q)
    ve = _expand_kv(np.asarray(v, dtype=dtype), h_q)
    s = np.matmul(q, np.swapaxes(ke, -1, -2)) * dtype(scale)
    lse_safe = np.where(np.isfinite(lse), lse, 0.0)[..., None]
    p = np.exp(s - lse_safe)
    invalid = ~np.isfinite(lse)[..., None] | np.zeros_like(p, dtype=bool)
    if causal:
        invalid = invalid | causal_mask(q.shape[2], ke.shape[2])
    p = np.where(invalid, 0.0, p)
    dv_e = np.matmul(np.swapaxes(p, -1, -2), do)
    dp = np.matmul(do, np.swapaxes(ve, -1, -2))
    d_row = (do * o).sum(axis=-1, keepdims=True)
    ds = p * (dp - d_row) * dtype(scale)
    dq = np.matmul(ds, ke)
    dk_e = np.matmul(np.swapaxes(ds, -1, -2), q)
    b, _, n_k, d = ke.shape
    dk = dk_e.reshape(b, h_kv, h_q // h_kv, n_k, d).sum(axis=2)
    dv = dv_e.reshape(b, h_kv, h_q // h_kv, n_k, d).sum(axis=2)
    return dq.astype(dtype), dk.astype(dtype), dv.astype(dtype)


def _segments(cu):
    cu = [int(x) for x in np.asarray(cu).reshape(-1)]
    return [(cu[i], cu[i + 1]) for i in range(len(cu) - 1)]


def varlen_fwd(q, k, v, cu_q, cu_k, scale, causal=False, dtype=np.float64):
    """Packed forward.  q [total_q,Hq,d], k/v [total_k,Hkv,d] -> (O [total_q,Hq,d], L [total_q,Hq]).

    One independent attention per segment with local causal indices
    (``tests/test_flash_attn.py:293-308``, ``flash_attn_fwd_volta.cu:448-449``); L is
    laid out ``[total_q, H_q]`` as the reference returns it (``flash_attn_legacy.cpp:222``).
    """
    q = np.asarray(q, dtype=dtype)
    o = np.zeros_like(q)
    lse = np.full(q.shape[:2], NEG_INF, dtype=dtype)
    for (qs, qe), (ks, ke) in zip(_segments(cu_q), _segments(cu_k)):
        if qe == qs:
            continue
        qi = np.swapaxes(q[qs:qe], 0, 1)[None]
        ki = np.swapaxes(np.asarray(k[ks:ke], dtype=dtype), 0, 1)[None]
        vi = np.swapaxes(np.asarray(v[ks:ke], dtype=dtype), 0, 1)[None]
        oi, li = attention_fwd(qi, ki, vi, scale, causal, dtype)
        o[qs:qe] = np.swapaxes(oi[0], 0, 1)
        lse[qs:qe] = li[0].T
    return o, lse


def varlen_bwd(q, k, v, do, cu_q, cu_k, scale, causal=False, dtype=np.float64):
    """Packed backward: per-segment gradients, ``dk/dv +=`` into the packed buffers.

    Semantics of ``FlashAttnVarlenFunc.backward`` (``flash_attn_legacy/flash_attn.py:133-157``).
    """
    q = np.asarray(q, dtype=dtype)
    dq = np.zeros_like(q)
    dk = np.zeros(np.shape(k), dtype=dtype)
    dv = np.zeros(np.shape(v), dtype=dtype)
    for (qs, qe), (ks, ke) in zip(_segments(cu_q), _segments(cu_k)):
        if qe == qs:
            continue
        sw = lambda x: np.swapaxes(np.asarray(x, dtype=dtype), 0, 1)[None]
        dqi, dki, dvi = attention_bwd(sw(q[qs:qe]), sw(k[ks:ke]), sw(v[ks:ke]), sw(do[qs:qe]),
                                      scale, causal, dtype)
        dq[qs:qe] = np.swapaxes(dqi[0], 0, 1)
        dk[ks:ke] += np.swapaxes(dki[0], 0, 1)
        dv[ks:ke] += np.swapaxes(dvi[0], 0, 1)
    return dq, dk, dv


def decode(q, k_cache, v_cache, cache_seqlens, scale, bias=None, dtype=np.float64):
    """KV-cache decode, one query token per sequence, no causal mask.

    q [B,1,Hq,d]; k_cache/v_cache [B,S_max,Hkv,d]; cache_seqlens [B] -> (O [B,1,Hq,d], L [B,Hq]).
    Restates the eager branch of ``flash_attn_legacy_forward``
    (``flash_attn_legacy/integrations.py:77-98``): GQA by head repetition,
    ``s = q k^T * scale (+ mask)``, softmax, ``@ v``; ``bias`` is the additive mask row
    ``[B, S]`` (only the first ``cache_seqlens[b]`` entries are used).
    """
    q = np.asarray(q, dtype=dtype)
    b_sz, _, h_q, d = q.shape
    o = np.zeros_like(q)
    lse = np.full((b_sz, h_q), NEG_INF, dtype=dtype)
    for b in range(b_sz):
        n = int(cache_seqlens[b])
        if n == 0:
            continue
        qi = q[b, 0][None, :, None, :]                       # [1,Hq,1,d]
        ki = np.swapaxes(np.asarray(k_cache[b, :n], dtype=dtype), 0, 1)[None]
        vi = np.swapaxes(np.asarray(v_cache[b, :n], dtype=dtype), 0, 1)[None]
        ke = _expand_kv(ki, h_q)
        ve = _expand_kv(vi, h_q)
        s = np.matmul(qi, np.swapaxes(ke, -1, -2)) * dtype(scale)   # [1,Hq,1,n]
        if bias is not None:
            s = s + np.asarray(bias[b, :n], dtype=dtype)
        m = s.max(axis=-1, keepdims=True)
        p = np.exp(s - m)
        l = p.sum(axis=-1, keepdims=True)
        o[b, 0] = np.matmul(p / l, ve)[0, :, 0, :]
        lse[b] = (m + np.log(l))[0, :, 0, 0]
    return o, lse


# ---------------------------------------------------------------------------
# Seeded inputs for the five benchmark configurations (fp16, i.i.d. N(0,1)).
# ---------------------------------------------------------------------------

def make_rng(seed: int = 0) -> np.random.Generator:
    return np.random.default_rng(seed)


def randn_f16(rng: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    return (rng.standard_normal(shape, dtype=np.float32) * scale).astype(np.float16)

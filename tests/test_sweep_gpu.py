"""Seeded random-shape parity sweeps on the GPU: batched forward and backward, packed
varlen forward and backward, and decode, over random head dims, GQA ratios, batch
sizes, lengths (ragged, Nq != Nk, length 1, empty segments), causal flags, cache
layouts, mask biases and both element types.  References are the reference's own
fp32 formulas (oracle/torch_ref.py: tests/test_flash_attn.py:19-58 and the eager
decode branch of integrations.py:77-98) on the same inputs, on the host.

Tolerances: fp16 as everywhere else (forward max-abs 2e-3 against max(1, |O|),
gradients max |g - g_ref| / max(|g_ref|, 1e-3) <= 1e-2); bf16 scaled to its 8-bit
mantissa (2^-6 on the forward, 4e-2 on gradients).  The 1e-3 floor keeps gradients
that are zero in exact arithmetic (one key per row: O = V, so dQ = dK = 0) from
turning fp32 rounding noise into a large relative error.
"""

import math
import random

import pytest
import torch

from oracle.torch_ref import ref_attention, ref_backward, ref_decode

pytestmark = pytest.mark.gpu

FWD_TOL = {torch.float16: 2e-3, torch.bfloat16: 2.0 ** -6}
GRAD_TOL = {torch.float16: 1e-2, torch.bfloat16: 4e-2}


def fwd_err(o, ref):
    ref = ref.float()
    return float((o.float().cpu() - ref).abs().max()) / max(1.0, float(ref.abs().max()))


def grad_err(g, ref):
    if ref.numel() == 0:
        return 0.0
    return float((g.float().cpu() - ref).abs().max()) / max(float(ref.abs().max()), 1e-3)


def draw(gen, shape, dt, scale=0.7):
    return (torch.randn(shape, generator=gen) * scale).to(dt)


@pytest.mark.parametrize("seed", range(4))
def test_batched_sweep(seed):
    from flash_attn_legacy import hip_ext
    rng = random.Random(1000 + seed)
    for it in range(15):
        d = rng.choice([32, 64, 96, 128, 256])
        g, hk, B = rng.choice([1, 2, 4, 8]), rng.choice([1, 2]), rng.choice([1, 2])
        nq = rng.choice([1, rng.randint(1, 300)])
        nk = rng.choice([nq, rng.randint(1, 300)])
        causal = rng.random() < 0.5
        dt = rng.choice([torch.float16, torch.bfloat16])
        scale = rng.choice([1.0, 0.5, 2.0]) / math.sqrt(d)
        gen = torch.Generator().manual_seed(seed * 100 + it)
        q, do = draw(gen, (B, hk * g, nq, d), dt), draw(gen, (B, hk * g, nq, d), dt)
        k, v = draw(gen, (B, hk, nk, d), dt), draw(gen, (B, hk, nk, d), dt)
        case = f"it={it} d={d} B={B} hq={hk * g} hk={hk} nq={nq} nk={nk} causal={causal} {dt}"
        o, lse = hip_ext.forward(q.cuda(), k.cuda(), v.cuda(), scale, causal)
        assert fwd_err(o, ref_attention(q, k, v, scale, causal)) <= FWD_TOL[dt], case
        grads = hip_ext.backward(do.cuda(), q.cuda(), k.cuda(), v.cuda(), o, lse, scale, causal)
        for name, got, ref in zip(("dq", "dk", "dv"), grads, ref_backward(q, k, v, do, scale, causal)):
            assert grad_err(got, ref) <= GRAD_TOL[dt], f"{name} {case}"


@pytest.mark.parametrize("seed", range(3))
def test_varlen_sweep(seed):
    from flash_attn_legacy import hip_ext
    rng = random.Random(2000 + seed)
    for it in range(10):
        d = rng.choice([32, 64, 96, 128, 256])
        g, hk = rng.choice([1, 2, 4]), rng.choice([1, 2])
        causal = rng.random() < 0.5
        dt = rng.choice([torch.float16, torch.bfloat16])
        ns = rng.randint(1, 6)
        lq = [rng.choice([0, 1, rng.randint(1, 250)]) for _ in range(ns)]
        lk = [n if rng.random() < 0.7 else rng.randint(1, 250) for n in lq]
        lk = [max(n, 1) if m > 0 else n for m, n in zip(lq, lk)]   # a query row needs a key
        if sum(lq) == 0:
            continue
        cq = [0]
        ck = [0]
        for a, b in zip(lq, lk):
            cq.append(cq[-1] + a)
            ck.append(ck[-1] + b)
        gen = torch.Generator().manual_seed(seed * 100 + it)
        q, do = draw(gen, (cq[-1], hk * g, d), dt), draw(gen, (cq[-1], hk * g, d), dt)
        k, v = draw(gen, (ck[-1], hk, d), dt), draw(gen, (ck[-1], hk, d), dt)
        cu_q = torch.tensor(cq, dtype=torch.int32, device="cuda")
        cu_k = torch.tensor(ck, dtype=torch.int32, device="cuda")
        scale = 1.0 / math.sqrt(d)
        case = f"it={it} d={d} hq={hk * g} hk={hk} lq={lq} lk={lk} causal={causal} {dt}"
        o, lse = hip_ext.forward_varlen(q.cuda(), k.cuda(), v.cuda(), cu_q, cu_k, max(lq), max(lk), scale, causal)
        dq, dk, dv = hip_ext.backward_varlen(do.cuda(), q.cuda(), k.cuda(), v.cuda(), o, lse, cu_q, cu_k,
                                             max(lq), max(lk), scale, causal)
        for i in range(ns):
            if lq[i] == 0:
                continue
            sq, sk = slice(cq[i], cq[i + 1]), slice(ck[i], ck[i + 1])
            t = lambda x, s: x[s].transpose(0, 1).unsqueeze(0)
            ref_o = ref_attention(t(q, sq), t(k, sk), t(v, sk), scale, causal)
            assert fwd_err(t(o, sq), ref_o) <= FWD_TOL[dt], f"seg {i} {case}"
            refs = ref_backward(t(q, sq), t(k, sk), t(v, sk), t(do, sq), scale, causal)
            for name, got, ref in zip(("dq", "dk", "dv"), (t(dq, sq), t(dk, sk), t(dv, sk)), refs):
                assert grad_err(got, ref) <= GRAD_TOL[dt], f"{name} seg {i} {case}"


@pytest.mark.parametrize("seed", range(3))
def test_decode_sweep(seed):
    from flash_attn_legacy import hip_ext
    rng = random.Random(3000 + seed)
    for it in range(10):
        d = rng.choice([32, 64, 96, 128, 256])
        g, hk, B = rng.choice([1, 4, 8, 16, 32]), rng.choice([1, 2]), rng.randint(1, 4)
        S = rng.randint(1, 3000)
        lens = [rng.choice([0, 1, S, rng.randint(0, S)]) for _ in range(B)]
        dt = rng.choice([torch.float16, torch.bfloat16])
        layout = rng.choice(["bshd", "bhsd"])
        gen = torch.Generator().manual_seed(seed * 100 + it)
        q = draw(gen, (B, hk * g, d), dt, 1.0)
        kc, vc = draw(gen, (B, S, hk, d), dt, 1.0), draw(gen, (B, S, hk, d), dt, 1.0)
        use_bias = rng.random() < 0.3
        bias = None
        if use_bias:
            bias = torch.zeros(B, S)
            bias[torch.rand(B, S, generator=gen) < 0.2] = float("-inf")
            bias[:, 0] = 0.0   # every non-empty row keeps a key
        scale = 1.0 / math.sqrt(d)
        case = f"it={it} d={d} B={B} hq={hk * g} hk={hk} S={S} lens={lens} {layout} bias={use_bias} {dt}"
        kd = kc if layout == "bshd" else kc.transpose(1, 2).contiguous()
        vd = vc if layout == "bshd" else vc.transpose(1, 2).contiguous()
        seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
        o = hip_ext.decode(q.cuda(), kd.cuda(), vd.cuda(), seq, scale,
                           mask_bias=None if bias is None else bias.cuda(), cache_layout=layout)
        ref = torch.zeros(B, hk * g, d)
        for b in range(B):
            n = lens[b]
            if n == 0:
                continue
            if bias is None:
                ref[b] = ref_decode(q[b:b + 1, None], kc[b:b + 1], vc[b:b + 1], [n], scale)[0, 0]
            else:
                kk = kc[b, :n].float().transpose(0, 1).repeat_interleave(g, 0)
                vv = vc[b, :n].float().transpose(0, 1).repeat_interleave(g, 0)
                s = (kk @ q[b].float()[:, :, None])[..., 0] * scale + bias[b, :n]
                ref[b] = (torch.softmax(s, -1)[:, None, :] @ vv)[:, 0]
        assert fwd_err(o, ref) <= FWD_TOL[dt], case
        for b in range(B):
            if lens[b] == 0:
                assert float(o[b].float().abs().max()) == 0.0, f"empty cache row {b} {case}"

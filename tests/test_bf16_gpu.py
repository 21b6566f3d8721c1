"""bfloat16 entry points (fal_*_bf16) on the GPU, against the float64 oracle on the
same bf16 inputs.

The reference is fp16 only; bf16 is this library's extension (bf16 MFMA with fp32
accumulation, the softmax scale applied to the fp32 scores).  Tolerances, written
against bf16's 8-bit mantissa (one unit in the last place at 1 is 2^-7):
  * forward O: |O - O_ref| <= 2^-7 * max(1, |O_ref|) elementwise -- the output's own
    rounding is half a unit, P rounded to bf16 for the PV product adds up to about one;
  * forward L (fp32): |L - L_ref| <= 2e-3;
  * gradients: max |g - g_ref| / max |g_ref| <= 4e-2 (P and dS are rounded to bf16
    for their second products; fp16's bound is 1e-2, eight times finer mantissa).
Coverage: every head dim, causal and not, MHA/GQA/MQA, ragged lengths; varlen
forward and backward; decode; the autograd function; determinism of the backward;
a bf16 HF model against eager attention (also with a padded batch); the attention
module; C2 (sampled rows) and C3 at full size.
"""

import math

import numpy as np
import pytest
import torch

from helpers import cu_from_lens, np64, oracle_bwd, oracle_fwd, rel_err
from oracle import attention as orc

pytestmark = pytest.mark.gpu

BF16_ULP1 = 2.0 ** -7
LSE_ATOL = 2e-3
GRAD_RTOL_BF16 = 4e-2


def rbf(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16).cuda()


def check_out(o, ref):
    o = o.detach().float().cpu()
    ref = ref.float()
    assert o.shape == ref.shape
    bound = BF16_ULP1 * torch.clamp(ref.abs(), min=1.0)
    excess = ((o - ref).abs() - bound).max().item() if o.numel() else -1.0
    assert excess <= 0.0, f"max excess over the bf16 bound {excess:.3e}"


@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (4, 1)])
def test_forward(d, causal, hq, hkv):
    from flash_attn_legacy import hip_ext
    N = 200
    q, k, v = rbf((2, hq, N, d), 1), rbf((2, hkv, N, d), 2), rbf((2, hkv, N, d), 3)
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, causal)
    assert o.dtype == torch.bfloat16 and lse.dtype == torch.float32
    o_ref, l_ref = oracle_fwd(q, k, v, scale, causal)
    check_out(o, o_ref)
    assert (lse.cpu().double() - l_ref).abs().max().item() <= LSE_ATOL


@pytest.mark.parametrize("nq,nk", [(1, 1), (64, 200), (200, 64), (129, 129)])
def test_forward_ragged(nq, nk):
    from flash_attn_legacy import hip_ext
    q, k, v = rbf((1, 4, nq, 128), 4), rbf((1, 2, nk, 128), 5), rbf((1, 2, nk, 128), 6)
    o, _ = hip_ext.forward(q, k, v, 0.1, True)
    check_out(o, oracle_fwd(q, k, v, 0.1, True)[0])


@pytest.mark.parametrize("d", [32, 64, 96, 128, 256])
@pytest.mark.parametrize("causal", [False, True])
def test_backward(d, causal):
    from flash_attn_legacy import hip_ext
    N, hq, hkv = 160, 4, 2
    q, k, v = rbf((2, hq, N, d), 7, 0.5), rbf((2, hkv, N, d), 8, 0.5), rbf((2, hkv, N, d), 9, 0.5)
    do = rbf((2, hq, N, d), 10)
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, causal)
    dq, dk, dv = hip_ext.backward(do, q, k, v, o, lse, scale, causal)
    assert dq.dtype == dk.dtype == dv.dtype == torch.bfloat16
    refs = oracle_bwd(q, k, v, do, scale, causal)
    for name, g, r in zip(("dq", "dk", "dv"), (dq, dk, dv), refs):
        e = rel_err(g, r)
        assert e <= GRAD_RTOL_BF16, f"{name} rel err {e:.3e}"


@pytest.mark.parametrize("d", [64, 128])
def test_backward_deterministic(d):
    from flash_attn_legacy import hip_ext
    q, k, v, do = (rbf((2, 8, 384, d), s) for s in (11, 12, 13, 14))
    o, lse = hip_ext.forward(q, k, v, 0.125, True)
    a = hip_ext.backward(do, q, k, v, o, lse, 0.125, True)
    b = hip_ext.backward(do, q, k, v, o, lse, 0.125, True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_autograd_function():
    from flash_attn_legacy import flash_attention
    q = rbf((1, 8, 96, 64), 15, 0.5).requires_grad_(True)
    k = rbf((1, 2, 96, 64), 16, 0.5).requires_grad_(True)
    v = rbf((1, 2, 96, 64), 17, 0.5).requires_grad_(True)
    do = rbf((1, 8, 96, 64), 18)
    o = flash_attention(q, k, v, is_causal=True)
    o.backward(do)
    check_out(o, oracle_fwd(q, k, v, 0.125, True)[0])
    for g, r in zip((q.grad, k.grad, v.grad), oracle_bwd(q, k, v, do, 0.125, True)):
        assert g.dtype == torch.bfloat16 and rel_err(g, r) <= GRAD_RTOL_BF16


def test_mixed_dtypes_rejected():
    from flash_attn_legacy import hip_ext
    q = rbf((1, 2, 16, 64), 19)
    with pytest.raises(RuntimeError, match="like Q"):
        hip_ext.forward(q, q.half(), q, 0.1, False)


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_forward_backward(causal):
    from flash_attn_legacy import hip_ext
    lens = [37, 256, 1, 190]
    cu = cu_from_lens(lens)
    tot, hq, hkv, d = sum(lens), 8, 2, 128
    q, k, v = rbf((tot, hq, d), 20, 0.5), rbf((tot, hkv, d), 21, 0.5), rbf((tot, hkv, d), 22, 0.5)
    do = rbf((tot, hq, d), 23)
    mx = max(lens)
    o, lse = hip_ext.forward_varlen(q, k, v, cu, cu, mx, mx, 0.09, causal)
    dq, dk, dv = hip_ext.backward_varlen(do, q, k, v, o, lse, cu, cu, mx, mx, 0.09, causal)
    a = 0
    for n in lens:
        sl = slice(a, a + n)
        t = lambda x: x[sl].transpose(0, 1).unsqueeze(0)
        o_ref, _ = oracle_fwd(t(q), t(k), t(v), 0.09, causal)
        check_out(t(o), o_ref)
        refs = oracle_bwd(t(q), t(k), t(v), t(do), 0.09, causal)
        for g, r in zip((t(dq), t(dk), t(dv)), refs):
            assert rel_err(g, r) <= GRAD_RTOL_BF16
        a += n


@pytest.mark.parametrize("causal", [False, True])
def test_varlen_four_heads_pair_walk(causal):
    """bf16 on the varlen pair walk (head dim 128, Hq/Hkv = 4, more than 64 sequences so
    the schedule kernel builds the pair list): O and L of every sequence against the
    oracle."""
    from flash_attn_legacy import hip_ext
    g = torch.Generator().manual_seed(95)
    lens = [int(x) for x in torch.randint(1, 300, (68,), generator=g)] + [64, 65]
    cu = cu_from_lens(lens)
    tot, hq, hkv, d = sum(lens), 8, 2, 128
    q, k, v = rbf((tot, hq, d), 96), rbf((tot, hkv, d), 97), rbf((tot, hkv, d), 98)
    mx = max(lens)
    o, lse = hip_ext.forward_varlen(q, k, v, cu, cu, mx, mx, 1.0 / math.sqrt(d), causal)
    a = 0
    for n in lens:
        sl = slice(a, a + n)
        t = lambda x: x[sl].transpose(0, 1).unsqueeze(0)
        o_ref, l_ref = oracle_fwd(t(q), t(k), t(v), 1.0 / math.sqrt(d), causal)
        check_out(t(o), o_ref)
        err = (lse[sl].transpose(0, 1).unsqueeze(0).float().cpu() - l_ref.float()).abs().max().item()
        assert err <= LSE_ATOL, err
        a += n


@pytest.mark.parametrize("d", [64, 128, 256])
@pytest.mark.parametrize("layout", ["bshd", "bhsd"])
def test_decode(d, layout):
    from flash_attn_legacy import hip_ext
    B, hq, hkv, S = 3, 8, 2, 900
    lens = [900, 1, 417]
    q = rbf((B, hq, d), 24)
    shape = (B, S, hkv, d) if layout == "bshd" else (B, hkv, S, d)
    kc, vc = rbf(shape, 25), rbf(shape, 26)
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    o, lse = hip_ext.decode(q, kc, vc, seq, 1 / math.sqrt(d), cache_layout=layout, return_lse=True)
    assert o.dtype == torch.bfloat16
    k = kc if layout == "bshd" else kc.transpose(1, 2)
    v = vc if layout == "bshd" else vc.transpose(1, 2)
    o_ref, l_ref = orc.decode(np64(q)[:, None], np64(k), np64(v), np.array(lens), 1 / math.sqrt(d), None)
    check_out(o, torch.from_numpy(o_ref[:, 0]))
    assert (lse.cpu().double() - torch.from_numpy(l_ref)).abs().max().item() <= LSE_ATOL


def test_hf_bf16_model_runs_natively(monkeypatch):
    """A bf16 LLaMA: the attention function receives bf16 and the kernels run in bf16
    (no cast to fp16); prefill logits match eager attention's."""
    import flash_attn_legacy  # noqa: F401
    from flash_attn_legacy import hip_ext
    from transformers import LlamaConfig, LlamaForCausalLM
    seen = []
    real = hip_ext.forward
    monkeypatch.setattr(hip_ext, "forward", lambda q, *a, **kw: seen.append(q.dtype) or real(q, *a, **kw))

    def model(impl):
        cfg = LlamaConfig(vocab_size=256, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                          num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=512)
        cfg._attn_implementation = impl
        torch.manual_seed(0)
        return LlamaForCausalLM(cfg).cuda().to(torch.bfloat16).eval()

    flash, eager = model("flash_attn_legacy"), model("eager")
    eager.load_state_dict(flash.state_dict())
    ids = torch.randint(0, 256, (2, 96), device="cuda", generator=torch.Generator("cuda").manual_seed(1))
    with torch.no_grad():
        a = flash(ids).logits.float()
        b = eager(ids).logits.float()
    assert seen and all(dt == torch.bfloat16 for dt in seen)
    cos = torch.nn.functional.cosine_similarity(a.reshape(1, -1), b.reshape(1, -1)).item()
    assert cos > 0.999, cos


def test_c2_full_size_sampled_rows():
    """C2 in bf16 at full size (B=4, 32q/8kv heads, N=4096, d=128, causal): O and L of
    sampled rows of several heads against exact float64 rows of the same bf16 inputs."""
    from flash_attn_legacy import hip_ext
    B, Hq, Hkv, N, d = 4, 32, 8, 4096, 128
    q, k, v = rbf((B, Hq, N, d), 30), rbf((B, Hkv, N, d), 31), rbf((B, Hkv, N, d), 32)
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, True)
    rows = [0, 1, 127, 128, 2047, 4000, N - 1]
    for bb, h in ((0, 0), (1, 13), (3, 31)):
        qf, kf, vf = (np64(t) for t in (q[bb, h], k[bb, h // 4], v[bb, h // 4]))
        ref_o, ref_l = [], []
        for r in rows:
            s = kf[: r + 1] @ qf[r] * scale
            m = s.max()
            p = np.exp(s - m)
            ref_o.append(p @ vf[: r + 1] / p.sum())
            ref_l.append(m + np.log(p.sum()))
        check_out(o[bb, h, rows], torch.from_numpy(np.stack(ref_o)))
        assert np.abs(lse[bb, h, rows].double().cpu().numpy() - np.array(ref_l)).max() <= LSE_ATOL


def test_c3_full_size_gradients():
    """C3 in bf16 at full size (B=2, 16 heads, N=2048, d=128, causal): dQ/dK/dV of two
    heads against the float64 oracle on the same bf16 inputs."""
    from flash_attn_legacy import hip_ext
    B, H, N, d = 2, 16, 2048, 128
    q, k, v, do = (rbf((B, H, N, d), s) for s in (33, 34, 35, 36))
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, True)
    dq, dk, dv = hip_ext.backward(do, q, k, v, o, lse, scale, True)
    for bb, h in ((0, 0), (1, 9)):
        sl = lambda t: t[bb:bb + 1, h:h + 1]
        refs = oracle_bwd(sl(q), sl(k), sl(v), sl(do), scale, True)
        for name, g, r in zip(("dq", "dk", "dv"), (sl(dq), sl(dk), sl(dv)), refs):
            e = rel_err(g, r)
            assert e <= GRAD_RTOL_BF16, f"{name} head {h}: rel err {e:.3e}"


def test_module_bf16_forward_backward():
    """FlashMultiHeadAttention in bf16 runs the bf16 kernels (no cast to fp16): output and
    input gradient against an fp32 copy of the module with fp32 attention."""
    import torch.nn.functional as F
    from flash_attn_legacy import FlashMultiHeadAttention
    from oracle.torch_ref import ref_attention
    torch.manual_seed(0)
    m = FlashMultiHeadAttention(512, num_heads=8, num_kv_heads=2, causal=True).cuda().to(torch.bfloat16)
    x = rbf((2, 64, 512), 40).requires_grad_(True)
    out = m(x)
    assert out.dtype == torch.bfloat16
    g = rbf((2, 64, 512), 41, 0.1)
    out.backward(g)
    p = {n: t.detach().float().cpu() for n, t in m.named_parameters()}
    xf = x.detach().float().cpu().requires_grad_(True)
    q = F.linear(xf, p["q_proj.weight"], p["q_proj.bias"]).view(2, 64, 8, 64).transpose(1, 2)
    k = F.linear(xf, p["k_proj.weight"], p["k_proj.bias"]).view(2, 64, 2, 64).transpose(1, 2)
    v = F.linear(xf, p["v_proj.weight"], p["v_proj.bias"]).view(2, 64, 2, 64).transpose(1, 2)
    o = ref_attention(q, k, v, m.scale, True).transpose(1, 2).reshape(2, 64, 512)
    ref = F.linear(o, p["out_proj.weight"], p["out_proj.bias"])
    ref.backward(g.float().cpu())
    cos = lambda a, b: F.cosine_similarity(a.float().cpu().reshape(1, -1), b.reshape(1, -1)).item()
    assert cos(out.detach(), ref.detach()) > 0.999
    assert cos(x.grad, xf.grad) > 0.99


def test_hf_bf16_padded_batch():
    """A bf16 LLaMA with a left-padded batch: the padded prefill runs the bf16 varlen
    kernel; logits of real tokens match eager attention's."""
    import flash_attn_legacy  # noqa: F401
    from transformers import LlamaConfig, LlamaForCausalLM

    def model(impl):
        cfg = LlamaConfig(vocab_size=256, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                          num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=512)
        cfg._attn_implementation = impl
        torch.manual_seed(0)
        return LlamaForCausalLM(cfg).cuda().to(torch.bfloat16).eval()

    flash, eager = model("flash_attn_legacy"), model("eager")
    eager.load_state_dict(flash.state_dict())
    ids = torch.randint(0, 256, (2, 80), device="cuda", generator=torch.Generator("cuda").manual_seed(3))
    mask = torch.ones_like(ids)
    mask[0, :25] = 0
    with torch.no_grad():
        a = flash(ids, attention_mask=mask).logits.float()
        b = eager(ids, attention_mask=mask).logits.float()
    real = mask.bool()
    cos = torch.nn.functional.cosine_similarity(a[real].reshape(1, -1), b[real].reshape(1, -1)).item()
    assert torch.isfinite(a[real]).all() and cos > 0.999, cos


@pytest.mark.parametrize("hkv", [4, 16])
def test_persistent_grid_every_head(hkv):
    """bf16 head_dim 128 on the persistent forward grid (four heads per workgroup for
    16/4, 256-row items for MHA): every row of every head within one bf16 ulp of the fp32
    formula (computed on the GPU)."""
    from flash_attn_legacy import hip_ext
    B, Hq, N, d = 2, 16, 4352, 128
    q, k, v = rbf((B, Hq, N, d), 41), rbf((B, hkv, N, d), 42), rbf((B, hkv, N, d), 43)
    scale = 1.0 / math.sqrt(d)
    o, _ = hip_ext.forward(q, k, v, scale, True)
    G = Hq // hkv
    mask = torch.triu(torch.ones(N, N, dtype=torch.bool, device="cuda"), 1)
    for b in range(B):
        for g in range(hkv):
            qs = q[b, g * G:(g + 1) * G].float()
            s = torch.matmul(qs, k[b, g].float().t()) * scale
            ref = torch.matmul(torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1), v[b, g].float())
            check_out(o[b, g * G:(g + 1) * G], ref.cpu())

"""The attention modules and the forward's memory footprint on the GPU.

Mirrors the reference's TestModules (tests/test_flash_attn.py:422-463), which checks
output shapes only, and compares values as well: against the module's own
projections, fp32 attention (oracle/torch_ref.py) and an fp32 output projection.
It also mirrors TestMemoryScaling (:554-586) and adds an exact bound: the forward
allocates only O and L beyond its inputs.
"""

import pytest
import torch
import torch.nn.functional as F

from helpers import max_abs, randn, rel_err
from oracle.torch_ref import ref_attention

pytestmark = pytest.mark.gpu


def module_reference(m, x, kv=None):
    """fp32 result of FlashMultiHeadAttention.forward (flash_attn.py) for module m: the
    module's q/k/v projections, fp32 attention on the host, fp32 output projection."""
    B, N, E = x.shape
    kv = x if kv is None else kv
    with torch.no_grad():
        q = m.q_proj(x).view(B, N, m.num_heads, m.head_dim).transpose(1, 2)
        k = m.k_proj(kv).view(B, -1, m.num_kv_heads, m.head_dim).transpose(1, 2)
        v = m.v_proj(kv).view(B, -1, m.num_kv_heads, m.head_dim).transpose(1, 2)
        o = ref_attention(q.cpu(), k.cpu(), v.cpu(), m.scale, m.causal)
        o = o.transpose(1, 2).reshape(B, N, E)
        w = m.out_proj.weight.float().cpu()
        b = m.out_proj.bias.float().cpu() if m.out_proj.bias is not None else None
        return F.linear(o, w, b)


def make_module(embed_dim, num_heads, num_kv_heads=None, causal=False, seed=0):
    from flash_attn_legacy import FlashMultiHeadAttention
    torch.manual_seed(seed)
    return FlashMultiHeadAttention(embed_dim, num_heads=num_heads, num_kv_heads=num_kv_heads,
                                   causal=causal).cuda().half()


def check_module(m, x, kv=None):
    out = m(x) if kv is None else m(x, kv)
    assert out.shape == x.shape and out.dtype == torch.float16
    ref = module_reference(m, x, kv)
    cos = F.cosine_similarity(out.float().cpu().reshape(1, -1), ref.reshape(1, -1)).item()
    assert cos > 0.9999, cos
    assert max_abs(out, ref) < 1e-2


@pytest.mark.parametrize("num_heads,num_kv_heads,causal", [(8, None, True), (8, 2, True), (8, 1, False)])
def test_mha_gqa_mqa_modules(num_heads, num_kv_heads, causal):
    m = make_module(512, num_heads, num_kv_heads, causal)
    check_module(m, randn((2, 128, 512), 1))


@pytest.mark.parametrize("embed_dim,num_heads,head_dim", [(384, 12, 32), (768, 8, 96), (512, 2, 256)])
def test_module_other_head_dims(embed_dim, num_heads, head_dim):
    m = make_module(embed_dim, num_heads, causal=True)
    assert m.head_dim == head_dim
    check_module(m, randn((2, 64, embed_dim), 2))


def test_cross_attention_module():
    m = make_module(512, 8, 2, causal=False)
    check_module(m, randn((2, 40, 512), 3), randn((2, 96, 512), 4))


def test_module_backward_matches_fp32():
    """Input gradient of the fp16 module against an fp32 copy of it using fp32 autograd
    attention (same weights)."""
    m = make_module(512, 8, 2, causal=True)
    x = randn((2, 64, 512), 5).requires_grad_(True)
    g = randn((2, 64, 512), 6, scale=0.1)
    m(x).backward(g)
    assert x.grad is not None and torch.isfinite(x.grad).all()

    mf = {n: p.detach().float().cpu() for n, p in m.named_parameters()}
    xf = x.detach().float().cpu().requires_grad_(True)
    B, N, E, H, Hk, d = 2, 64, 512, 8, 2, 64
    q = F.linear(xf, mf["q_proj.weight"], mf["q_proj.bias"]).view(B, N, H, d).transpose(1, 2)
    k = F.linear(xf, mf["k_proj.weight"], mf["k_proj.bias"]).view(B, N, Hk, d).transpose(1, 2)
    v = F.linear(xf, mf["v_proj.weight"], mf["v_proj.bias"]).view(B, N, Hk, d).transpose(1, 2)
    o = ref_attention(q, k, v, m.scale, True).transpose(1, 2).reshape(B, N, E)
    F.linear(o, mf["out_proj.weight"], mf["out_proj.bias"]).backward(g.float().cpu())
    assert rel_err(x.grad, xf.grad) < 2e-2


def test_memory_linear_in_sequence_length():
    """O(N) memory (reference test_memory_subquadratic, :557-586): the ratio of the extra
    memory at N=4096 and N=1024 stays well under the quadratic 16; and the extra memory
    of a forward call is O (fp16) plus L (fp32) plus, for grids smaller than the GPU, the
    split-KV workspace (partial outputs, linear in N, freed after the call)."""
    from flash_attn_legacy import flash_attention, hip_ext
    B, H, d = 2, 8, 64

    def extra(N):
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        q = randn((B, H, N, d), 7)
        k, v = randn((B, H, N, d), 8), randn((B, H, N, d), 9)
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        out = flash_attention(q, k, v, is_causal=True)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated()
        del q, k, v, out
        return peak - base

    e1, e4 = extra(1024), extra(4096)
    assert e4 / e1 < 10
    for N, e in ((1024, e1), (4096, e4)):
        ws = hip_ext._lib.fal_fwd_workspace_size(B, H, N, N, d, 1)
        assert ws <= 32 * B * H * N * (d + 2)              # a bounded number of fp32 partial rows
        expected = B * H * N * d * 2 + B * H * N * 4 + ws
        assert e <= expected + (1 << 20), (N, e, expected)

"""HuggingFace integration on the GPU with a tiny random LLaMA built offline (8 query
heads, 2 KV heads, head_dim 64), after the reference's tests/test_transformers.py:38-162.
attn_implementation="flash_attn_legacy" is compared with transformers' own "eager"
attention on the same weights: prefill logits, one cached decode step (which runs
the split-K decode kernel), generate, and gradients."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def tiny_llama(impl):
    import flash_attn_legacy  # noqa: F401  (registers the implementation)
    from transformers import LlamaConfig, LlamaForCausalLM
    cfg = LlamaConfig(vocab_size=256, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, max_position_embeddings=512,
                      rms_norm_eps=1e-5)
    cfg._attn_implementation = impl
    torch.manual_seed(0)
    return LlamaForCausalLM(cfg).cuda().half()


@pytest.fixture(scope="module")
def models():
    flash = tiny_llama("flash_attn_legacy")
    eager = tiny_llama("eager")
    eager.load_state_dict(flash.state_dict())
    flash.eval()
    eager.eval()
    return flash, eager


def cos(a, b):
    return torch.nn.functional.cosine_similarity(a.float().reshape(1, -1), b.float().reshape(1, -1)).item()


def test_prefill_logits_match_eager(models):
    flash, eager = models
    ids = torch.randint(0, 256, (2, 96), device="cuda", generator=torch.Generator("cuda").manual_seed(1))
    with torch.no_grad():
        a = flash(ids).logits
        b = eager(ids).logits
    assert torch.isfinite(a).all()
    assert cos(a, b) > 0.9999
    assert (a.float() - b.float()).abs().max().item() < 0.05


def test_cached_decode_step_uses_decode_kernel(models, monkeypatch):
    from flash_attn_legacy import hip_ext
    flash, eager = models
    calls = []
    real = hip_ext.decode
    monkeypatch.setattr(hip_ext, "decode", lambda *a, **k: calls.append(1) or real(*a, **k))
    ids = torch.randint(0, 256, (2, 40), device="cuda", generator=torch.Generator("cuda").manual_seed(2))
    nxt = torch.randint(0, 256, (2, 1), device="cuda", generator=torch.Generator("cuda").manual_seed(3))
    with torch.no_grad():
        pa = flash(ids, use_cache=True)
        la = flash(nxt, past_key_values=pa.past_key_values, use_cache=True).logits
        pb = eager(ids, use_cache=True)
        lb = eager(nxt, past_key_values=pb.past_key_values, use_cache=True).logits
    assert len(calls) == 2          # one decode call per layer
    assert cos(la, lb) > 0.9999
    assert (la.float() - lb.float()).abs().max().item() < 0.05


def test_generate(models):
    flash, _ = models
    ids = torch.randint(0, 256, (1, 8), device="cuda", generator=torch.Generator("cuda").manual_seed(4))
    with torch.no_grad():
        out = flash.generate(ids, max_new_tokens=16, do_sample=False)
    assert out.shape[1] == 8 + 16


@pytest.mark.parametrize("seq_len", [1, 16, 64, 128, 256])
def test_different_seq_lengths(models, seq_len):
    flash, _ = models
    ids = torch.randint(0, 256, (1, seq_len), device="cuda")
    with torch.no_grad():
        out = flash(ids)
    assert out.logits.shape == (1, seq_len, 256) and torch.isfinite(out.logits).all()


def test_backward_matches_eager():
    flash = tiny_llama("flash_attn_legacy")
    eager = tiny_llama("eager")
    eager.load_state_dict(flash.state_dict())
    ids = torch.randint(0, 256, (1, 64), device="cuda", generator=torch.Generator("cuda").manual_seed(5))
    la = flash(ids, labels=ids).loss
    lb = eager(ids, labels=ids).loss
    assert abs(la.item() - lb.item()) < 1e-2
    la.backward()
    lb.backward()
    pa = dict(flash.named_parameters())
    for name, p in eager.named_parameters():
        if p.grad is not None and "self_attn" in name:
            assert cos(pa[name].grad, p.grad) > 0.999, name


def test_llama_monkey_patch_example(models):
    """examples/hf_llama_patch.py (reference examples/hf_llama_patch.py:18-130): the patched
    model's prefill and cached decode logits match eager attention on the same weights."""
    import importlib.util, os
    path = os.path.join(os.path.dirname(__file__), "..", "flash-attention-legacy_amd", "examples", "hf_llama_patch.py")
    spec = importlib.util.spec_from_file_location("hf_llama_patch", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    _, eager = models
    patched = tiny_llama("eager")
    patched.load_state_dict(eager.state_dict())
    patched.eval()
    mod.patch_llama_attention(patched)
    ids = torch.randint(0, 256, (2, 50), device="cuda", generator=torch.Generator("cuda").manual_seed(6))
    nxt = torch.randint(0, 256, (2, 1), device="cuda", generator=torch.Generator("cuda").manual_seed(7))
    with torch.no_grad():
        pa = patched(ids, use_cache=True)
        pb = eager(ids, use_cache=True)
        assert cos(pa.logits, pb.logits) > 0.9999
        la = patched(nxt, past_key_values=pa.past_key_values, use_cache=True).logits
        lb = eager(nxt, past_key_values=pb.past_key_values, use_cache=True).logits
    assert cos(la, lb) > 0.9999
    assert (la.float() - lb.float()).abs().max().item() < 0.05


def padded_batch(seed):
    """Two left-padded prompts of 80 tokens (30 and 0 pad tokens) and their mask."""
    g = torch.Generator("cuda").manual_seed(seed)
    ids = torch.randint(0, 256, (2, 80), device="cuda", generator=g)
    mask = torch.ones_like(ids)
    mask[0, :30] = 0
    return ids, mask


def test_padded_prefill_matches_eager(models):
    """A padded batch: transformers passes this implementation the 2-D padding mask
    (FlashAttention-2's mask function is registered for it), prefill runs the varlen
    kernel over the real tokens, and the logits of real tokens match eager attention's."""
    flash, eager = models
    ids, mask = padded_batch(6)
    with torch.no_grad():
        a = flash(ids, attention_mask=mask).logits
        b = eager(ids, attention_mask=mask).logits
    real = mask.bool()
    assert torch.isfinite(a[real]).all()
    assert cos(a[real], b[real]) > 0.9999
    assert (a[real].float() - b[real].float()).abs().max().item() < 0.05
    # the padding changes the first sequence's result: it is not attended
    with torch.no_grad():
        c = flash(ids).logits
    assert (a[0, -1].float() - c[0, -1].float()).abs().max().item() > 0.05


def test_padded_cached_decode_matches_eager(models, monkeypatch):
    """Decode step after a padded prefill: the mask's last row becomes the decode
    kernel's additive bias."""
    from flash_attn_legacy import hip_ext
    flash, eager = models
    calls = []
    real = hip_ext.decode
    monkeypatch.setattr(hip_ext, "decode", lambda *a, **k: calls.append(k.get("mask_bias")) or real(*a, **k))
    ids, mask = padded_batch(7)
    nxt = torch.randint(0, 256, (2, 1), device="cuda", generator=torch.Generator("cuda").manual_seed(8))
    mask2 = torch.cat([mask, torch.ones_like(nxt)], dim=1)
    with torch.no_grad():
        pa = flash(ids, attention_mask=mask, use_cache=True)
        la = flash(nxt, attention_mask=mask2, past_key_values=pa.past_key_values, use_cache=True).logits
        pb = eager(ids, attention_mask=mask, use_cache=True)
        lb = eager(nxt, attention_mask=mask2, past_key_values=pb.past_key_values, use_cache=True).logits
    assert len(calls) == 2 and all(b is not None for b in calls)
    assert cos(la, lb) > 0.9999
    assert (la.float() - lb.float()).abs().max().item() < 0.05


def test_padded_backward_matches_eager():
    flash = tiny_llama("flash_attn_legacy")
    eager = tiny_llama("eager")
    eager.load_state_dict(flash.state_dict())
    ids, mask = padded_batch(9)
    # causal-LM labels shift by one: the last padded position (29) would predict the
    # first real token; its output is padding's (zeros here, eager attention's
    # uniform average there), so that label is masked too
    labels = ids.masked_fill(mask == 0, -100)
    labels[0, 30] = -100
    la = flash(ids, attention_mask=mask, labels=labels).loss
    lb = eager(ids, attention_mask=mask, labels=labels).loss
    assert abs(la.item() - lb.item()) < 1e-2
    la.backward()
    lb.backward()
    pa = dict(flash.named_parameters())
    for name, p in eager.named_parameters():
        if p.grad is not None and "self_attn" in name:
            assert cos(pa[name].grad, p.grad) > 0.999, name


@pytest.mark.parametrize("causal", [True, False])
def test_padded_prefill_attention_against_fp32(causal):
    """The integration's padded-prefill branch on its own: output and q/k/v gradients
    of the real rows against fp32 attention with the padding mask (keys masked out,
    causal over positions), GQA 8/2, head_dim 64."""
    import math
    from flash_attn_legacy.integrations import flash_attn_legacy_forward
    g = torch.Generator().manual_seed(10)
    B, Hq, Hk, N, d = 3, 8, 2, 72, 64
    q = torch.randn(B, Hq, N, d, generator=g).half().cuda().requires_grad_(True)
    k = torch.randn(B, Hk, N, d, generator=g).half().cuda().requires_grad_(True)
    v = torch.randn(B, Hk, N, d, generator=g).half().cuda().requires_grad_(True)
    keep = torch.ones(B, N, dtype=torch.bool)
    keep[0, :20] = False            # left padding
    keep[2, 50:] = False            # right padding
    mod = type("M", (), {"is_causal": causal})()
    o, _ = flash_attn_legacy_forward(mod, q, k, v, keep.cuda(), scaling=1 / math.sqrt(d))
    do = torch.randn(B, N, Hq, d, generator=g).half().cuda()
    o.backward(do)

    qf, kf, vf = (t.detach().float().cpu().requires_grad_(True) for t in (q, k, v))
    kr, vr = kf.repeat_interleave(Hq // Hk, 1), vf.repeat_interleave(Hq // Hk, 1)
    s = qf @ kr.transpose(-1, -2) / math.sqrt(d)
    allowed = keep[:, None, None, :].expand(B, 1, N, N)
    if causal:
        allowed = allowed & torch.ones(N, N, dtype=torch.bool).tril()
    # fully masked (padded) query rows get finite uniform weights; they carry no gradient
    p = torch.softmax(s.masked_fill(~allowed, -1e9), -1)
    ref = (p @ vr).transpose(1, 2)                      # [B, N, H, d]
    real = keep
    ref[real].backward(do.float().cpu()[real])
    out = o.detach().float().cpu()
    assert (out[real] - ref[real].detach()).abs().max().item() < 2e-3
    assert (out[~real] == 0).all()
    for name, a, r in (("dq", q.grad, qf.grad), ("dk", k.grad, kf.grad), ("dv", v.grad, vf.grad)):
        a = a.float().cpu()
        err = ((a - r).norm() / r.norm()).item()
        assert err < 1e-2, (name, err)

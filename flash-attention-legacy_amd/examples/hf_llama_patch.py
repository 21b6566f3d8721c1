"""
Monkey-patch the attention layers of a HuggingFace LLaMA model to run on
flash_attn_legacy (MI355X build).  Same entry point and behaviour as the
reference example (examples/hf_llama_patch.py:18-130), with one change: decode
steps (q_len < kv_len) run the split-K decode kernel over the DynamicCache
instead of an fp32 matmul/softmax/matmul with GQA repeat_interleave
(reference examples/hf_llama_patch.py:95-103).

    python examples/hf_llama_patch.py --model /path/to/local/llama --prompt "Hello"
"""

import argparse
import math
from typing import Optional, Tuple

import torch


def patch_llama_attention(model):
    """Replace every LLaMA attention layer's forward with one that calls
    flash_attention for prefill and flash_attn_with_kvcache for single-token
    decode.  GQA is handled by the kernels' head mapping.  Returns the model."""
    from flash_attn_legacy import flash_attention, flash_attn_with_kvcache
    from transformers.models.llama.modeling_llama import apply_rotary_pos_emb

    def make_flash_forward(attn):
        def flash_forward(hidden_states: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                          position_ids: Optional[torch.LongTensor] = None, past_key_value=None,
                          past_key_values=None, output_attentions: bool = False, use_cache: bool = False,
                          position_embeddings: Optional[Tuple] = None, **kwargs):
            bsz, q_len, _ = hidden_states.size()
            cache = past_key_values if past_key_values is not None else past_key_value
            cfg = attn.config
            n_heads = getattr(attn, "num_heads", None) or cfg.num_attention_heads
            n_kv = getattr(attn, "num_key_value_heads", None) or cfg.num_key_value_heads
            head_dim = getattr(attn, "head_dim", None) or cfg.hidden_size // n_heads

            q = attn.q_proj(hidden_states).view(bsz, q_len, n_heads, head_dim).transpose(1, 2)
            k = attn.k_proj(hidden_states).view(bsz, q_len, n_kv, head_dim).transpose(1, 2)
            v = attn.v_proj(hidden_states).view(bsz, q_len, n_kv, head_dim).transpose(1, 2)
            if position_embeddings is not None:
                cos, sin = position_embeddings
            else:
                cos, sin = attn.rotary_emb(v, position_ids)
            q, k = apply_rotary_pos_emb(q, k, cos, sin)

            if cache is not None and hasattr(cache, "update"):
                k, v = cache.update(k, v, attn.layer_idx)
            elif cache is not None:                       # legacy tuple cache
                k = torch.cat([cache[0], k], dim=2)
                v = torch.cat([cache[1], v], dim=2)

            scale = 1.0 / math.sqrt(head_dim)
            # fp16 and bf16 run natively; other dtypes are cast to fp16
            half = lambda t: t if t.dtype in (torch.float16, torch.bfloat16) else t.half()
            kv_len = k.shape[2]
            if q_len == 1 and kv_len > 1:
                # decode: [B, H_q, d] query against the [B, H_kv, S, d] cache
                o = flash_attn_with_kvcache(half(q)[:, :, 0, :], half(k), half(v), kv_len,
                                            softmax_scale=scale, cache_layout="bhsd")
                out = o.unsqueeze(1)                       # [B, 1, H_q, d]
            else:
                # prefill is causal; a multi-token chunk against a longer cache attends to
                # all of it, as the reference's unmasked else-branch does
                out = flash_attention(half(q), half(k), half(v), softmax_scale=scale,
                                      is_causal=q_len == kv_len).transpose(1, 2)
            out = out.to(hidden_states.dtype).contiguous().view(bsz, q_len, -1)
            return attn.o_proj(out), None

        return flash_forward

    patched = 0
    for _, module in model.named_modules():
        if module.__class__.__name__ in ("LlamaAttention", "LlamaSdpaAttention", "LlamaFlashAttention2"):
            module.forward = make_flash_forward(module)
            patched += 1
    print(f"Patched {patched} attention layers with flash_attn_legacy")
    return model


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--model", type=str, required=True, help="local path of a LLaMA checkpoint")
    ap.add_argument("--prompt", type=str, default="The meaning of life is")
    ap.add_argument("--max-new-tokens", type=int, default=50)
    a = ap.parse_args()

    from flash_attn_legacy import check_gpu_compatibility
    check_gpu_compatibility()
    from transformers import AutoModelForCausalLM, AutoTokenizer

    tok = AutoTokenizer.from_pretrained(a.model)
    model = AutoModelForCausalLM.from_pretrained(a.model, torch_dtype=torch.float16, device_map="cuda")
    patch_llama_attention(model)
    ids = tok(a.prompt, return_tensors="pt").to("cuda")
    with torch.no_grad():
        out = model.generate(**ids, max_new_tokens=a.max_new_tokens, do_sample=False)
    print(tok.decode(out[0], skip_special_tokens=True))


if __name__ == "__main__":
    main()

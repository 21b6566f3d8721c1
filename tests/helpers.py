"""Test helpers: seeded inputs, the oracle on device tensors, error metrics.

Inputs follow the benchmark configurations: fp16 drawn i.i.d. N(0,1) (times an
optional factor) from a seeded generator on the CPU, then copied to the device.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import attention as orc

FWD_ATOL = 2e-3      # forward: max |O - O_ref| against the fp32/fp64 closed form
GRAD_RTOL = 1e-2     # backward: max |g - g_ref| / max |g_ref| per gradient


def randn(shape, seed, scale=1.0, device="cuda"):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=g, dtype=torch.float32) * scale).half()
    return x.to(device) if device is not None else x


def np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def max_abs(a, b) -> float:
    a = a.detach().float().cpu() if isinstance(a, torch.Tensor) else torch.as_tensor(a).float()
    b = b.detach().float().cpu() if isinstance(b, torch.Tensor) else torch.as_tensor(b).float()
    return float((a - b).abs().max()) if a.numel() else 0.0


def rel_err(g, ref) -> float:
    """max |g - ref| / max |ref| (0 if ref is identically zero and g matches)."""
    g = g.detach().float().cpu() if isinstance(g, torch.Tensor) else torch.as_tensor(g).float()
    ref = ref.detach().float().cpu() if isinstance(ref, torch.Tensor) else torch.as_tensor(ref).float()
    den = float(ref.abs().max()) if ref.numel() else 0.0
    num = float((g - ref).abs().max()) if g.numel() else 0.0
    return num / den if den > 0 else num


def oracle_fwd(q, k, v, scale, causal):
    o, lse = orc.attention_fwd(np64(q), np64(k), np64(v), scale, causal)
    return torch.from_numpy(o), torch.from_numpy(lse)


def oracle_bwd(q, k, v, do, scale, causal):
    dq, dk, dv = orc.attention_bwd(np64(q), np64(k), np64(v), np64(do), scale, causal)
    return torch.from_numpy(dq), torch.from_numpy(dk), torch.from_numpy(dv)


def cu_from_lens(lens, device="cuda"):
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + int(n))
    return torch.tensor(cu, dtype=torch.int32, device=device)

"""fal_decode_noalloc through the C ABI: the same results as fal_decode, which takes
a caller workspace, on two calls in a row (the second smaller, so it reuses the
fixed device array the first one wrote), and a clear error above the array's size.
"""

import ctypes
import math

import pytest
import torch

from helpers import randn

pytestmark = pytest.mark.gpu

FAL_ERR_WORKSPACE = 4


def _noalloc(q, kc, vc, seqlens, scale, bias=None, want_lse=True):
    from flash_attn_legacy import hip_ext
    B, Hq, d = q.shape
    S, Hkv = kc.shape[1], kc.shape[2]
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=q.device) if want_lse else None
    s3 = lambda t, dims: (ctypes.c_int64 * 3)(*[t.stride()[i] if i is not None else 0 for i in dims])
    rc = hip_ext._lib.fal_decode_noalloc(
        q.data_ptr(), kc.data_ptr(), vc.data_ptr(), seqlens.data_ptr(),
        bias.data_ptr() if bias is not None else None, bias.stride(0) if bias is not None else 0,
        o.data_ptr(), lse.data_ptr() if lse is not None else None,
        B, Hq, Hkv, d, S, s3(q, (0, 1, None)), s3(kc, (0, 2, 1)), s3(vc, (0, 2, 1)), s3(o, (0, 1, None)),
        ctypes.c_float(scale), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, hip_ext._lib.fal_last_error().decode()
    return o, lse


def _case(B, Hq, Hkv, S, d, seed, with_bias):
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(1, S + 1, (B,), generator=g)
    lens[0] = S
    q = randn((B, Hq, d), seed=seed + 1)
    kc, vc = randn((B, S, Hkv, d), seed=seed + 2), randn((B, S, Hkv, d), seed=seed + 3)
    seq = lens.to(torch.int32).cuda()
    bias = (torch.randn((B, S), generator=g) * 2).cuda() if with_bias else None
    return q, kc, vc, seq, bias


def test_noalloc_matches_workspace_entry_point_twice():
    from flash_attn_legacy import hip_ext
    cases = [(8, 32, 8, 6000, 128, 1, True), (3, 8, 2, 700, 64, 2, False)]   # second call smaller
    for B, Hq, Hkv, S, d, seed, with_bias in cases:
        print(f"noalloc case B={B} Hq={Hq} Hkv={Hkv} S={S} d={d}", flush=True)
        q, kc, vc, seq, bias = _case(B, Hq, Hkv, S, d, seed, with_bias)
        scale = 1.0 / math.sqrt(d)
        ref_o, ref_l = hip_ext.decode(q, kc, vc, seq, scale, mask_bias=bias, return_lse=True)
        o, lse = _noalloc(q, kc, vc, seq, scale, bias)
        torch.cuda.synchronize()
        assert torch.equal(o, ref_o)
        assert torch.equal(lse, ref_l)


def test_noalloc_rejects_oversized_calls():
    """A call whose workspace would pass the array's 16 MiB fails with FAL_ERR_WORKSPACE.
    Every pointer is a real device buffer that a launch could use safely (cache lengths 0,
    zero K/V strides onto one row), so a regression in the order of the checks would
    show as a failed assertion, not as a launch on invalid addresses."""
    from flash_attn_legacy import hip_ext
    B, Hq, Hkv, S, d = 64, 64, 8, 1 << 17, 128
    need = hip_ext._lib.fal_decode_workspace_size(B, Hq, Hkv, S, d)
    assert need > 16 << 20
    q = torch.zeros((B, Hq, d), dtype=torch.float16, device="cuda")
    o = torch.empty_like(q)
    lse = torch.empty((B, Hq), dtype=torch.float32, device="cuda")
    row = torch.zeros((d,), dtype=torch.float16, device="cuda")     # every K/V address lands here
    seq = torch.zeros((B,), dtype=torch.int32, device="cuda")
    qs = (ctypes.c_int64 * 3)(Hq * d, d, 0)
    kvs = (ctypes.c_int64 * 3)(0, 0, 0)
    rc = hip_ext._lib.fal_decode_noalloc(q.data_ptr(), row.data_ptr(), row.data_ptr(), seq.data_ptr(), None, 0,
                                         o.data_ptr(), lse.data_ptr(), B, Hq, Hkv, d, S,
                                         qs, kvs, kvs, qs, ctypes.c_float(0.1),
                                         ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    assert rc == FAL_ERR_WORKSPACE
    assert "16777216" in hip_ext._lib.fal_last_error().decode()

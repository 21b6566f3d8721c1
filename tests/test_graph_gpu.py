"""The kernels' launch sequences contain no memset or host synchronisation, so a
caller can capture them in a HIP graph.  Each entry point is captured once and the
graph is replayed several times, with eager work and synchronisations between the
replays; every replay must reproduce the eager result bit for bit."""

import math

import pytest
import torch

from helpers import randn

pytestmark = pytest.mark.gpu


def replay_check(fn, eager_out, n=4, inexact=()):
    """`inexact`: indices of outputs accumulated with atomics (d 256 dQ), compared to
    within 1e-3 of their largest magnitude instead of bit for bit."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()   # warm-up on the capture stream (allocator pools)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = fn()
    for r in range(n):
        # unrelated eager work between replays
        junk = torch.randn(1 << 20, device="cuda").sum()
        torch.cuda.synchronize()
        for t in outs:
            t.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for idx, (got, ref) in enumerate(zip(outs, eager_out)):
            if idx in inexact:
                tol = 1e-3 * float(ref.float().abs().max())
                assert float((got.float() - ref.float()).abs().max()) <= tol, f"replay {r}, output {idx}"
                continue
            same = torch.equal(got, ref) or (torch.equal(torch.isnan(got), torch.isnan(ref)) and
                                             torch.equal(torch.nan_to_num(got), torch.nan_to_num(ref)))
            assert same, (f"replay {r}, output {idx}: nan {int(torch.isnan(got).sum())} vs "
                          f"{int(torch.isnan(ref).sum())}, max diff "
                          f"{float((torch.nan_to_num(got).float() - torch.nan_to_num(ref).float()).abs().max())}")
        del junk


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("d", [128, 256])
def test_graph_forward_backward(dtype, d):
    """d 128 takes the split backward (two kernels), d 256 the atomic one (D and the
    zeroed fp32 dQ accumulator from a kernel, the cast after it)."""
    from flash_attn_legacy import hip_ext
    B, Hq, Hkv, N = 2, 8, 2, 384
    q, k, v, do = (randn(shape, seed=s).to(dtype) for shape, s in
                   (((B, Hq, N, d), 1), ((B, Hkv, N, d), 2), ((B, Hkv, N, d), 3), ((B, Hq, N, d), 4)))
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, True)
    grads = hip_ext.backward(do, q, k, v, o, lse, scale, True)
    torch.cuda.synchronize()
    replay_check(lambda: tuple(hip_ext.forward(q, k, v, scale, True)), (o, lse))
    replay_check(lambda: tuple(hip_ext.backward(do, q, k, v, o, lse, scale, True)), tuple(grads),
                 inexact=(0,) if d == 256 else ())


def test_graph_varlen_and_decode():
    from flash_attn_legacy import hip_ext
    lens = [5, 130, 257, 64]
    cu = torch.tensor([0, 5, 135, 392, 456], dtype=torch.int32, device="cuda")
    tot = sum(lens)
    q, k, v = randn((tot, 8, 64), seed=5), randn((tot, 4, 64), seed=6), randn((tot, 4, 64), seed=7)
    o, lse = hip_ext.forward_varlen(q, k, v, cu, cu, max(lens), max(lens), 0.125, True)
    replay_check(lambda: tuple(hip_ext.forward_varlen(q, k, v, cu, cu, max(lens), max(lens), 0.125, True)), (o, lse))
    seq = torch.tensor([1, 700, 3000, 129], dtype=torch.int32, device="cuda")
    qd = randn((4, 16, 128), seed=8)
    kc, vc = randn((4, 3000, 4, 128), seed=9), randn((4, 3000, 4, 128), seed=10)
    od, ld = hip_ext.decode(qd, kc, vc, seq, 0.088, return_lse=True)
    replay_check(lambda: tuple(hip_ext.decode(qd, kc, vc, seq, 0.088, return_lse=True)), (od, ld))


@pytest.mark.parametrize("hkv", [8, 32])
def test_graph_persistent_forward(hkv):
    """Batched head-dim-128 forward on the persistent grid (four heads per workgroup for
    32/8, 256-row items for MHA), captured and replayed."""
    from flash_attn_legacy import hip_ext
    B, Hq, N, d = 2, 32, 2048, 128
    q = randn((B, Hq, N, d), seed=11)
    k, v = randn((B, hkv, N, d), seed=12), randn((B, hkv, N, d), seed=13)
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, True)
    replay_check(lambda: hip_ext.forward(q, k, v, scale, True), (o, lse))


def test_graph_varlen_pair_walk_and_backward():
    """More than 64 packed sequences at head dim 128 with 8/2 heads: the schedule kernel
    builds the pair list on the device, the four-heads forward walks it, and the
    one-launch varlen backward builds its own lists; all captured and replayed."""
    from flash_attn_legacy import hip_ext
    g = torch.Generator().manual_seed(14)
    lens = [int(x) for x in torch.randint(1, 300, (70,), generator=g)]
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0)), dtype=torch.int32, device="cuda")
    tot, mx = sum(lens), max(lens)
    q, k, v = randn((tot, 8, 128), seed=15), randn((tot, 2, 128), seed=16), randn((tot, 2, 128), seed=17)
    do = randn((tot, 8, 128), seed=18)
    scale = 1.0 / math.sqrt(128)
    assert hip_ext._lib.fal_fwd_varlen_workspace_size(len(lens), tot, mx, 128) > 0   # the list path
    o, lse = hip_ext.forward_varlen(q, k, v, cu, cu, mx, mx, scale, True)
    grads = hip_ext.backward_varlen(do, q, k, v, o, lse, cu, cu, mx, mx, scale, True)
    torch.cuda.synchronize()
    replay_check(lambda: tuple(hip_ext.forward_varlen(q, k, v, cu, cu, mx, mx, scale, True)), (o, lse))
    replay_check(lambda: tuple(hip_ext.backward_varlen(do, q, k, v, o, lse, cu, cu, mx, mx, scale, True)),
                 tuple(grads))

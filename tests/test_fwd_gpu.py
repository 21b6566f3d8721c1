"""Forward parity on the GPU: the HIP kernel against the CPU oracle.

Cases follow the reference's tests/test_flash_attn.py (TestForwardMHA :79-138,
TestForwardGQA :145-193, TestLongSequences :486-547, TestNumericalStability
:593-676) with seeded inputs and the stricter bound max|O - O_ref| <= 2e-3
(fp64 oracle), plus the benchmark configurations C1 and C2.
"""

import math

import numpy as np

import pytest
import torch

from helpers import FWD_ATOL, max_abs, np64, oracle_fwd, randn

pytestmark = pytest.mark.gpu

HEAD_DIMS = [32, 64, 96, 128, 256]


def fa():
    from flash_attn_legacy import flash_attention
    return flash_attention


def ext():
    from flash_attn_legacy import hip_ext
    return hip_ext


@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N", [32, 64, 128, 256, 512])
def test_seq_lengths(d, causal, N):
    B, H = 2, 4
    scale = 1.0 / math.sqrt(d)
    q, k, v = (randn((B, H, N, d), seed=s, scale=0.3) for s in (1, 2, 3))
    out = fa()(q, k, v, softmax_scale=scale, is_causal=causal)
    ref, _ = oracle_fwd(q, k, v, scale, causal)
    assert max_abs(out, ref) <= FWD_ATOL


@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("N", [1, 33, 65, 100, 200])
@pytest.mark.parametrize("causal", [False, True])
def test_non_power_of_2_and_lse(d, N, causal):
    B, H = 1, 2
    scale = 1.0 / math.sqrt(d)
    q, k, v = (randn((B, H, N, d), seed=s) for s in (4, 5, 6))
    o, lse = ext().forward(q, k, v, scale, causal)
    ref_o, ref_lse = oracle_fwd(q, k, v, scale, causal)
    assert max_abs(o, ref_o) <= FWD_ATOL
    assert max_abs(lse, ref_lse) <= 1e-3


@pytest.mark.parametrize("d", HEAD_DIMS)
def test_deterministic(d):
    q, k, v = (randn((1, 4, 256, d), seed=s) for s in (7, 8, 9))
    assert torch.equal(fa()(q, k, v), fa()(q, k, v))


@pytest.mark.parametrize("d", HEAD_DIMS)
def test_single_token_is_v(d):
    q, k, v = (randn((2, 4, 1, d), seed=s) for s in (10, 11, 12))
    out = fa()(q, k, v)
    torch.testing.assert_close(out, v, rtol=0, atol=1e-3)


@pytest.mark.parametrize("d", HEAD_DIMS)
def test_uniform_attention(d):
    q = torch.zeros(1, 1, 64, d, device="cuda", dtype=torch.float16)
    k = torch.zeros_like(q)
    v = randn((1, 1, 64, d), seed=13, scale=0.1)
    out = fa()(q, k, v)
    expected = v.float().mean(dim=2, keepdim=True).expand_as(v)
    assert max_abs(out, expected) <= FWD_ATOL


@pytest.mark.parametrize("d", HEAD_DIMS)
def test_batch_independence(d):
    B, H, N = 4, 2, 128
    scale = 1.0 / math.sqrt(d)
    q, k, v = (randn((B, H, N, d), seed=s, scale=0.3) for s in (14, 15, 16))
    full = fa()(q, k, v, softmax_scale=scale)
    for b in range(B):
        single = fa()(q[b:b + 1], k[b:b + 1], v[b:b + 1], softmax_scale=scale)
        torch.testing.assert_close(full[b:b + 1], single, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("hq,hkv", [(8, 2), (8, 4), (8, 1), (4, 1), (4, 2)])
@pytest.mark.parametrize("causal", [False, True])
def test_gqa(d, hq, hkv, causal):
    B, N = 2, 128
    scale = 1.0 / math.sqrt(d)
    q = randn((B, hq, N, d), seed=17, scale=0.3)
    k = randn((B, hkv, N, d), seed=18, scale=0.3)
    v = randn((B, hkv, N, d), seed=19, scale=0.3)
    out = fa()(q, k, v, softmax_scale=scale, is_causal=causal)
    ref, _ = oracle_fwd(q, k, v, scale, causal)
    assert max_abs(out, ref) <= FWD_ATOL


@pytest.mark.parametrize("d", HEAD_DIMS)
def test_mqa_equals_broadcast(d):
    B, Hq, N = 2, 8, 128
    q = randn((B, Hq, N, d), seed=20, scale=0.3)
    k = randn((B, 1, N, d), seed=21, scale=0.3)
    v = randn((B, 1, N, d), seed=22, scale=0.3)
    out_mqa = fa()(q, k, v)
    out_mha = fa()(q, k.expand(B, Hq, N, d), v.expand(B, Hq, N, d))
    torch.testing.assert_close(out_mqa, out_mha, rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("d", HEAD_DIMS)
def test_causal_first_row(d):
    q, k = (randn((1, 2, 64, d), seed=s, scale=0.3) for s in (23, 24))
    v = randn((1, 2, 64, d), seed=25)
    out = fa()(q, k, v, is_causal=True)
    torch.testing.assert_close(out[:, :, 0], v[:, :, 0], rtol=0, atol=1e-3)


@pytest.mark.parametrize("d", HEAD_DIMS)
def test_large_and_small_values(d):
    scale = 1.0 / math.sqrt(d)
    q, k = (randn((1, 2, 128, d), seed=s, scale=5.0) for s in (26, 27))
    v = randn((1, 2, 128, d), seed=28, scale=0.1)
    out = fa()(q, k, v, softmax_scale=scale)
    assert torch.isfinite(out).all()
    ref, _ = oracle_fwd(q, k, v, scale, False)
    assert max_abs(out, ref) <= FWD_ATOL
    q, k = (randn((1, 2, 128, d), seed=s, scale=1e-3) for s in (29, 30))
    v = randn((1, 2, 128, d), seed=31, scale=0.5)
    out = fa()(q, k, v)
    assert max_abs(out, v.float().mean(dim=2, keepdim=True).expand_as(v)) <= FWD_ATOL


@pytest.mark.parametrize("d", [64, 128])
def test_custom_and_negative_scale(d):
    q, k, v = (randn((1, 2, 64, d), seed=s, scale=0.3) for s in (32, 33, 34))
    for scale in (0.01, 1.0, -0.2):
        out = fa()(q, k, v, softmax_scale=scale, is_causal=True)
        ref, _ = oracle_fwd(q, k, v, scale, True)
        assert max_abs(out, ref) <= FWD_ATOL


@pytest.mark.parametrize("d", [64, 128])
def test_strided_inputs_no_copy(d):
    """[B, N, H, d] storage viewed as [B, H, N, d] (the HF / module layout)."""
    B, N, H = 2, 96, 4
    base = randn((3, B, N, H, d), seed=35)
    q, k, v = (base[i].transpose(1, 2) for i in range(3))
    out = fa()(q, k, v, is_causal=True)
    ref, _ = oracle_fwd(q, k, v, 1.0 / math.sqrt(d), True)
    assert max_abs(out, ref) <= FWD_ATOL


@pytest.mark.parametrize("nq,nk", [(64, 200), (200, 64), (1, 77)])
@pytest.mark.parametrize("causal", [False, True])
def test_unequal_lengths_top_left(nq, nk, causal):
    d = 64
    q = randn((1, 4, nq, d), seed=36)
    k, v = (randn((1, 2, nk, d), seed=s) for s in (37, 38))
    o, lse = ext().forward(q, k, v, 0.125, causal)
    ref_o, ref_lse = oracle_fwd(q, k, v, 0.125, causal)
    assert max_abs(o, ref_o) <= FWD_ATOL
    assert max_abs(lse, ref_lse) <= 1e-3


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("N", [1024, 2048, 4096])
def test_long_sequences(d, N):
    q, k, v = (randn((1, 2, N, d), seed=s) for s in (39, 40, 41))
    out = fa()(q, k, v, is_causal=True)
    assert torch.isfinite(out).all()
    from oracle.torch_ref import ref_attention
    ref = ref_attention(q.cpu(), k.cpu(), v.cpu(), 1.0 / math.sqrt(d), True)
    assert max_abs(out, ref) <= FWD_ATOL


def test_config_c1_full():
    """C1: B=2, H=8, N=1024, d=64, causal, N(0,1) inputs, seed 0."""
    B, H, N, d = 2, 8, 1024, 64
    q, k, v = (randn((B, H, N, d), seed=s) for s in (0, 1, 2))
    o, lse = ext().forward(q, k, v, 1.0 / math.sqrt(d), True)
    ref_o, ref_lse = oracle_fwd(q, k, v, 1.0 / math.sqrt(d), True)
    assert max_abs(o, ref_o) <= FWD_ATOL
    assert max_abs(lse, ref_lse) <= 1e-3


def cpu_oracle_group(q, k, v, scale, causal):
    """O and L (natural log) of one KV group from the CPU oracle's fp32 torch formula
    (the reference's closed form, tests/test_flash_attn.py:19-32, with
    L = m + ln(l) of flash_attn_fwd_volta.cu:343); q [1, G, Nq, d], k/v [1, 1, Nk, d]."""
    from oracle.torch_ref import ref_attention_lse
    torch.set_num_threads(max(torch.get_num_threads(), 8))
    return ref_attention_lse(q.cpu(), k.cpu(), v.cpu(), scale, causal)


def check_groups(o, lse, q, k, v, scale, causal, groups):
    """O within FWD_ATOL and L within 1e-3 of the CPU oracle for each (batch, KV group)."""
    G = q.shape[1] // k.shape[1]
    oc, lc = o.cpu(), lse.cpu()
    for b, g in groups:
        hs = slice(g * G, (g + 1) * G)
        ref_o, ref_l = cpu_oracle_group(q[b:b + 1, hs], k[b:b + 1, g:g + 1], v[b:b + 1, g:g + 1], scale, causal)
        assert max_abs(oc[b:b + 1, hs], ref_o) <= FWD_ATOL, (b, g)
        fin = torch.isfinite(ref_l)
        assert torch.equal(torch.isfinite(lc[b:b + 1, hs]), fin), (b, g)
        assert max_abs(lc[b:b + 1, hs][fin], ref_l[fin]) <= 1e-3, (b, g)


def test_config_c2_full_shape():
    """C2 at full size (B=4, 32q/8kv heads, N=4096, d=128, causal), the bench's headline
    call on the persistent four-heads grid: O and the per-row log-sum-exp of every one of
    the 32 (batch, KV group) slices against the CPU oracle in fp32."""
    B, Hq, Hkv, N, d = 4, 32, 8, 4096, 128
    q = randn((B, Hq, N, d), seed=0)
    k = randn((B, Hkv, N, d), seed=1)
    v = randn((B, Hkv, N, d), seed=2)
    scale = 1.0 / math.sqrt(d)
    o, lse = ext().forward(q, k, v, scale, True)
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    check_groups(o, lse, q, k, v, scale, True, [(b, g) for b in range(B) for g in range(Hkv)])


def exact_rows(q, k, v, rows, scale, causal):
    """float64 attention output and log-sum-exp (natural log) of the given query rows of
    one head (q [Nq, d], k/v [Nk, d]), the closed form of oracle/attention.py one row
    at a time, with top-left causal alignment."""
    qf, kf, vf = (np64(t) for t in (q, k, v))
    outs, lses = [], []
    for r in rows:
        kk = kf[: r + 1] if causal else kf
        vv = vf[: r + 1] if causal else vf
        s = kk @ qf[r] * scale
        m = s.max()
        p = np.exp(s - m)
        outs.append(p @ vv / p.sum())
        lses.append(m + np.log(p.sum()))
    return np.stack(outs), np.array(lses)


@pytest.mark.parametrize("causal,nq,nk", [(True, 32768, 32768), (False, 4000, 32768)])
def test_very_long_sequence_sampled_rows(causal, nq, nk):
    """N up to 32768 (beyond the dense oracle's reach): O and L of sampled rows, first,
    middle and last, against exact float64 rows; GQA with 2 query heads per KV head."""
    Hq, Hkv, d = 2, 1, 128
    q = randn((1, Hq, nq, d), seed=60)
    k, v = randn((1, Hkv, nk, d), seed=61), randn((1, Hkv, nk, d), seed=62)
    scale = 1.0 / math.sqrt(d)
    o, lse = ext().forward(q, k, v, scale, causal)
    rows = [0, 1, 63, 64, nq // 2 - 1, nq // 2 + 17, nq - 2, nq - 1]
    for h in range(Hq):
        ref_o, ref_l = exact_rows(q[0, h], k[0, 0], v[0, 0], rows, scale, causal)
        assert max_abs(o[0, h, rows], torch.from_numpy(ref_o)) <= FWD_ATOL, h
        assert float(np.abs(lse[0, h, rows].cpu().numpy() - ref_l).max()) <= 1e-3, h


@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("nq,nk", [(4096, 4096), (2000, 5000), (5000, 2000)])
def test_split_kv_small_grid(d, causal, nq, nk):
    """Grids smaller than the GPU split each query tile's key range over several
    workgroups and merge the partials (fal_fwd_workspace_size > 0 for these shapes);
    O and L must match the oracle as the unsplit kernel does."""
    from flash_attn_legacy import hip_ext
    B, hq, hkv = 1, 2, 1
    assert hip_ext._lib.fal_fwd_workspace_size(B, hq, nq, nk, d, int(causal)) > 0
    q = randn((B, hq, nq, d), seed=41)
    k, v = randn((B, hkv, nk, d), seed=42), randn((B, hkv, nk, d), seed=43)
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, causal)
    ref_o, ref_l = oracle_fwd(q, k, v, scale, causal)
    assert max_abs(o, ref_o) <= FWD_ATOL
    fin = torch.isfinite(ref_l)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert max_abs(lse.cpu()[fin], ref_l[fin]) <= 1e-3


def test_head_slice_beyond_2gib():
    """K/V stored with the heads interleaved in each row ([B, N, H, d] viewed as
    [B, H, N, d]) and N = 2^20 + 4096 keys: one head's rows span 2.15 GB, more than a
    buffer resource's 2^31-byte record count, so the copies must bound each tile
    separately.  Sampled rows of the first and last head against exact float64 rows."""
    Hkv, d, nq = 8, 128, 8192     # 256 workgroups: no split of the key range
    nk = (1 << 20) + 4096
    assert ext()._lib.fal_fwd_workspace_size(1, Hkv, nq, nk, d, 0) == 0
    g = torch.Generator(device="cuda").manual_seed(70)
    k = torch.randn((1, nk, Hkv, d), generator=g, device="cuda", dtype=torch.float16)
    v = torch.randn((1, nk, Hkv, d), generator=g, device="cuda", dtype=torch.float16)
    q = randn((1, Hkv, nq, d), seed=71)
    kv, vv = k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)
    assert kv.stride(2) * 2 * nk > 2 ** 31
    scale = 1.0 / math.sqrt(d)
    o, lse = ext().forward(q, kv, vv, scale, False)
    rows = [0, 4095, nq - 1]
    for h in (0, Hkv - 1):
        ref_o, ref_l = exact_rows(q[0, h], kv[0, h], vv[0, h], rows, scale, False)
        assert max_abs(o[0, h, rows], torch.from_numpy(ref_o)) <= FWD_ATOL, h
        assert float(np.abs(lse[0, h, rows].cpu().numpy() - ref_l).max()) <= 1e-3, h


def test_persistent_grid_negative_scale():
    """A negative softmax scale on the persistent grid: the sign is folded into Q, so the
    next item's Q slices are not loaded early; every head against the fp32 formula."""
    B, Hq, Hkv, N, d = 2, 16, 4, 4160, 128
    scale = -1.0 / math.sqrt(d)
    q, k, v = randn((B, Hq, N, d), seed=24), randn((B, Hkv, N, d), seed=25), randn((B, Hkv, N, d), seed=26)
    o, lse = ext().forward(q, k, v, scale, True)
    check_groups(o, lse, q, k, v, scale, True, [(b, g) for b in range(B) for g in range(Hkv)])


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk", [(2, 16, 4, 4160, 4160), (1, 32, 4, 4160, 4160),
                                            (2, 8, 2, 8192, 8192), (2, 16, 16, 4352, 4352),
                                            (2, 16, 8, 4352, 4352), (2, 16, 4, 4160, 5000),
                                            (2, 16, 4, 5000, 3000)])
def test_persistent_grid_every_head(B, Hq, Hkv, Nq, Nk, causal):
    """head_dim 128 with at least two items per CU runs the persistent grid (pairs of query
    tiles per workgroup; items of 64 rows of four heads when Hq/Hkv is a multiple of 4,
    else of 256 rows of one head; an odd tile count leaves the middle tile unpaired;
    Nq != Nk with top-left causal alignment): O and L of every row of every head against
    the CPU oracle."""
    d = 128
    scale = 1.0 / math.sqrt(d)
    q, k, v = randn((B, Hq, Nq, d), seed=21), randn((B, Hkv, Nk, d), seed=22), randn((B, Hkv, Nk, d), seed=23)
    o, lse = ext().forward(q, k, v, scale, causal)
    check_groups(o, lse, q, k, v, scale, causal, [(b, g) for b in range(B) for g in range(Hkv)])

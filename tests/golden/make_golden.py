"""Writes the golden vectors in this directory from the float64 oracle.

    python tests/golden/make_golden.py

The reference ships no golden vectors or fixtures for this path (its tests compare
against an fp32 closed form computed at run time), so these vectors are produced by
the oracle in oracle/attention.py, which tests/test_oracle.py pins against float64
autograd, brute-force loops, finite differences and closed forms.  Inputs are fp16
values (stored as float16) so the GPU path sees exactly the same numbers.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import attention as orc  # noqa: E402


def f16(rng, *shape, scale=1.0):
    return (rng.standard_normal(shape) * scale).astype(np.float16)


def f32(**arrays):
    return {k: (v.astype(np.float32) if isinstance(v, np.ndarray) and v.dtype == np.float64 else v)
            for k, v in arrays.items()}


def main():
    rng = np.random.default_rng(2024)
    # forward + backward, GQA 4:2, causal, N not a multiple of any tile
    q, k, v, do = f16(rng, 1, 4, 77, 64), f16(rng, 1, 2, 77, 64), f16(rng, 1, 2, 77, 64), f16(rng, 1, 4, 77, 64)
    o, lse = orc.attention_fwd(q, k, v, 0.125, True)
    dq, dk, dv = orc.attention_bwd(q, k, v, do, 0.125, True)
    np.savez_compressed(os.path.join(HERE, "fwd_bwd_gqa_causal_d64.npz"), **f32(q=q, k=k, v=v, do=do, scale=0.125,
                        causal=True, o=o, lse=lse, dq=dq, dk=dk, dv=dv))
    # non-causal MHA, d=128, unequal q / k lengths
    q, k, v = f16(rng, 2, 2, 19, 128), f16(rng, 2, 2, 45, 128), f16(rng, 2, 2, 45, 128)
    o, lse = orc.attention_fwd(q, k, v, 0.09, False)
    np.savez_compressed(os.path.join(HERE, "fwd_noncausal_d128_nq19_nk45.npz"), **f32(q=q, k=k, v=v, scale=0.09,
                        causal=False, o=o, lse=lse))
    # varlen, causal, with an empty and a one-token segment
    lens = [37, 0, 1, 90]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    q, k, v, do = f16(rng, cu[-1], 4, 64), f16(rng, cu[-1], 1, 64), f16(rng, cu[-1], 1, 64), f16(rng, cu[-1], 4, 64)
    o, lse = orc.varlen_fwd(q, k, v, cu, cu, 0.125, True)
    dq, dk, dv = orc.varlen_bwd(q, k, v, do, cu, cu, 0.125, True)
    np.savez_compressed(os.path.join(HERE, "varlen_causal_d64.npz"), **f32(q=q, k=k, v=v, do=do, cu=cu, scale=0.125,
                        causal=True, o=o, lse=lse, dq=dq, dk=dk, dv=dv))
    # decode, GQA 8:2, [B, S, Hkv, d] cache, lengths 150 / 1 / 67
    lens = np.array([150, 1, 67], dtype=np.int32)
    q, kc, vc = f16(rng, 3, 1, 8, 128), f16(rng, 3, 150, 2, 128), f16(rng, 3, 150, 2, 128)
    o, lse = orc.decode(q, kc, vc, lens, 0.088)
    np.savez_compressed(os.path.join(HERE, "decode_gqa_d128.npz"), **f32(q=q, k_cache=kc, v_cache=vc,
                        cache_seqlens=lens, scale=0.088, o=o, lse=lse))
    print("wrote golden vectors to", HERE)


if __name__ == "__main__":
    main()

"""ctypes binding of libfal_hip.so -- the drop-in for the reference's compiled
extension module ``flash_attn_legacy_cuda`` (csrc/flash_attn_legacy.cpp:294-310).

It exposes the reference's three functions with the same arguments, outputs and
error behaviour (``RuntimeError`` with the library's message):

* ``forward(Q, K, V, softmax_scale, is_causal=False) -> [O, L]``
* ``forward_varlen(Q, K, V, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
  softmax_scale, is_causal=False) -> [O, L]``
* ``backward(dO, Q, K, V, O, L, softmax_scale, is_causal=False) -> [dQ, dK, dV]``

plus two entry points the reference does not have:

* ``backward_varlen(...)`` -- one launch for all packed sequences;
* ``decode(q, k_cache, v_cache, cache_seqlens, softmax_scale, ...)`` -- split-K
  KV-cache decode.

Outputs and workspaces are allocated here with torch on the input's device; the
library itself never allocates.  Work is enqueued on the current torch stream.
There is no fallback: if the shared library is missing, importing this module
raises ``ImportError``.
"""

from __future__ import annotations

import ctypes
import os
from typing import List, Optional

import torch

_LIB_NAME = "libfal_hip.so"
# FLASH_ATTN_LEGACY_LIB selects another build of the same library (e.g. a tuning variant).
_LIB_PATH = os.environ.get("FLASH_ATTN_LEGACY_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)

_VP = ctypes.c_void_p
_I64 = ctypes.c_int64
_F32 = ctypes.c_float
_INT = ctypes.c_int
_SZ = ctypes.c_size_t
_STR = ctypes.c_void_p   # int64[3] stride triples, passed as arrays or byref(array, offset)


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        raise ImportError(
            f"flash_attn_legacy HIP library not found at {_LIB_PATH}. "
            "Build it with: python flash-attention-legacy_amd/build.py"
        )
    lib = ctypes.CDLL(_LIB_PATH)
    sig = {
        "fal_last_error": (ctypes.c_char_p, []),
        "fal_version": (ctypes.c_char_p, []),
        "fal_device_supported": (_INT, [_INT]),
        "fal_fwd_workspace_size": (_SZ, [_I64] * 5 + [_INT]),
        "fal_fwd": (_INT, [_VP] * 5 + [_I64] * 6 + [_STR] * 4 + [_F32, _INT, _VP, _SZ, _VP]),
        "fal_fwd_varlen_workspace_size": (_SZ, [_I64] * 4),
        "fal_fwd_varlen": (_INT, [_VP] * 7 + [_I64] * 8 + [_STR] * 4 + [_F32, _INT, _VP, _SZ, _VP]),
        "fal_bwd_workspace_size": (_SZ, [_I64] * 4),
        "fal_bwd": (_INT, [_VP] * 9 + [_I64] * 6 + [_STR] * 8 + [_F32, _INT, _VP, _SZ, _VP]),
        "fal_bwd_varlen_workspace_size": (_SZ, [_I64] * 5),
        "fal_bwd_varlen": (_INT, [_VP] * 11 + [_I64] * 8 + [_STR] * 8 + [_F32, _INT, _VP, _SZ, _VP]),
        "fal_decode_workspace_size": (_SZ, [_I64] * 5),
        "fal_decode": (_INT, [_VP] * 5 + [_I64, _VP, _VP] + [_I64] * 5 + [_STR] * 4 + [_F32, _VP, _SZ, _VP]),
        "fal_decode_noalloc": (_INT, [_VP] * 5 + [_I64, _VP, _VP] + [_I64] * 5 + [_STR] * 4 + [_F32, _VP]),
    }
    for name in ("fal_fwd", "fal_fwd_varlen", "fal_bwd", "fal_bwd_varlen", "fal_decode"):
        sig[name + "_bf16"] = sig[name]   # bf16 forms: same arguments
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()

# Exported names, for introspection and tests.
SYMBOLS = (
    "fal_last_error", "fal_version", "fal_device_supported",
    "fal_fwd_workspace_size", "fal_fwd", "fal_fwd_varlen_workspace_size", "fal_fwd_varlen",
    "fal_bwd_workspace_size", "fal_bwd", "fal_bwd_varlen_workspace_size", "fal_bwd_varlen",
    "fal_decode_workspace_size", "fal_decode",
    "fal_fwd_bf16", "fal_fwd_varlen_bf16", "fal_bwd_bf16", "fal_bwd_varlen_bf16", "fal_decode_bf16",
    "fal_decode_noalloc",
)


def library_path() -> str:
    return _LIB_PATH


def version() -> str:
    return _lib.fal_version().decode()


def device_supported(device: int = 0) -> bool:
    return bool(_lib.fal_device_supported(int(device)))


def _check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(_lib.fal_last_error().decode() or f"flash_attn_legacy error {rc}")


def _strides(t: torch.Tensor, dims=(0, 1, 2)):
    s = t.stride()
    return (ctypes.c_int64 * 3)(*[s[i] if i is not None else 0 for i in dims])


def _stride_block(*ts: torch.Tensor):
    """The (batch, head, sequence) strides of 4-D tensors in one ctypes array, and a
    pointer to each tensor's triple (one allocation instead of one per tensor)."""
    vals = []
    for t in ts:
        vals.extend(t.stride()[:3])
    arr = (ctypes.c_int64 * len(vals))(*vals)
    return arr, [ctypes.byref(arr, 24 * i) for i in range(len(ts))]


def _packed_block(*ts: torch.Tensor):
    """The (unused, head, token) strides of packed [total, H, d] tensors in one ctypes
    array, and a pointer to each tensor's triple."""
    vals = []
    for t in ts:
        s = t.stride()
        vals.extend((0, s[1], s[0]))
    arr = (ctypes.c_int64 * len(vals))(*vals)
    return arr, [ctypes.byref(arr, 24 * i) for i in range(len(ts))]


try:
    _raw_stream = torch._C._cuda_getCurrentRawStream   # the current stream's hipStream_t as an int
except AttributeError:   # pragma: no cover - older torch
    def _raw_stream(index):
        return torch.cuda.current_stream(index).cuda_stream


def _run(dev: torch.device, fn, *args):
    """Call fn(*args) with dev as the current device (switching only if needed)."""
    if dev.index == torch.cuda.current_device():
        return fn(*args)
    with torch.cuda.device(dev):
        return fn(*args)


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device):
    return _raw_stream(dev.index)


def _usable(t: torch.Tensor) -> torch.Tensor:
    """Keep strided views the kernels can address directly (unit last stride, other
    strides multiples of 8 elements, 16-byte aligned base); copy anything else."""
    if t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and all(s % 8 == 0 for s in t.stride()[:-1]):
        return t
    return t.contiguous()


def _workspace(nbytes: int, dev: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


DTYPES = (torch.float16, torch.bfloat16)


def _check_half_cuda(name: str, t: torch.Tensor, dtype: Optional[torch.dtype] = None) -> None:
    """t is a CUDA tensor of dtype (or, with dtype None, of float16 or bfloat16)."""
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be on CUDA")
    if dtype is None:
        if t.dtype not in DTYPES:
            raise RuntimeError(f"{name} must be float16 or bfloat16")
    elif t.dtype != dtype:
        raise RuntimeError(f"{name} must be {str(dtype)[6:]} like Q")


def _check_lse(L: torch.Tensor, shape, device) -> None:
    """L is the forward's fp32 log-sum-exp of `shape` on `device` (the kernels index it
    by the problem's sizes, so a smaller tensor would be read out of bounds)."""
    if L.dtype != torch.float32 or tuple(L.shape) != tuple(shape) or L.device != device:
        raise RuntimeError(f"L must be float32 {list(shape)} on {device}, got {L.dtype} "
                           f"{list(L.shape)} on {L.device}")


def _fn(name: str, dtype: torch.dtype):
    """The library entry point for an element type (fp16, or its _bf16 form)."""
    return getattr(_lib, name + "_bf16") if dtype == torch.bfloat16 else getattr(_lib, name)


# ---------------------------------------------------------------------------
# Reference-compatible entry points
# ---------------------------------------------------------------------------

def forward(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, softmax_scale: float,
            is_causal: bool = False) -> List[torch.Tensor]:
    """[O, L] for Q [B,Hq,N,d], K/V [B,Hkv,Nk,d]; L is [B,Hq,N] fp32 natural-log LSE.
    Checks of ``flash_attn_forward`` (csrc/flash_attn_legacy.cpp:48-60)."""
    _check_half_cuda("Q", Q)
    if Q.dim() != 4:
        raise RuntimeError("Q must be [B, H_q, N, d]")
    if K.dim() != 4 or V.dim() != 4:
        raise RuntimeError("K,V must be 4D")
    _check_half_cuda("K", K, Q.dtype)
    _check_half_cuda("V", V, Q.dtype)
    B, Hq, N, d = Q.shape
    Hkv, Nk = K.shape[1], K.shape[2]
    if K.shape[0] != B or K.shape[3] != d:
        raise RuntimeError("K shape mismatch")
    if tuple(V.shape) != (B, Hkv, Nk, d):
        raise RuntimeError("V shape mismatch")
    Q, K, V = _usable(Q), _usable(K), _usable(V)
    dev = Q.device
    O = torch.empty((B, Hq, N, d), dtype=Q.dtype, device=dev)
    L = torch.empty((B, Hq, N), dtype=torch.float32, device=dev)
    arr, (qs, ks, vs, os_) = _stride_block(Q, K, V, O)
    fwd = _fn("fal_fwd", Q.dtype)
    causal = int(bool(is_causal))
    # non-zero only for grids smaller than the GPU (split-KV partials)
    nws = _lib.fal_fwd_workspace_size(B, Hq, N, Nk, d, causal)
    ws = _workspace(nws, dev) if nws else None
    _check(_run(dev, lambda: fwd(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), L.data_ptr(),
                                 B, Hq, Hkv, N, Nk, d, qs, ks, vs, os_, float(softmax_scale), causal,
                                 ws.data_ptr() if ws is not None else None, nws,
                                 _raw_stream(dev.index))))
    return [O, L]


def forward_varlen(Q, K, V, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, max_seqlen_k: int,
                   softmax_scale: float, is_causal: bool = False) -> List[torch.Tensor]:
    """[O, L] for packed Q [total_q,Hq,d], K/V [total_k,Hkv,d]; L is [total_q,Hq].
    Checks of ``flash_attn_forward_varlen`` (csrc/flash_attn_legacy.cpp:201-217).
    The (sequence, tile) schedule is built on the device: no host synchronisation."""
    _check_half_cuda("Q", Q)
    if Q.dim() != 3:
        raise RuntimeError("Q must be [total_q, H_q, d]")
    if K.dim() != 3 or V.dim() != 3:
        raise RuntimeError("K,V must be 3D")
    _check_half_cuda("K", K, Q.dtype)
    _check_half_cuda("V", V, Q.dtype)
    if cu_seqlens_q.dtype != torch.int32:
        raise RuntimeError("cu_seqlens_q must be int32")
    if cu_seqlens_k.dtype != torch.int32:
        raise RuntimeError("cu_seqlens_k must be int32")
    total_q, Hq, d = Q.shape
    total_k, Hkv = K.shape[0], K.shape[1]
    num_seqs = cu_seqlens_q.shape[0] - 1
    if K.shape[2] != d or V.shape[2] != d:
        raise RuntimeError("K,V head_dim mismatch")
    if V.shape[1] != Hkv:
        raise RuntimeError("V num_heads mismatch")
    if cu_seqlens_k.shape[0] != num_seqs + 1:
        raise RuntimeError("cu_seqlens_k length mismatch")
    Q, K, V = _usable(Q), _usable(K), _usable(V)
    dev = Q.device
    cu_q = cu_seqlens_q if cu_seqlens_q.device == dev and cu_seqlens_q.is_contiguous() else \
        cu_seqlens_q.to(dev).contiguous()
    cu_k = cu_seqlens_k if cu_seqlens_k.device == dev and cu_seqlens_k.is_contiguous() else \
        cu_seqlens_k.to(dev).contiguous()
    O = torch.empty((total_q, Hq, d), dtype=Q.dtype, device=dev)
    L = torch.empty((total_q, Hq), dtype=torch.float32, device=dev)
    # zero for up to 64 sequences (the kernel derives its work items from cu_seqlens)
    nws = _lib.fal_fwd_varlen_workspace_size(num_seqs, total_q, int(max_seqlen_q), d)
    ws = _workspace(nws, dev) if nws else None
    arr, (qs, ks, vs, os_) = _packed_block(Q, K, V, O)
    fwd = _fn("fal_fwd_varlen", Q.dtype)
    _check(_run(dev, lambda: fwd(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), L.data_ptr(),
                                 cu_q.data_ptr(), cu_k.data_ptr(), num_seqs, total_q, total_k, Hq, Hkv, d,
                                 int(max_seqlen_q), int(max_seqlen_k), qs, ks, vs, os_, float(softmax_scale),
                                 int(bool(is_causal)), ws.data_ptr() if ws is not None else None, nws,
                                 _raw_stream(dev.index))))
    return [O, L]


def backward(dO, Q, K, V, O, L, softmax_scale: float, is_causal: bool = False) -> List[torch.Tensor]:
    """[dQ, dK, dV] from the saved forward (O, L).  Checks of ``flash_attn_backward``
    (csrc/flash_attn_legacy.cpp:115-120); dQ has Q's shape, dK/dV have K/V's."""
    if not (Q.is_cuda and Q.dtype in DTYPES):
        raise RuntimeError("Q must be CUDA float16 or bfloat16")
    if Q.dim() != 4 or K.dim() != 4:
        raise RuntimeError("Q, K must be 4D")
    if dO.shape != Q.shape:
        raise RuntimeError("dO shape must match Q")
    B, Hq, N, d = Q.shape
    Hkv, Nk = K.shape[1], K.shape[2]
    if Hq % Hkv != 0:
        raise RuntimeError("H_q must be divisible by H_kv for GQA")
    for name, t in (("dO", dO), ("K", K), ("V", V), ("O", O)):
        _check_half_cuda(name, t, Q.dtype)
    if K.shape[0] != B or K.shape[3] != d:
        raise RuntimeError("K shape mismatch")
    if V.shape != K.shape:
        raise RuntimeError("V shape must match K")
    if O.shape != Q.shape:
        raise RuntimeError("O shape must match Q")
    _check_lse(L, (B, Hq, N), Q.device)
    dO, Q, K, V, O = (_usable(t) for t in (dO, Q, K, V, O))
    L = L.contiguous()
    dQ = torch.empty((B, Hq, N, d), dtype=Q.dtype, device=Q.device)
    dK = torch.empty((B, Hkv, Nk, d), dtype=Q.dtype, device=Q.device)
    dV = torch.empty((B, Hkv, Nk, d), dtype=Q.dtype, device=Q.device)
    ws = _workspace(_lib.fal_bwd_workspace_size(B, Hq, N, d), Q.device)
    with torch.cuda.device(Q.device):
        _check(_fn("fal_bwd", Q.dtype)(
            _ptr(dO), _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(L), _ptr(dQ), _ptr(dK), _ptr(dV),
            B, Hq, Hkv, N, Nk, d,
            _strides(dO), _strides(Q), _strides(K), _strides(V), _strides(O),
            _strides(dQ), _strides(dK), _strides(dV),
            float(softmax_scale), int(bool(is_causal)), _ptr(ws), ws.numel(), _stream(Q.device)))
    return [dQ, dK, dV]


# ---------------------------------------------------------------------------
# Entry points without a reference counterpart
# ---------------------------------------------------------------------------

def backward_varlen(dO, Q, K, V, O, L, cu_seqlens_q, cu_seqlens_k, max_seqlen_q: int, max_seqlen_k: int,
                    softmax_scale: float, is_causal: bool = False) -> List[torch.Tensor]:
    """[dQ, dK, dV] for packed sequences in one launch.  Same results as the reference's
    per-sequence loop (flash_attn_legacy/flash_attn.py:133-157): dK/dV rows outside every
    segment are zero."""
    if not (Q.is_cuda and Q.dtype in DTYPES):
        raise RuntimeError("Q must be CUDA float16 or bfloat16")
    for name, t in (("dO", dO), ("K", K), ("V", V), ("O", O)):
        _check_half_cuda(name, t, Q.dtype)
    if Q.dim() != 3 or K.dim() != 3:
        raise RuntimeError("Q, K must be 3D")
    if dO.shape != Q.shape:
        raise RuntimeError("dO shape must match Q")
    total_q, Hq, d = Q.shape
    total_k, Hkv = K.shape[0], K.shape[1]
    if Hq % Hkv != 0:
        raise RuntimeError("H_q must be divisible by H_kv for GQA")
    if K.shape[2] != d:
        raise RuntimeError("K,V head_dim mismatch")
    if V.shape != K.shape:
        raise RuntimeError("V shape must match K")
    if O.shape != Q.shape:
        raise RuntimeError("O shape must match Q")
    _check_lse(L, (total_q, Hq), Q.device)
    if cu_seqlens_q.dim() != 1 or cu_seqlens_q.shape[0] < 1:
        raise RuntimeError("cu_seqlens_q must be a 1-D tensor of num_seqs + 1 offsets")
    num_seqs = cu_seqlens_q.shape[0] - 1
    if tuple(cu_seqlens_k.shape) != (num_seqs + 1,):
        raise RuntimeError("cu_seqlens_k length mismatch")
    for name, cu in (("cu_seqlens_q", cu_seqlens_q), ("cu_seqlens_k", cu_seqlens_k)):
        if cu.dtype != torch.int32:
            raise RuntimeError(f"{name} must be int32")
    dO, Q, K, V, O = (_usable(t) for t in (dO, Q, K, V, O))
    L = L.contiguous()
    cu_q = cu_seqlens_q.to(Q.device).contiguous()
    cu_k = cu_seqlens_k.to(Q.device).contiguous()
    # rows outside every segment come back zero (written by the library's schedule kernels)
    dQ = torch.empty((total_q, Hq, d), dtype=Q.dtype, device=Q.device)
    dK = torch.empty((total_k, Hkv, d), dtype=Q.dtype, device=Q.device)
    dV = torch.empty((total_k, Hkv, d), dtype=Q.dtype, device=Q.device)
    ws = _workspace(_lib.fal_bwd_varlen_workspace_size(num_seqs, total_q, total_k, Hq, d), Q.device)
    st = lambda t: _strides(t, (None, 1, 0))
    with torch.cuda.device(Q.device):
        _check(_fn("fal_bwd_varlen", Q.dtype)(
            _ptr(dO), _ptr(Q), _ptr(K), _ptr(V), _ptr(O), _ptr(L), _ptr(dQ), _ptr(dK), _ptr(dV), _ptr(cu_q), _ptr(cu_k),
            num_seqs, total_q, total_k, Hq, Hkv, d, int(max_seqlen_q), int(max_seqlen_k),
            st(dO), st(Q), st(K), st(V), st(O), st(dQ), st(dK), st(dV),
            float(softmax_scale), int(bool(is_causal)), _ptr(ws), ws.numel(), _stream(Q.device)))
    return [dQ, dK, dV]


def decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, cache_seqlens: torch.Tensor,
           softmax_scale: float, mask_bias: Optional[torch.Tensor] = None, cache_layout: str = "bshd",
           return_lse: bool = False):
    """Split-K decode.  q [B,Hq,d] (one token per sequence); caches [B,S,Hkv,d]
    (``cache_layout="bshd"``) or [B,Hkv,S,d] (``"bhsd"``); cache_seqlens int32 [B];
    mask_bias optional fp32 [B,S] additive mask.  Returns O [B,Hq,d] (and L [B,Hq])."""
    _check_half_cuda("q", q)
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        _check_half_cuda(name, t, q.dtype)
    if q.dim() != 3 or k_cache.dim() != 4 or v_cache.dim() != 4:
        raise RuntimeError("decode expects q [B,Hq,d] and 4-D caches")
    B, Hq, d = q.shape
    if cache_layout == "bshd":
        S, Hkv = k_cache.shape[1], k_cache.shape[2]
        cdims = (0, 2, 1)
    elif cache_layout == "bhsd":
        Hkv, S = k_cache.shape[1], k_cache.shape[2]
        cdims = (0, 1, 2)
    else:
        raise RuntimeError(f"unknown cache_layout {cache_layout!r}")
    if k_cache.shape != v_cache.shape or k_cache.shape[0] != B or k_cache.shape[3] != d:
        raise RuntimeError("k_cache / v_cache shape mismatch")
    if cache_seqlens.numel() != B:
        raise RuntimeError(f"cache_seqlens must hold {B} lengths, got {cache_seqlens.numel()}")
    if mask_bias is not None and (mask_bias.dim() != 2 or mask_bias.shape[0] != B or mask_bias.shape[1] < S):
        raise RuntimeError(f"mask_bias must be [B={B}, >= S={S}], got {tuple(mask_bias.shape)}")
    q, k_cache, v_cache = _usable(q), _usable(k_cache), _usable(v_cache)
    seqlens = cache_seqlens.reshape(-1).to(device=q.device, dtype=torch.int32).contiguous()
    bias = None
    if mask_bias is not None:
        bias = mask_bias.to(device=q.device, dtype=torch.float32)
        if bias.stride(-1) != 1:
            bias = bias.contiguous()
    o = torch.empty((B, Hq, d), dtype=q.dtype, device=q.device)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=q.device) if return_lse else None
    ws = _workspace(_lib.fal_decode_workspace_size(B, Hq, Hkv, S, d), q.device)
    with torch.cuda.device(q.device):
        _check(_fn("fal_decode", q.dtype)(
            _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(seqlens), _ptr(bias),
            bias.stride(0) if bias is not None else 0, _ptr(o), _ptr(lse), B, Hq, Hkv, d, S,
            _strides(q, (0, 1, None)), _strides(k_cache, cdims), _strides(v_cache, cdims),
            _strides(o, (0, 1, None)), float(softmax_scale), _ptr(ws), ws.numel(), _stream(q.device)))
    return (o, lse) if return_lse else o

"""Device detection, compatibility report and a flash-vs-standard benchmark for
AMD Instinct GPUs.

The public names and arguments are those of the reference's ``utils.py``
(``get_device_info``, ``check_gpu_compatibility``, ``benchmark_flash_vs_standard``,
flash_attn_legacy/utils.py:16-125).  What decides support here is the library
itself: ``fal_device_supported`` reports whether ``libfal_hip.so`` holds code for
the device (gfx950, MI350X / MI355X).  The benchmark reports absolute rates and
the fraction of the device's dense fp16 MFMA peak next to the timings.
"""

from __future__ import annotations

import math
from typing import Callable, Dict, Optional

import torch

# gfx target -> (family, products)
_TARGETS = {
    "gfx950": ("CDNA4", "MI350X / MI355X"),
    "gfx942": ("CDNA3", "MI300X / MI325X"),
    "gfx90a": ("CDNA2", "MI200"),
    "gfx908": ("CDNA1", "MI100"),
}

# Published per-device peaks of the supported target: dense fp16 MFMA (TFLOP/s) and HBM (GB/s)
_PEAKS = {"gfx950": (2500.0, 8000.0)}


def _target(props) -> str:
    """'gfx950' from a gcnArchName such as 'gfx950:sramecc+:xnack-'."""
    return (getattr(props, "gcnArchName", "") or "").split(":", 1)[0]


def _library_supports(index: int) -> bool:
    try:
        from . import hip_ext
    except ImportError:
        return False
    return hip_ext.device_supported(index)


def get_device_info(device: Optional[int] = None) -> Dict:
    """Properties of a GPU and whether this library runs on it.

    Keys shared with the reference: name, sm_version (HIP's major*10 + minor, 95 on
    gfx950), arch, total_memory_gb, shared_mem_per_block, multiprocessor_count,
    has_tensor_cores (MFMA matrix cores), kernel_path, supported.  Added: gfx_arch,
    peak_fp16_tflops and peak_hbm_gbs (None for an unsupported target).
    Raises RuntimeError without a GPU, like the reference."""
    if not torch.cuda.is_available():
        raise RuntimeError("CUDA not available")
    index = torch.cuda.current_device() if device is None else int(device)
    props = torch.cuda.get_device_properties(index)
    gfx = _target(props)
    family, products = _TARGETS.get(gfx, ("unknown", gfx or "unknown target"))
    supported = _library_supports(index)
    peak_flops, peak_hbm = _PEAKS.get(gfx, (None, None))
    return {
        "name": props.name,
        "sm_version": props.major * 10 + props.minor,
        "gfx_arch": gfx,
        "arch": f"{family} ({products})",
        "total_memory_gb": round(props.total_memory / 2 ** 30, 2),
        "shared_mem_per_block": int(getattr(props, "shared_memory_per_block",
                                            getattr(props, "max_shared_memory_per_block", 0))),
        "multiprocessor_count": props.multi_processor_count,
        "has_tensor_cores": family in ("CDNA2", "CDNA3", "CDNA4"),
        "kernel_path": ("gfx950 HIP kernels: fp16/bf16 MFMA, LDS-staged K/V, split-K decode"
                        if supported else f"none: libfal_hip.so has no code for {gfx or 'this device'}"),
        "peak_fp16_tflops": peak_flops,
        "peak_hbm_gbs": peak_hbm,
        "supported": supported,
    }


def check_gpu_compatibility(device: Optional[int] = None, verbose: bool = True) -> bool:
    """True if flash_attn_legacy's kernels run on the GPU; with verbose, print a report."""
    if not torch.cuda.is_available():
        if verbose:
            print("No GPU visible to PyTorch (torch.cuda.is_available() is False)")
        return False
    info = get_device_info(device)
    if verbose:
        rows = [
            ("device", info["name"]),
            ("target", f"{info['gfx_arch']} - {info['arch']}"),
            ("compute units", info["multiprocessor_count"]),
            ("memory", f"{info['total_memory_gb']} GiB"),
            ("LDS per workgroup", f"{info['shared_mem_per_block']} bytes"),
            ("kernels", info["kernel_path"]),
        ]
        width = max(len(k) for k, _ in rows)
        for k, val in rows:
            print(f"{k:<{width}} : {val}")
        print("supported" if info["supported"] else "NOT supported (needs gfx950)")
    return bool(info["supported"])


def _event_ms(fn: Callable[[], object], warmup: int, iters: int) -> float:
    """Mean milliseconds of fn() over `iters` back-to-back calls, from HIP events on the
    current stream (the stream both implementations launch on)."""
    for _ in range(max(warmup, 0)):
        fn()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / iters


def _peak_mb(fn: Callable[[], object]) -> float:
    """Device memory (MB) one call needs beyond what is already allocated: its
    outputs plus its temporaries at their high-water mark."""
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    torch.cuda.reset_peak_memory_stats()
    out = fn()
    torch.cuda.synchronize()
    peak = torch.cuda.max_memory_allocated() - base
    del out
    return peak / 1e6


def benchmark_flash_vs_standard(
    batch_size: int = 2, num_heads: int = 8, seq_len: int = 2048,
    head_dim: int = 64, is_causal: bool = False,
    num_warmup: int = 10, num_iters: int = 100
) -> Dict:
    """Time ``flash_attention`` against standard attention (fp32 scores, softmax, fp16
    P @ V -- the reference's comparison formula) on seeded fp16 N(0,1) inputs.

    Returns the reference's keys (config, flash_ms, std_ms, speedup, flash_mem_mb,
    std_mem_mb, mem_savings_pct; memory is what one call needs beyond its inputs)
    plus flash_tflops and flash_frac_peak (FA2 flop convention, 4*B*H*N^2*d, halved
    when causal, against the device's dense fp16 MFMA peak), std_tflops and
    max_abs_diff between the two outputs."""
    from .flash_attn import flash_attention

    dev = torch.device("cuda", torch.cuda.current_device())
    gen = torch.Generator().manual_seed(0)
    shape = (batch_size, num_heads, seq_len, head_dim)
    q, k, v = (torch.randn(shape, generator=gen).half().to(dev) for _ in range(3))
    scale = 1.0 / math.sqrt(head_dim)
    future = (torch.triu(torch.ones(seq_len, seq_len, dtype=torch.bool, device=dev), diagonal=1)
              if is_causal else None)

    def flash():
        return flash_attention(q, k, v, softmax_scale=scale, is_causal=is_causal)

    def standard():
        s = (q.float() @ k.float().transpose(-1, -2)) * scale
        if future is not None:
            s = s.masked_fill(future, float("-inf"))
        return torch.softmax(s, dim=-1).half() @ v

    diff = float((flash().float() - standard().float()).abs().max())
    flash_ms = _event_ms(flash, num_warmup, num_iters)
    std_ms = _event_ms(standard, num_warmup, num_iters)
    flash_mb, std_mb = _peak_mb(flash), _peak_mb(standard)

    flops = 4.0 * batch_size * num_heads * seq_len * seq_len * head_dim * (0.5 if is_causal else 1.0)
    peak = get_device_info(dev.index)["peak_fp16_tflops"]
    flash_tflops = flops / (flash_ms * 1e-3) / 1e12
    return {
        "config": f"B={batch_size} H={num_heads} N={seq_len} d={head_dim}" + (" causal" if is_causal else ""),
        "flash_ms": round(flash_ms, 3),
        "std_ms": round(std_ms, 3),
        "speedup": round(std_ms / flash_ms, 2) if flash_ms > 0 else 0.0,
        "flash_tflops": round(flash_tflops, 1),
        "flash_frac_peak": round(flash_tflops / peak, 4) if peak else None,
        "std_tflops": round(flops / (std_ms * 1e-3) / 1e12, 1),
        "flash_mem_mb": round(flash_mb, 1),
        "std_mem_mb": round(std_mb, 1),
        "mem_savings_pct": round(100.0 * (1.0 - flash_mb / std_mb), 1) if std_mb > 0 else 0.0,
        "max_abs_diff": round(diff, 5),
    }

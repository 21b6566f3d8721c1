"""Benchmark of the attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--prerun-s S] [--no-cpu] [--only c2]

A step is one forward call of configuration C2 (GQA causal prefill: B=4, 32 query
heads / 8 KV heads, N=4096, d=128, fp16 N(0,1) inputs from seed 0) -- the
configuration the headline metric is quoted on.  The line printed at the end is
one JSON object:

* ``value``: C2 forward TFLOP/s (FA2 flop convention: 4*B*Hq*N^2*d, halved for
  causal), inputs resident in HBM, K steps between two device synchronisations;
* ``roofline``: the forward kernel's algorithmic flops per launch over its
  average launch time (HIP events on the launch stream, same timed region),
  against the 2.5 PFLOP/s dense fp16 MFMA peak; ``traffic`` comes from the
  committed rocprofv3 counter summary when present;
* ``prerun_s``: seconds of untimed calls of the workload right before its warmup
  (a quarter of it for each extra workload), so the timed steps run at the clock the
  GPU holds under sustained load rather than in the ramp after the host-side input
  creation left it idle;
* ``cpu_baseline``: fp32 PyTorch attention (the reference's own test formula) on
  this host's CPU cores over the whole C2 workload (its 32 (batch, KV-group) slices,
  the GPU call's seeded inputs), median of 3 passes;
* ``extra``: the other configurations measured the same way -- C1 forward, C3
  backward (2.5x forward flops), C4 varlen forward, C5 split-K decode (KV bytes
  read, GB/s against 8 TB/s HBM), and the reference's packed-vs-padded varlen
  scenarios.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "flash-attention-legacy_amd"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
METRIC = "attn fwd/bwd TFLOP/s (% fp16 MFMA peak); decode KV GB/s (% HBM peak)"


def randn(shape, seed, device="cuda"):
    """fp16 N(0,1) drawn on the CPU from a seeded generator; `device` None keeps it there."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g, dtype=torch.float32).half()
    return x.to(device) if device is not None else x


def fwd_flops(b, hq, nq, nk, d, causal):
    f = 4.0 * b * hq * nq * nk * d
    return f / 2 if causal else f


PRERUN_S = 0.0   # seconds of untimed calls before each workload's warmup (set from --prerun-s)


def settle(fn, seconds):
    """Call `fn` back to back for `seconds` of wall time, untimed.  After the host has
    kept the GPU idle (creating inputs), its first launches run up to ~30% slower while
    clocks and power ramp back; this brings every timed region to the steady state."""
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(8):
            fn()
        torch.cuda.synchronize()


def time_steps(fn, steps, warmup, prerun=None):
    """Run `fn` for the pre-run time, `warmup` more times, then time `steps` calls.
    Returns (wall ms/step, event ms/step) -- the events are recorded on the current
    stream, which is the stream the kernels are launched on."""
    settle(fn, PRERUN_S if prerun is None else prerun)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        fn()
    e1.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    return wall, e0.elapsed_time(e1) / steps


def bench_c2(steps, warmup):
    from flash_attn_legacy import hip_ext
    B, Hq, Hkv, N, d = 4, 32, 8, 4096, 128
    q, k, v = randn((B, Hq, N, d), 0), randn((B, Hkv, N, d), 1), randn((B, Hkv, N, d), 2)
    scale = 1.0 / math.sqrt(d)
    wall, ev = time_steps(lambda: hip_ext.forward(q, k, v, scale, True), steps, warmup)
    return wall, ev, fwd_flops(B, Hq, N, N, d, True)


def bench_extra(steps, warmup, which=("c1", "c3", "c4", "c5")):
    out = {}
    if "c1" in which:
        bench_c1(out, steps, warmup)
    if "c3" in which:
        bench_c3(out, steps, warmup)
    if "c4" in which:
        bench_c4(out, steps, warmup)
    if "c5" in which:
        bench_c5(out, steps, warmup)
    return out


def bench_c1(out, steps, warmup):
    from flash_attn_legacy import hip_ext
    q, k, v = (randn((2, 8, 1024, 64), s) for s in (0, 1, 2))
    _, ev = time_steps(lambda: hip_ext.forward(q, k, v, 0.125, True), steps, warmup)
    f = fwd_flops(2, 8, 1024, 1024, 64, True)
    out["c1_fwd"] = {"tflops": round(f / ev / 1e9, 2), "ms": round(ev, 4),
                     "frac_peak": round(f / ev / 1e9 / PEAK_FP16_TFLOPS, 4)}


def bench_c3(out, steps, warmup):
    from flash_attn_legacy import hip_ext
    B, H, N, d = 2, 16, 2048, 128
    q, k, v, do = (randn((B, H, N, d), s) for s in (0, 1, 2, 3))
    scale = 1.0 / math.sqrt(d)
    o, lse = hip_ext.forward(q, k, v, scale, True)
    _, ev = time_steps(lambda: hip_ext.backward(do, q, k, v, o, lse, scale, True), steps, warmup)
    f = 2.5 * fwd_flops(B, H, N, N, d, True)
    out["c3_bwd"] = {"tflops": round(f / ev / 1e9, 2), "ms": round(ev, 4),
                     "frac_peak": round(f / ev / 1e9 / PEAK_FP16_TFLOPS, 4)}


def bench_c4(out, steps, warmup):
    from flash_attn_legacy import hip_ext
    scale = 1.0 / math.sqrt(128)
    g = torch.Generator().manual_seed(0)
    lens = [int(x) for x in torch.randint(64, 4097, (16,), generator=g)]
    tot = sum(lens)
    q, k, v = randn((tot, 32, 128), 0), randn((tot, 8, 128), 1), randn((tot, 8, 128), 2)
    cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32, device="cuda")
    mx = max(lens)
    _, ev = time_steps(lambda: hip_ext.forward_varlen(q, k, v, cu, cu, mx, mx, scale, True), steps, warmup)
    f = sum(fwd_flops(1, 32, n, n, 128, True) for n in lens)
    out["c4_varlen_fwd"] = {"tflops": round(f / ev / 1e9, 2), "ms": round(ev, 4),
                            "frac_peak": round(f / ev / 1e9 / PEAK_FP16_TFLOPS, 4), "total_tokens": tot}


def bench_c5(out, steps, warmup):
    from flash_attn_legacy import hip_ext
    scale = 1.0 / math.sqrt(128)
    g = torch.Generator().manual_seed(0)
    lens = [int(x) for x in torch.randint(1024, 32769, (32,), generator=g)]
    S = max(lens)
    q = randn((32, 32, 128), 1)
    kc, vc = randn((32, S, 8, 128), 2), randn((32, S, 8, 128), 3)
    seq = torch.tensor(lens, dtype=torch.int32, device="cuda")
    _, ev = time_steps(lambda: hip_ext.decode(q, kc, vc, seq, scale), steps, warmup)
    nbytes = sum(lens) * 8 * 128 * 2 * 2
    out["c5_decode"] = {"gbs": round(nbytes / ev / 1e6, 1), "ms": round(ev, 4),
                        "frac_peak": round(nbytes / ev / 1e6 / PEAK_HBM_GBS, 4), "kv_bytes": nbytes}


# Packed-vs-padded scenarios of the reference's varlen benchmark
# (tests/test_generation_benchmark.py:465-472, README.md:253-274): H=8, d=64, causal.
VARLEN_SCENARIOS = [
    ("uniform_short", [64] * 16),
    ("uniform_medium", [256] * 8),
    ("mixed_short", [32, 64, 48, 16, 96, 80, 24, 128]),
    ("mixed_heavy", [512, 64, 256, 32, 128, 64, 512, 32]),
    ("one_long_rest_short", [1024] + [32] * 15),
    ("all_long", [1024] * 4),
]


def graph_ms(fn, calls=20, replays=5):
    """GPU time per call without the host's per-call overhead: `calls` calls captured in
    one HIP graph, replayed `replays` times between events (after one untimed replay)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (calls * replays)


def bench_varlen_vs_padded(steps, warmup):
    """Padded batch (every sequence padded to the longest, ``flash_attention``) against
    the packed batch (``flash_attn_varlen_func``) through the public API, as the
    reference's benchmark does; plus the same comparison on C4's lengths (16 sequences
    U[64, 4096], 32/8 heads, d=128), where the padded batch is [16, H, 4096, 128].
    *_ms are per call through the API (host overhead included: the small scenarios are
    host-bound); *_gpu_ms are the same calls replayed from a captured HIP graph."""
    from flash_attn_legacy import flash_attention, flash_attn_varlen_func
    out = {}

    def one(name, lens, hq, hkv, d, seed):
        B, mx, tot = len(lens), max(lens), sum(lens)
        scale = 1.0 / math.sqrt(d)
        qp, kp, vp = randn((B, hq, mx, d), seed), randn((B, hkv, mx, d), seed + 1), randn((B, hkv, mx, d), seed + 2)
        qv, kv, vv = randn((tot, hq, d), seed), randn((tot, hkv, d), seed + 1), randn((tot, hkv, d), seed + 2)
        cu = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()), dtype=torch.int32, device="cuda")
        pad = lambda: flash_attention(qp, kp, vp, softmax_scale=scale, is_causal=True)
        pack = lambda: flash_attn_varlen_func(qv, kv, vv, cu, cu, mx, mx, softmax_scale=scale, causal=True)
        with torch.no_grad():
            _, pad_ms = time_steps(pad, steps, warmup)
            _, pack_ms = time_steps(pack, steps, warmup)
            pad_gpu, pack_gpu = graph_ms(pad), graph_ms(pack)
        useful = sum(fwd_flops(1, hq, n, n, d, True) for n in lens)
        out[name] = {"seqs": B, "max_len": mx, "tokens": tot,
                     "padding_waste": round(1 - tot / (B * mx), 3),
                     "padded_ms": round(pad_ms, 4), "packed_ms": round(pack_ms, 4),
                     "speedup": round(pad_ms / pack_ms, 2),
                     "padded_gpu_ms": round(pad_gpu, 4), "packed_gpu_ms": round(pack_gpu, 4),
                     "gpu_speedup": round(pad_gpu / pack_gpu, 2),
                     "packed_useful_tflops": round(useful / pack_ms / 1e9, 1)}

    for i, (name, lens) in enumerate(VARLEN_SCENARIOS):
        one(name, lens, 8, 8, 64, 100 + 3 * i)
    g = torch.Generator().manual_seed(0)
    c4 = [int(x) for x in torch.randint(64, 4097, (16,), generator=g)]
    one("c4_lengths_32q8kv_d128", c4, 32, 8, 128, 200)
    return out


def cpu_baseline(runs=3, budget_s=60.0):
    """fp32 PyTorch attention (reference tests/test_flash_attn.py:19-32) on the host CPU
    over the whole C2 workload, on the same seeded inputs as the GPU call: every one of
    the 32 (batch, KV-group) slices (4 query heads x N=4096 x d=128, causal; one slice at
    a time bounds the fp32 score matrix), `runs` passes, median pass time (one pass when
    a pass takes longer than `budget_s` / runs).  Rate in TFLOP/s (same flop convention)."""
    from oracle.torch_ref import ref_attention
    # the GPU box grants one GPU's job 16 CPUs, whatever os.cpu_count() reports
    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    B, Hq, Hkv, N, d = 4, 32, 8, 4096, 128
    G = Hq // Hkv
    q, k, v = (randn(s, seed, device=None) for s, seed in (((B, Hq, N, d), 0), ((B, Hkv, N, d), 1),
                                                            ((B, Hkv, N, d), 2)))
    scale = 1.0 / math.sqrt(d)
    ref_attention(q[:1, :G, :256], k[:1, :1, :256], v[:1, :1, :256], scale, True)   # warm the thread pool
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        for b in range(B):
            for g in range(Hkv):
                ref_attention(q[b:b + 1, g * G:(g + 1) * G], k[b:b + 1, g:g + 1], v[b:b + 1, g:g + 1],
                              scale, True)
        times.append(time.perf_counter() - t0)
        if sum(times) * runs > budget_s:
            break
    dt = statistics.median(times)
    flops = fwd_flops(B, Hq, N, N, d, True)
    cpu_model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(flops / dt / 1e12, 5), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"all 32 (batch, KV-group) slices of C2 (4 query heads x N=4096 x d=128, causal each), "
                      f"the GPU call's seeded inputs, fp32 torch on CPU; median of {len(times)} passes "
                      f"({', '.join(f'{t:.2f}' for t in times)} s); threads={threads}, "
                      f"os.cpu_count()={os.cpu_count()}; cpu={cpu_model}"}


def load_traffic():
    """HBM bytes per C2 forward launch from the committed rocprofv3 counter summary."""
    path = os.path.join(ROOT, "profiles", "fwd_c2_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--prerun-s", type=float, default=2.0,
                    help="seconds of untimed calls of the workload right before its warmup (clock "
                         "settling); the extra workloads get a quarter of it each")
    ap.add_argument("--only", choices=["c2", "all", "copy", "c1", "c3", "c4", "c5"], default="all",
                    help="c2: the headline line without the extra configurations; copy: a 1 GiB "
                         "device copy only, the known-size kernel that calibrates HBM byte counters; "
                         "c1/c3/c4/c5: that one extra workload alone (for profiler runs), printed as "
                         "{\"extra\": ...}")
    a = ap.parse_args()
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(every box has one MI355X); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    if a.only == "copy":
        src = torch.empty(1 << 29, dtype=torch.float16, device="cuda").fill_(1.0)
        dst = torch.empty_like(src)
        wall, ev = time_steps(lambda: dst.copy_(src), a.steps, a.warmup)
        print(json.dumps({"copy_bytes_read": src.numel() * 2, "copy_bytes_written": dst.numel() * 2,
                          "gbs": round(2 * src.numel() * 2 / ev / 1e6, 1)}), flush=True)
        return

    global PRERUN_S
    PRERUN_S = max(a.prerun_s, 0.0)
    if a.only in ("c1", "c3", "c4", "c5"):
        print(json.dumps({"extra": bench_extra(a.steps, a.warmup, (a.only,))}), flush=True)
        return
    wall, ev, flops = bench_c2(a.steps, a.warmup)
    value = flops / (wall * 1e-3) / 1e12
    achieved = flops / (ev * 1e-3) / 1e12
    # the other workloads: a quarter of the pre-run each (they are short)
    PRERUN_S = PRERUN_S / 4
    extra = bench_extra(max(5, a.steps // 2), max(2, a.warmup // 2)) if a.only == "all" else {}
    if a.only == "all":
        extra["varlen_vs_padded"] = bench_varlen_vs_padded(max(5, a.steps // 2), max(2, a.warmup // 2))
    traffic = load_traffic()
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "prerun_s": max(a.prerun_s, 0.0),
        "ms_per_step": round(wall, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic",
        "config": {"workload": "C2 fwd GQA causal prefill", "batch": 4, "heads_q": 32, "heads_kv": 8,
                   "seq_len": 4096, "head_dim": 128, "causal": True, "inputs": "fp16 N(0,1) seed 0"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP16_TFLOPS, 4),
                     "traffic": traffic,
                     "traffic_source": "profiles/fwd_c2_traffic.json: committed rocprofv3 --pmc FETCH_SIZE and "
                                       "WRITE_SIZE passes of this workload, not measured in this run",
                     "kernel": "fwd_kernel<_Float16,128,4,64,true,2,false> (pipelined tile loop, persistent four-heads grid)",
                     "flops_per_launch": flops},
        "cpu_baseline": None if a.no_cpu else cpu_baseline(),
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()

#!/usr/bin/env python3
"""Headline benchmark: FlashAttention-2 forward + backward, FP32, on one MI355X.

Workload (benchmark config 2): B=4, H=32, N=4096, D=64, causal; Q, K, V, dO ~ N(0, 1) from fixed
seeds; softmax scale 1/sqrt(64).  One step = the forward kernel then the three backward
stages, launched through the C ABI on torch's current stream with all inputs and outputs
already resident in HBM.  The backward runs the schedule the flash_attention_bwd operator
uses: delta, dK/dV storing dS, dQ from the stored dS (--bwd-schedule stored, default); or the
reference's schedule, delta, dQ recomputing S and dP, dK/dV (--bwd-schedule recompute).

Reported:
  value          whole-step TFLOPS by the reference's formula (benchmark/cuda_bench.py:63-68):
                 fwd 4*B*H*N^2*D, halved for causal; bwd 2.5x fwd; divided by the wall time of
                 exactly --steps steps bracketed by device synchronisation.
  per_kernel_ms  HIP-event durations of each kernel on its launch stream, averaged over the
                 timed steps; per_kernel_ms_flushed: the median of each kernel launched alone
                 after 1 GiB of device memory was written (cold L2 and MALL), after the timed
                 steps.
  roofline       the dominant kernel's algorithmic FLOPs per launch / its mean duration in the
                 timed steps, vs the 157.3 TFLOP/s dense FP32 MFMA peak (achieved_flushed: the
                 same from the cache-cold launches); traffic (HBM bytes per launch) from the
                 committed rocprofv3 counter summary profiles/fa2_config2_counters.md.
  cpu_baseline   the reference's CPU comparison path, torch FP32 SDPA forward + autograd
                 backward (its test oracle), timed on this host's cores on whole heads of the
                 same workload, with the backend torch chose, the CPU model and the estimated
                 time of the full step.
  recompute      the same step with the reference's workspace-free backward schedule (delta,
                 dQ recomputing S and dP, dK/dV without the dS store: O(N) memory), timed in
                 the same run: per-kernel ms, fwd/bwd TFLOPS and its own roofline.  `value`
                 stays the operator's default (stored-dS) schedule; ds_workspace_bytes states
                 what that default allocates.
  cpu_baseline_port (--cpu-port only)
                 the CPU oracle (numpy port of the reference algorithm, float32) timed on a
                 bounded sample of whole heads of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import re
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

MFMA_FP32_PEAK_TFLOPS = 157.3
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense; FP16 is the same
HBM_PEAK_GBPS = 8000.0
METRIC = "FA2 fwd+bwd FP32 TFLOPS @B4 H32 N4096 D64 causal; % of FP32 MFMA peak"
# The reference's own numbers for this exact configuration (RTX 5070, README.md:60-67,197):
# forward 212.73 ms + backward 1259.32 ms.  Different hardware: reported for context only.
REFERENCE_RTX5070_MS = {"fwd": 212.73, "bwd": 1259.32}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--workload", choices=["fa2", "fa2-sweep", "ops", "gpt", "gemm", "fa2-bf16",
                                          "fa2-f16"],
                   default="fa2",
                   help="fa2: the headline step (default, one JSON line); fa2-sweep: benchmark "
                        "config 3; ops: benchmark config 4 (one JSON line per op); gpt: benchmark "
                        "config 5 training step; gemm: the config-4/5 GEMMs A/B against torch's "
                        "FP32 GEMM; fa2-bf16 / fa2-f16: the BF16 / FP16 forward and "
                        "backward at the config-2 shape, causal and full (an extension beyond "
                        "the FP32 metric)")
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--batch", type=int, default=4)
    p.add_argument("--heads", type=int, default=32)
    p.add_argument("--seq", type=int, default=4096)
    p.add_argument("--head-dim", type=int, default=64)
    p.add_argument("--non-causal", action="store_true")
    p.add_argument("--seqs", default="",
                   help="fa2-sweep workload: comma-separated sequence lengths (default "
                        "1024,2048,4096,8192,16384)")
    p.add_argument("--masks", choices=["both", "causal", "full"], default="both",
                   help="fa2-bf16 workload: which masks to time")
    p.add_argument("--gpt-adamw", choices=["fused", "foreach"], default="fused",
                   help="gpt workload: torch AdamW implementation (fused: one multi-tensor kernel "
                        "per step; foreach: torch's default list kernels)")
    p.add_argument("--gpt-mlp", choices=["fused", "reference"], default="fused",
                   help="gpt workload: fused: CudaMLP (GELU in the GEMM epilogues, the model's "
                        "default); reference: CudaLinearLayer -> CudaGeluLayer -> CudaLinearLayer")
    p.add_argument("--bwd-schedule", choices=["stored", "recompute", "fold"], default="stored",
                   help="stored: dK/dV writes dS and dQ reads it (what the operator runs); "
                        "recompute: the reference's delta / dQ / dK/dV schedule; fold: the stored "
                        "schedule with delta computed inside the dK/dV stage (no delta launch)")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--warm-seconds", type=float, default=1.0,
                   help="back-to-back untimed steps before the timed ones, at least this long")
    p.add_argument("--cpu-port", action="store_true",
                   help="also time the numpy oracle on the CPU (cpu_baseline_port, ~10 s)")
    p.add_argument("--no-recompute", action="store_true",
                   help="leave out the recompute-schedule object of the headline line")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="target CPU time of the bounded CPU-baseline sample")
    p.add_argument("--no-autograd", action="store_true",
                   help="skip the extra autograd-path timing (CudaFlashAttention fwd + backward)")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="only run a plain device copy of this many MiB (3 times): the known-size "
                        "reference that scales the FETCH_SIZE / WRITE_SIZE counters")
    return p.parse_args()


def copy_calibration(mib):
    import torch

    n = mib * (1 << 20) // 4
    x = torch.ones(n, device="cuda")
    y = torch.empty_like(x)
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n * 4, "bytes_written": n * 4,
                      "launches": 3}), flush=True)
    return 0


# Bytes read between cache-cold repetitions, and the least footprint of the buffer copies that
# rotating op timings cycle through: both well above the 256 MB MALL (Infinity Cache) and the
# 8 x 4 MB of L2.
FLUSH_BYTES = 1 << 30
ROTATE_BYTES = 1 << 30


class CacheFlush:
    """Reads FLUSH_BYTES of device memory (one reduction kernel on the current stream), so the
    L2s and the MALL hold only clean lines of this buffer when the next timed launch starts.  A
    read, not a write: a written buffer would leave up to 256 MB of dirty lines in the MALL for
    the timed kernel to write back (measured: +256 MB of traffic, e.g. the row softmax at 99 us
    instead of 71 us)."""

    def __init__(self, dev):
        import torch

        self.buf = torch.ones(FLUSH_BYTES // 4, device=dev)
        self.out = torch.empty((), device=dev)

    def __call__(self):
        import torch

        torch.sum(self.buf, dim=0, out=self.out)


def host_info():
    """CPU model, logical CPUs and the GPU's architecture, for the CPU-baseline records."""
    import torch

    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    info = {"cpu_model": model, "cpu_count": os.cpu_count()}
    if torch.cuda.is_available():
        props = torch.cuda.get_device_properties(0)
        info["gpu"] = torch.cuda.get_device_name(0)
        info["gpu_arch"] = getattr(props, "gcnArchName", "unknown")
        info["gpu_cus"] = props.multi_processor_count
    return info


def attn_flops(B, H, N, D, causal):
    fwd = 4.0 * B * H * N * N * D * (0.5 if causal else 1.0)
    return fwd, 2.5 * fwd


def kernel_algorithmic(name, B, H, N, D, causal):
    """(amount, unit, bound) of algorithmic work per launch of one kernel.

    Attention kernels: 2*D FLOPs per (query, key) pair for each N x N x D product the kernel
    must form — forward 2 products (S, PV), dQ 3 (S, dP, dQ), dK/dV 4 (S, dP, dV, dK), dQ from
    stored dS 1 — over B*H*N^2 pairs, halved when causal.  delta: bytes of O and dO read plus
    delta written."""
    pairs = B * H * N * N * (0.5 if causal else 1.0)
    products = {"fwd": 2, "dq": 3, "dkdv": 4, "dq_ds": 1}
    if name in products:
        return 2.0 * D * pairs * products[name], "TFLOP/s", "mfma"
    return float(2 * B * H * N * D * 4 + B * H * N * 4), "GB/s", "hbm"


def load_traffic(kernel: str, summary: str = "fa2_config2_counters.md"):
    """HBM bytes per launch of `kernel` from a committed PMC summary under profiles/, or None."""
    path = ROOT / "profiles" / summary
    if not path.exists():
        return None
    m = re.search(rf"traffic_bytes_per_launch\[{re.escape(kernel)}(<[^\]]*>)?\]\s*=\s*([0-9.eE+]+)",
                  path.read_text())
    return float(m.group(2)) if m else None


def cpu_port_baseline(B, H, N, D, causal, target_s):
    """Time the CPU oracle (float32 numpy, BLAS-threaded) on whole heads until target_s."""
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import attention as ora

    cores = min(16, os.cpu_count() or 1)  # the GPU box's CPU share is 16 cores
    with threadpool_limits(limits=cores, user_api="blas"):
        threads = max([i["num_threads"] for i in threadpool_info()
                       if i.get("user_api") == "blas"] or [1])
        rng = np.random.default_rng(0)
        chunk = 4  # heads per chunk
        shape = (1, chunk, N, D)
        q, k, v, do = (rng.standard_normal(shape, dtype=np.float32) for _ in range(4))
        heads = 0
        t0 = time.perf_counter()
        while heads < B * H:
            O, L = ora.fa2_forward(q, k, v, causal, br=512, bc=512)
            ora.fa2_backward(q, k, v, O, do, L, causal, br=512, bc=512)
            heads += chunk
            if time.perf_counter() - t0 >= target_s:
                break
        elapsed = time.perf_counter() - t0
    fwd, bwd = attn_flops(1, heads, N, D, causal)
    return {
        "value": (fwd + bwd) / elapsed / 1e12,
        "unit": "TFLOPS",
        "cores": threads,
        "kind": "port",
        "sample": (f"{heads} of {B * H} heads (N={N}, D={D}, {'causal' if causal else 'full'}) "
                   f"fwd+bwd, float32 numpy oracle (oracle/attention.py), 512x512 tiles, "
                   f"{elapsed:.1f} s on {threads} BLAS threads"),
        "seconds": elapsed,
    }


def cpu_reference_path(B, H, N, D, causal, step_s=2.0):
    """The reference's own CPU path, as its test suite and benchmark define correctness and the
    comparison point (test/test_flash_attention.py:10-21, benchmark/cuda_bench.py:44-68): torch
    FP32 scaled_dot_product_attention forward + autograd backward on this host's cores, on whole
    heads of the workload: as many as an estimated step_s per step allows (at ~1.4 TFLOP/s), all
    of them when that covers the workload.  One warm-up step, then the median of three."""
    import statistics

    import torch
    import torch.nn.functional as F

    threads = min(16, os.cpu_count() or 1)  # the GPU box's CPU share is 16 cores
    prev = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        per_head = sum(attn_flops(1, 1, N, D, causal))
        heads = max(1, min(B * H, int(step_s * 1.4e12 / per_head)))
        gen = torch.Generator().manual_seed(0)
        q, k, v = (torch.randn(1, heads, N, D, generator=gen).requires_grad_() for _ in range(3))
        do = torch.randn(1, heads, N, D, generator=torch.Generator().manual_seed(1))
        backend = torch.nn.attention.SDPBackend(torch._fused_sdp_choice(q, k, v, is_causal=causal))

        def step():
            o = F.scaled_dot_product_attention(q, k, v, is_causal=causal)
            o.backward(do)
            q.grad = k.grad = v.grad = None

        step()
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
        med = statistics.median(times)
    finally:
        torch.set_num_threads(prev)
    fwd, bwd = attn_flops(1, heads, N, D, causal)
    return {
        "value": round((fwd + bwd) / med / 1e12, 4),
        "unit": "TFLOPS",
        "cores": threads,
        "kind": "reference",
        "path": ("the reference's CPU comparison path: torch FP32 F.scaled_dot_product_attention "
                 "+ autograd backward (its test oracle, test/test_flash_attention.py:32,44-50); "
                 "the reference's CUDA kernels cannot build here"),
        "backend": backend.name,
        "sample": (f"{heads} of {B * H} heads (N={N}, D={D}, {'causal' if causal else 'full'}), "
                   f"torch {torch.__version__} F.scaled_dot_product_attention + backward, FP32, "
                   f"{threads} threads, median of 3 steps of {med:.3f} s"),
        "est_ms_per_full_step": round(med * 1e3 * B * H / heads, 1),
        **{k_: v_ for k_, v_ in host_info().items() if k_ in ("cpu_model", "cpu_count")},
    }


# Largest dS workspace the flash_attention_bwd operator allocates (torch_ops.cpp).
BWD_WORKSPACE_CAP = 8 << 30


def fa2_timings(B, H, N, D, causal, steps, warmup, schedule="stored", flushed_reps=5,
                warm_s=0.5):
    """Time `steps` FA2 steps through the C ABI on torch's current stream: fwd, then the
    backward stages of `schedule` ([delta, dkdv, dq_ds] stored; [dq forming delta, dkdv]
    recompute;
    one combined [bwd] launch when the stored schedule needs head chunks, as the operator
    runs it), after at least `warmup` untimed steps and warm_s seconds of them.  After the timed
    steps, each kernel is timed again `flushed_reps` times with FLUSH_BYTES read before every
    launch (cold L2 and MALL).  Returns (wall ms per step,
    {kernel: mean HIP-event ms in the timed steps}, {kernel: median flushed ms},
    (q, k, v, dO))."""
    import torch

    from cuda_transformer_amd import capi

    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, H, N, D, generator=gen).to(dev) for _ in range(3))
    do = torch.randn(B, H, N, D, generator=torch.Generator().manual_seed(1)).to(dev)
    O = torch.empty_like(q)
    L = torch.empty(B, H, N, device=dev)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)
    delta = torch.empty(B, H, N, device=dev)
    ws_full = capi.lib().cta_flash_attention_bwd_workspace(B, H, N, D, int(causal))
    ws_bytes = min(ws_full, BWD_WORKSPACE_CAP) if schedule in ("stored", "fold") else 0
    # small grids: the operator's split dK/dV and dQ-from-dS stages (their partial sums after
    # the dS tiles) and split forward, as flash_attention_fwd / flash_attention_bwd run them
    split_bytes = (capi.lib().cta_flash_attention_bwd_split_workspace(B, H, N, D, int(causal))
                   if schedule == "stored" and ws_bytes == ws_full else 0)
    ws_bytes += split_bytes
    ws = torch.empty(max(1, ws_bytes // 4), device=dev)
    fwd_ws_bytes = capi.lib().cta_flash_attention_fwd_workspace(B, H, N, D, int(causal))
    fwd_ws = torch.empty(max(1, fwd_ws_bytes // 4), device=dev)

    stream = torch.cuda.current_stream(dev)
    st = ctypes.c_void_p(stream.cuda_stream)
    s4 = capi.strides(q.stride())
    s3 = capi.strides(L.stride())
    P = {name: ctypes.c_void_p(t.data_ptr()) for name, t in
         dict(q=q, k=k, v=v, do=do, O=O, L=L, dq=dq, dk=dk, dv=dv, delta=delta, ws=ws,
              fws=fwd_ws).items()}
    lib = capi.lib()
    c = int(causal)

    def launch(kernel):
        if kernel == "fwd":
            rc = lib.cta_flash_attention_fwd_ex(P["q"], s4, P["k"], s4, P["v"], s4, B, H, N, D, c,
                                                P["O"], s4, P["L"], P["fws"], fwd_ws_bytes, st)
        elif kernel == "delta":
            rc = lib.cta_flash_attention_bwd_delta(P["O"], s4, P["do"], s4, B, H, N, D,
                                                   P["delta"], st)
        elif kernel == "dq":  # dQ of the reference schedule, forming delta as it goes
            rc = lib.cta_flash_attention_bwd_dq_delta(P["q"], s4, P["k"], s4, P["v"], s4, P["O"],
                                                      s4, P["do"], s4, P["L"], s3, B, H, N, D, c,
                                                      P["delta"], P["dq"], st)
        elif kernel == "dkdv" and schedule == "recompute":
            rc = lib.cta_flash_attention_bwd_dkdv(P["q"], s4, P["k"], s4, P["v"], s4, P["do"],
                                                  s4, P["L"], s3, P["delta"], B, H, N, D, c,
                                                  P["dk"], P["dv"], st)
        elif kernel == "dkdv":
            rc = lib.cta_flash_attention_bwd_dkdv_store_ds(
                P["q"], s4, P["k"], s4, P["v"], s4, P["do"], s4, P["L"], s3, P["delta"], B, H,
                N, D, c, P["dk"], P["dv"], P["ws"], st)
        elif kernel == "dq_ds":
            rc = lib.cta_flash_attention_bwd_dq_from_ds(P["k"], s4, P["ws"], B, H, N, D, c,
                                                        P["dq"], st)
        elif kernel == "bwd_fold":  # dK/dV with delta folded in, then dQ from dS
            rc = lib.cta_flash_attention_bwd_fold_delta(
                P["q"], s4, P["k"], s4, P["v"], s4, P["O"], s4, P["do"], s4, P["L"], s3, B, H, N,
                D, c, P["dq"], P["dk"], P["dv"], P["ws"], ws_bytes, st)
        else:  # "bwd": the combined entry point, chunked over heads
            rc = lib.cta_flash_attention_bwd(P["q"], s4, P["k"], s4, P["v"], s4, P["O"], s4,
                                             P["do"], s4, P["L"], s3, B, H, N, D, c, P["dq"],
                                             P["dk"], P["dv"], P["delta"], P["ws"], ws_bytes, st)
        if rc != 0:
            raise RuntimeError(f"{kernel}: {lib.cta_last_error().decode()}")

    if schedule == "recompute":
        kernels = ["fwd", "dq", "dkdv"]
    elif schedule == "fold":
        kernels = ["fwd", "bwd_fold"]
    elif ws_full <= ws_bytes and split_bytes == 0:
        kernels = ["fwd", "delta", "dkdv", "dq_ds"]
    else:
        kernels = ["fwd", "bwd"]

    def step(events=None):
        for i, kname in enumerate(kernels):
            if events is not None:
                events[i].record(stream)
            launch(kname)
        if events is not None:
            events[len(kernels)].record(stream)

    # at least `warmup` steps and at least warm_s of back-to-back steps: after the host-side CPU
    # baselines the GPU has idled and its clock must ramp up again
    t_warm, done = time.perf_counter(), 0
    while done < warmup or time.perf_counter() - t_warm < warm_s:
        step()
        done += 1
        if done % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()

    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(kernels) + 1)]
           for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(evs[i])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_kernel = {kname: sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps
                  for j, kname in enumerate(kernels)}

    # Cache-cold repetitions of each kernel (outside the timed region).
    import statistics

    flush = CacheFlush(dev)
    flushed = {}
    for kname in kernels:
        pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                 for _ in range(flushed_reps)]
        for a, b in pairs:
            flush()
            a.record(stream)
            launch(kname)
            b.record(stream)
        torch.cuda.synchronize()
        flushed[kname] = statistics.median(a.elapsed_time(b) for a, b in pairs)
    del flush
    return wall * 1e3 / steps, per_kernel, flushed, (q, k, v, do), done


def roofline_of(per_kernel, B, H, N, D, causal, flushed=None):
    """Roofline object of the dominant kernel among `per_kernel` (the combined "bwd" and
    "bwd_fold" launches are not single kernels and are left out): its algorithmic work per
    launch over its mean duration, against the FP32 MFMA or HBM peak."""
    kernel_symbols = {"fwd": "fa2_fwd_kernel", "delta": "fa2_bwd_delta_kernel",
                      "dq": "fa2_bwd_dq_kernel", "dkdv": "fa2_bwd_dkdv_kernel",
                      "dq_ds": "fa2_bwd_dq_ds_kernel"}
    dom = max((k_ for k_ in per_kernel if k_ in kernel_symbols), key=per_kernel.get)
    amount, unit, bound = kernel_algorithmic(dom, B, H, N, D, causal)
    scale, peak = (1e12, MFMA_FP32_PEAK_TFLOPS) if unit == "TFLOP/s" else (1e9, HBM_PEAK_GBPS)
    achieved = amount / (per_kernel[dom] * 1e-3) / scale
    out = {"kernel": kernel_symbols[dom], "bound": bound, "achieved": round(achieved, 3),
           "peak": peak, "unit": unit, "frac": round(achieved / peak, 4),
           "traffic": None, "algorithmic_per_launch": amount,
           "mean_launch_ms": round(per_kernel[dom], 4)}
    if flushed and dom in flushed:
        af = amount / (flushed[dom] * 1e-3) / scale
        out["achieved_flushed"] = round(af, 3)
        out["frac_flushed"] = round(af / peak, 4)
    return out


def fa2_sweep(args):
    """Benchmark config 3: non-causal B4 H32 D64, N in {1024 ... 16384} (or --seqs); one JSON
    line per N in the layout of the reference's sweep table (README.md:38-56): forward and
    backward TFLOPS and fraction of peak, per-kernel times (in the timed steps and cache-cold),
    the dominant kernel's roofline, and the torch SDPA CPU path on a bounded head sample."""
    import torch

    from cuda_transformer_amd import capi

    seqs = [int(x) for x in args.seqs.split(",")] if args.seqs else [1024, 2048, 4096, 8192,
                                                                      16384]
    B, H, D = 4, 32, 64
    for N in seqs:
        steps = max(2, args.steps // max(1, N // 2048))
        ms, per_kernel, flushed, _, warm = fa2_timings(B, H, N, D, False, steps, args.warmup,
                                                       args.bwd_schedule,
                                                       warm_s=args.warm_seconds)
        fwd_fl, bwd_fl = attn_flops(B, H, N, D, False)
        bwd_ms = sum(v_ for k_, v_ in per_kernel.items() if k_ != "fwd")
        bwd_ms_f = sum(v_ for k_, v_ in flushed.items() if k_ != "fwd")
        ws_full = capi.lib().cta_flash_attention_bwd_workspace(B, H, N, D, 0)
        head = capi.lib().cta_flash_attention_bwd_workspace(1, 1, N, D, 0)
        fit = min(B * H, BWD_WORKSPACE_CAP // head)
        chunks = -(-B * H // fit) if args.bwd_schedule == "stored" else 0
        line = {
            "workload": f"FA2 B{B} H{H} N{N} D{D} non-causal", "N": N, "steps": steps,
            "warmup_steps_run": warm,
            "dtype": "f32", "bwd_schedule": args.bwd_schedule, "bwd_head_chunks": chunks,
            "ds_workspace_bytes": min(ws_full, BWD_WORKSPACE_CAP),
            "ms_per_step": round(ms, 4),
            "fwd_ms": round(per_kernel["fwd"], 4), "bwd_ms": round(bwd_ms, 4),
            "fwd_tflops": round(fwd_fl / per_kernel["fwd"] / 1e9, 3),
            "bwd_tflops": round(bwd_fl / bwd_ms / 1e9, 3),
            "fwd_frac_of_peak": round(fwd_fl / per_kernel["fwd"] / 1e9 / MFMA_FP32_PEAK_TFLOPS, 4),
            "bwd_frac_of_peak": round(bwd_fl / bwd_ms / 1e9 / MFMA_FP32_PEAK_TFLOPS, 4),
            "fwd_tflops_flushed": round(fwd_fl / flushed["fwd"] / 1e9, 3),
            "bwd_tflops_flushed": round(bwd_fl / bwd_ms_f / 1e9, 3),
            "per_kernel_ms": {k_: round(v_, 4) for k_, v_ in per_kernel.items()},
            "per_kernel_ms_flushed": {k_: round(v_, 4) for k_, v_ in flushed.items()},
            "roofline": roofline_of(per_kernel, B, H, N, D, False, flushed),
        }
        torch.cuda.empty_cache()
        if not args.no_cpu_baseline:
            line["cpu_baseline"] = cpu_reference_path(B, H, N, D, False)
        print(json.dumps(line), flush=True)
    return 0


def fa2_half_workload(args, kind):
    """The 16-bit FlashAttention-2 step (kind "bf16" or "f16") at the config-2 shape, causal and
    non-causal: forward (cta_flash_attention_fwd_<kind>) and backward
    (cta_flash_attention_bwd_<kind>) in both schedules, recompute (no workspace: dQ recomputing
    S and dP and forming delta, then dK/dV) and stored dS (delta, dK/dV storing 16-bit dS, dQ from
    dS).  Each schedule is timed as whole steps [fwd, bwd] back to back on torch's current stream
    with inputs in HBM, HIP events around each launch, like the FP32 headline.  `value` is the
    wall-clock step rate with the schedule the operator runs (recompute at hs 32 and 64, stored
    at hs 128).  TFLOPS by the reference's formula (forward 4*B*H*N^2*D, halved when causal;
    backward 2.5x), against the 2.5 PFLOP/s dense BF16/FP16 MFMA peak.  One JSON line per
    mask."""
    import torch

    from cuda_transformer_amd import capi

    B, H, N, D = args.batch, args.heads, args.seq, args.head_dim
    dev = torch.device("cuda", 0)
    gen = torch.Generator().manual_seed(0)
    dt = torch.bfloat16 if kind == "bf16" else torch.float16
    q, k, v = (torch.randn(B, H, N, D, generator=gen).to(dt).to(dev) for _ in range(3))
    do = torch.randn(B, H, N, D, generator=torch.Generator().manual_seed(1)).to(dt).to(dev)
    O = torch.empty_like(q)
    L = torch.empty(B, H, N, device=dev)
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    delta = torch.empty(B, H, N, device=dev)
    lib = capi.lib()
    fwd_fn = getattr(lib, f"cta_flash_attention_fwd_{kind}")
    bwd_fn = getattr(lib, f"cta_flash_attention_bwd_{kind}")
    ws_fn = getattr(lib, f"cta_flash_attention_bwd_{kind}_workspace")
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    s4, s3 = capi.strides(q.stride()), capi.strides(L.stride())
    vp = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    masks = {"both": (True, False), "causal": (True,), "full": (False,)}[args.masks]
    default = "stored" if D == 128 else "recompute"
    for causal in masks:
        ws_bytes = ws_fn(B, H, N, D, int(causal))
        ws = torch.empty(ws_bytes // 4 + 4, device=dev)

        def fwd():
            if fwd_fn(vp(q), s4, vp(k), s4, vp(v), s4, B, H, N, D, int(causal), vp(O), vp(L),
                      st) != 0:
                raise RuntimeError(lib.cta_last_error().decode())

        def bwd(stored):
            if bwd_fn(vp(q), s4, vp(k), s4, vp(v), s4, vp(O), s4, vp(do), s4, vp(L), s3, B, H,
                      N, D, int(causal), vp(dq), vp(dk), vp(dv), vp(delta),
                      vp(ws) if stored else None, ws_bytes if stored else 0, st) != 0:
                raise RuntimeError(lib.cta_last_error().decode())
        # whole steps [fwd, bwd] per schedule, the operator's schedule first, timed as the FP32
        # headline is: the forward runs between backwards, as in training
        timed = {}
        for sch in (default, "stored" if default == "recompute" else "recompute"):
            timed[sch] = _time_steps(
                [("fwd", fwd), ("bwd", lambda sch=sch: bwd(sch == "stored"))],
                max(10, args.steps), args.warm_seconds)
        fwd_ms = timed[default][1]["fwd"]
        bwd_ms = {sch: t[1]["bwd"] for sch, t in timed.items()}
        fl, bfl = attn_flops(B, H, N, D, causal)
        ftf = fl / (fwd_ms * 1e-3) / 1e12
        btf = {sch: bfl / (ms * 1e-3) / 1e12 for sch, ms in bwd_ms.items()}
        stf = {sch: (fl + bfl) / (t[0] * 1e-3) / 1e12 for sch, t in timed.items()}
        print(json.dumps({
            "workload": f"FA2 {kind.upper()} fwd+bwd B{B} H{H} N{N} D{D} "
                        f"{'causal' if causal else 'non-causal'}",
            "metric": f"FA2 {kind.upper()} fwd+bwd TFLOPS", "value": round(stf[default], 2),
            "unit": "TFLOPS", "bwd_schedule": default,
            "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms[default], 4),
            "fwd_tflops": round(ftf, 2), "bwd_tflops": round(btf[default], 2),
            "ms_per_step": round(timed[default][0], 4),
            "schedules": {sch: {"fwd_ms": round(timed[sch][1]["fwd"], 4),
                                "bwd_ms": round(bwd_ms[sch], 4), "bwd_tflops": round(btf[sch], 2),
                                "ms_per_step": round(timed[sch][0], 4),
                                "step_tflops": round(stf[sch], 2),
                                "ds_workspace_bytes": ws_bytes if sch == "stored" else 0}
                          for sch in bwd_ms},
            "dtype": f"{kind} inputs, fp32 accumulation",
            "roofline": {"bound": "mfma", "achieved": round(stf[default], 2),
                         "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(stf[default] / MFMA_BF16_PEAK_TFLOPS, 4),
                         "algorithmic_per_launch": fl + bfl},
        }), flush=True)
        del ws
    return 0


def _time_kernel(fn, reps, warm_s=0.02, flush=None):
    """Median HIP-event duration (ms) of fn's launches on torch's current stream, over at least
    20 launches, after at least warm_s of back-to-back launches: the CPU-baseline timings between
    ops leave the GPU idle long enough for its clocks to drop.  With `flush` (a CacheFlush), the
    flush runs before every timed launch, outside its event pair, so each launch starts with
    cold L2s and MALL."""
    import statistics

    import torch

    t0 = time.perf_counter()
    while True:
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= warm_s:
            break
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(max(20, reps))]
    for a, b in evs:
        if flush is not None:
            flush()
        a.record(stream)
        fn()
        b.record(stream)
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in evs)


def _time_steps(kernels, steps, warm_s):
    """Whole steps of `kernels` ([(name, fn), ...], launched in order) back to back on torch's
    current stream: at least warm_s of untimed steps, then `steps` timed ones with HIP events
    around each kernel.  Returns (wall-clock ms per timed step, {name: mean event ms})."""
    import torch

    t0 = time.perf_counter()
    while True:
        for _ in range(2):
            for _, fn in kernels:
                fn()
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= warm_s:
            break
    stream = torch.cuda.current_stream()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(len(kernels) + 1)]
           for _ in range(steps)]
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    for e in evs:
        for j, (_, fn) in enumerate(kernels):
            e[j].record(stream)
            fn()
        e[len(kernels)].record(stream)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t1) * 1e3 / steps
    per = {name: sum(e[j].elapsed_time(e[j + 1]) for e in evs) / steps
           for j, (name, _) in enumerate(kernels)}
    return wall, per


def _time_rotating(fn, copies, reps, warm_s=0.02):
    """Median HIP-event duration (ms) of fn(i) over at least 20 back-to-back launches, launch i
    on buffer copy i % copies: with copies x footprint >= ROTATE_BYTES, each launch's operands
    were last touched copies - 1 launches earlier and have left the L2s and the MALL, and every
    launch pays in steady state for the write-backs of the lines it dirties."""
    import statistics

    import torch

    t0, i = time.perf_counter(), 0
    while True:
        for _ in range(2 * copies):
            fn(i % copies)
            i += 1
        torch.cuda.synchronize()
        if time.perf_counter() - t0 >= warm_s:
            break
    stream = torch.cuda.current_stream()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(max(20, reps))]
    for a, b in evs:
        a.record(stream)
        fn(i % copies)
        i += 1
        b.record(stream)
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in evs)


def rotation_copies(footprint_bytes):
    """Buffer copies a rotating timing needs for footprint_bytes per launch."""
    return max(2, -(-ROTATE_BYTES // int(footprint_bytes)))


def _cpu_time(fn, target_s=2.0):
    """Seconds per call of a CPU function, repeated until about target_s."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= target_s or n >= 50:
            return el / n


def ops_workload(args):
    """Benchmark config 4 (GPT-2-small widths, FP32): linear GEMM fwd/bwd, db, exact and
    tanh-approximated GELU, LayerNorm and row softmax, each launched through the C ABI.  One JSON
    line per op with the kernel's roofline (MFMA TFLOP/s for GEMMs, HBM GB/s otherwise).  Each op
    is timed cache-cold, the primary figure ("ms"): launches rotate over copies of the operands
    totalling at least ROTATE_BYTES, so every launch reads operands that left the caches and pays
    for its own write-backs in steady state.  Beside it, "ms_unflushed": back-to-back launches on
    one set of buffers (operands under 256 MB may then be served partly by the MALL).  CPU
    baseline: torch's own CPU kernels for the same op (the reference's test oracle path:
    test/test_linear.py, test_gelu.py, test_softmax.py; gpt/gpt.py:47-59 for LayerNorm) on 1/8 of
    the rows, on this host's cores."""
    import torch
    import torch.nn.functional as F

    from cuda_transformer_amd import capi

    lib = capi.lib()
    dev = torch.device("cuda", 0)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    reps = max(20, args.steps)
    g = torch.Generator().manual_seed(0)
    cores = min(16, os.cpu_count() or 1)
    torch.set_num_threads(cores)
    host = host_info()
    aten = torch.ops.aten

    def copies_of(*tensors):
        """Rotation sets: the given device tensors, then clones until ROTATE_BYTES."""
        nbytes = sum(t.numel() * t.element_size() for t in tensors if t is not None)
        k = rotation_copies(nbytes)
        return [tensors] + [tuple(None if t is None else t.clone() for t in tensors)
                            for _ in range(k - 1)]

    def cpu(fn):
        return None if args.no_cpu_baseline else _cpu_time(fn, 1.0)

    def timed(fn, sets):
        return (_time_rotating(lambda i: fn(*sets[i]), len(sets), reps),
                _time_kernel(lambda: fn(*sets[0]), reps))

    def emit(name, shape, ms_pair, amount, unit, cpu_s, cpu_amount, sample, copies):
        ms, ms_warm = ms_pair
        scale, peak = (1e12, MFMA_FP32_PEAK_TFLOPS) if unit == "TFLOP/s" else (1e9, HBM_PEAK_GBPS)
        achieved, warm = amount / (ms * 1e-3) / scale, amount / (ms_warm * 1e-3) / scale
        print(json.dumps({
            "workload": name, "shape": shape, "dtype": "f32", "ms": round(ms, 5),
            "ms_unflushed": round(ms_warm, 5), "rotation_copies": copies, "value": round(achieved, 3),
            "unit": unit,
            "roofline": {"bound": "mfma" if unit == "TFLOP/s" else "hbm",
                         "achieved": round(achieved, 3), "peak": peak,
                         "frac": round(achieved / peak, 4), "algorithmic_per_launch": amount,
                         "achieved_unflushed": round(warm, 3),
                         "frac_unflushed": round(warm / peak, 4)},
            "cpu_baseline": None if cpu_s is None else {
                "value": round(cpu_amount / cpu_s / scale, 4), "unit": unit, "cores": cores,
                "kind": "reference", "sample": sample, "cpu_model": host["cpu_model"]},
        }), flush=True)

    def cpu8(what):
        return f"torch {torch.__version__} CPU {what}, FP32, rows 0..1/8, {cores} threads"

    # ---- the practical HBM ceiling for a stream that reads and writes: a device-to-device copy
    # of 256 MiB (torch's copy kernel), timed the same way as the ops below
    src = torch.ones(1 << 26, device=dev)
    sets = copies_of(src, torch.empty_like(src))
    emit("device_copy (torch copy_, 256 MiB, reference ceiling)", [1 << 26],
         timed(lambda a_, b_: b_.copy_(a_), sets), 8.0 * (1 << 26), "GB/s", None, 0.0, "",
         len(sets))
    del src, sets
    # ... and this library's own dwordx4 copy (cta_device_copy) at 256 MiB and at the sizes of
    # the LayerNorm passes below (50.3 MB and 75.5 MB moved): the ceiling of a read + write
    # stream of that length, launch ramp included
    for nfl in (1 << 26, 8192 * 768, 8192 * 768 * 3 // 2):
        src = torch.ones(nfl, device=dev)
        sets = copies_of(src, torch.empty_like(src))
        emit(f"device_copy (cta_device_copy, {nfl * 4 / 2**20:.0f} MiB)", [nfl],
             timed(lambda a_, b_: lib.cta_device_copy(vp(a_), vp(b_), nfl, st), sets),
             8.0 * nfl, "GB/s", None, 0.0, "", len(sets))
        del src, sets

    # ---- linear layer: X[8192,768] . W[768,3072] + b, X, W ~ N(0, 0.02^2)
    M, K, Nn = 8192, 768, 3072
    x = (torch.randn(1, M, K, generator=g) * 0.02).to(dev)
    w = (torch.randn(K, Nn, generator=g) * 0.02).to(dev)
    b = (torch.randn(Nn, generator=g) * 0.02).to(dev)
    dy = (torch.randn(1, M, Nn, generator=g) * 0.02).to(dev)
    xs, ws = capi.strides(x.stride()), capi.strides((0, Nn, 1))
    wts = capi.strides((0, 1, Nn))              # W^T view (1, n=3072 -> k, 768)
    dys = capi.strides(dy.stride())
    xts = capi.strides((M * K, 1, K))           # x^T view (1, 768, 8192)
    fl = 2.0 * M * K * Nn
    rows = M // 8
    xc, wc, bc, dyc = x[0, :rows].cpu(), w.cpu(), b.cpu(), dy[0, :rows].cpu()
    zk, zn = torch.zeros(K, device=dev), torch.zeros(Nn, device=dev)

    def scratch(m_, k_, n_):
        nbytes = lib.cta_cuda_fma_workspace(1, m_, k_, n_)
        return torch.empty(max(1, nbytes // 4), device=dev) if nbytes else None

    def gemm_fwd(x_, w_, b_, out_, ws_):
        assert lib.cta_cuda_fma(vp(x_), xs, vp(w_), ws, vp(b_), 1, 1, M, K, Nn, 1, vp(out_),
                                vp(ws_), st) == 0
    sets = copies_of(x, w, b, torch.empty(1, M, Nn, device=dev), scratch(M, K, Nn))
    emit("linear_fwd (cuda_fma)", [M, K, Nn], timed(gemm_fwd, sets), fl, "TFLOP/s",
         cpu(lambda: torch.addmm(bc, xc, wc)), fl / 8, cpu8("addmm"), len(sets))

    def gemm_dx(dy_, w_, dx_, ws_):
        assert lib.cta_cuda_fma(vp(dy_), dys, vp(w_), wts, vp(zk), 1, 1, M, Nn, K, 1, vp(dx_),
                                vp(ws_), st) == 0
    sets = copies_of(dy, w, torch.empty(1, M, K, device=dev), scratch(M, Nn, K))
    emit("linear_bwd_dx (cuda_fma, W^T view)", [M, Nn, K], timed(gemm_dx, sets), fl, "TFLOP/s",
         cpu(lambda: dyc @ wc.T), fl / 8, cpu8("dy @ W^T"), len(sets))

    def gemm_dw(x_, dy_, dw_, ws_):
        assert lib.cta_cuda_fma(vp(x_), xts, vp(dy_), dys, vp(zn), 1, 1, K, M, Nn, 1, vp(dw_),
                                vp(ws_), st) == 0
    sets = copies_of(x, dy, torch.empty(1, K, Nn, device=dev), scratch(K, M, Nn))
    emit("linear_bwd_dw (cuda_fma, x^T view)", [K, M, Nn], timed(gemm_dw, sets), fl, "TFLOP/s",
         cpu(lambda: xc.T @ dyc), fl / 8, cpu8("x^T @ dy"), len(sets))

    def dbk(dy_, db_, ws_):
        assert lib.cta_db_calculation(vp(dy_), dys, 1, M, Nn, vp(db_), vp(ws_), st) == 0
    sets = copies_of(dy, torch.empty(Nn, device=dev),
                     torch.empty(lib.cta_db_calculation_workspace(1, M, Nn) // 4, device=dev))
    emit("db_calculation", [M, Nn], timed(dbk, sets), 4.0 * M * Nn + 4 * Nn, "GB/s",
         cpu(lambda: dyc.sum(0)), 4.0 * rows * Nn, cpu8("dy.sum(0)"), len(sets))
    del x, w, dy, sets

    # ---- exact and tanh-approximated GELU on [8192, 3072]
    n = M * Nn
    xg = torch.randn(n, generator=g).to(dev)
    gg = torch.randn(n, generator=g).to(dev)
    xgc, ggc = xg[: n // 8].cpu(), gg[: n // 8].cpu()
    fsets = copies_of(xg, torch.empty_like(xg))
    bsets = copies_of(xg, gg, torch.empty_like(xg))
    for approx, fwd_fn, bwd_fn, tag in (("none", lib.cta_gelu_fwd, lib.cta_gelu_bwd, ""),
                                        ("tanh", lib.cta_gelu_tanh_fwd, lib.cta_gelu_tanh_bwd,
                                         "_tanh")):
        emit(f"gelu{tag}_fwd", [M, Nn], timed(lambda x_, y_: fwd_fn(vp(x_), vp(y_), n, st), fsets),
             8.0 * n, "GB/s", cpu(lambda: F.gelu(xgc, approximate=approx)),
             8.0 * n / 8, cpu8(f"F.gelu(approximate={approx!r})"), len(fsets))
        emit(f"gelu{tag}_bwd", [M, Nn],
             timed(lambda x_, g_, d_: bwd_fn(vp(x_), vp(g_), vp(d_), n, st), bsets),
             12.0 * n, "GB/s",
             cpu(lambda: aten.gelu_backward(ggc, xgc, approximate=approx)),
             12.0 * n / 8, cpu8("aten.gelu_backward"), len(bsets))
    del xg, gg, fsets, bsets

    # ---- LayerNorm over 768 on [8192, 768], gamma = 1, beta = 0
    R, C = 8192, 768
    xl = torch.randn(R, C, generator=g).to(dev)
    gam, bet = torch.ones(C, device=dev), torch.zeros(C, device=dev)
    dyl = torch.randn(R, C, generator=g).to(dev)
    xlc, dylc = xl[: R // 8].cpu(), dyl[: R // 8].cpu()
    gamc, betc = gam.cpu(), bet.cpu()
    eps = ctypes.c_float(1e-5)
    mean, rstd = torch.empty(R, device=dev), torch.empty(R, device=dev)
    assert lib.cta_layernorm_fwd(vp(xl), vp(gam), vp(bet), R, C, eps, vp(torch.empty_like(xl)),
                                 vp(mean), vp(rstd), st) == 0

    def ln_fwd(x_, y_, m_, r_):
        assert lib.cta_layernorm_fwd(vp(x_), vp(gam), vp(bet), R, C, eps, vp(y_), vp(m_),
                                     vp(r_), st) == 0
    sets = copies_of(xl, torch.empty_like(xl), torch.empty(R, device=dev),
                     torch.empty(R, device=dev))
    emit("layernorm_fwd", [R, C], timed(ln_fwd, sets), 8.0 * R * C + 8 * R, "GB/s",
         cpu(lambda: aten.native_layer_norm(xlc, [C], gamc, betc, 1e-5)),
         (8.0 * R * C + 8 * R) / 8, cpu8("aten.native_layer_norm"), len(sets))
    _, mc, rc_ = aten.native_layer_norm(xlc, [C], gamc, betc, 1e-5)

    def ln_bwd(x_, m_, r_, dy_, dx_, dg_, db_, ws_):
        assert lib.cta_layernorm_bwd(vp(x_), vp(gam), vp(m_), vp(r_), vp(dy_), R, C, vp(dx_),
                                     vp(dg_), vp(db_), vp(ws_), st) == 0
    sets = copies_of(xl, mean, rstd, dyl, torch.empty_like(xl), torch.empty(C, device=dev),
                     torch.empty(C, device=dev),
                     torch.empty(lib.cta_layernorm_bwd_workspace(R, C) // 4, device=dev))
    emit("layernorm_bwd", [R, C], timed(ln_bwd, sets), 12.0 * R * C + 8 * R + 8 * C, "GB/s",
         cpu(lambda: aten.native_layer_norm_backward(dylc, xlc, [C], mc, rc_, gamc, betc,
                                                           [True, True, True])),
         (12.0 * R * C + 8 * R) / 8, cpu8("aten.native_layer_norm_backward"), len(sets))
    del xl, dyl, sets

    # ---- row softmax on [4*12*1024, 1024], logits ~ N(0, 4)
    R, C = 4 * 12 * 1024, 1024
    xs_ = (torch.randn(R, C, generator=g) * 2).to(dev)
    dps = torch.rand(R, C, generator=g).to(dev)
    xsc, dpsc = xs_[: R // 8].cpu(), dps[: R // 8].cpu()
    sets = copies_of(xs_, torch.empty_like(xs_))
    emit("softmax_fwd", [R, C],
         timed(lambda x_, y_: lib.cta_softmax_fwd(vp(x_), vp(y_), R, C, st), sets),
         8.0 * R * C, "GB/s", cpu(lambda: F.softmax(xsc, dim=-1)), 8.0 * R * C / 8,
         cpu8("F.softmax"), len(sets))
    ps_ = torch.empty_like(xs_)
    assert lib.cta_softmax_fwd(vp(xs_), vp(ps_), R, C, st) == 0
    del sets
    psc = F.softmax(xsc, dim=-1)
    sets = copies_of(ps_, dps, torch.empty_like(xs_))
    emit("softmax_bwd", [R, C],
         timed(lambda p_, g_, d_: lib.cta_softmax_bwd(vp(p_), vp(g_), vp(d_), R, C, st), sets),
         12.0 * R * C, "GB/s",
         cpu(lambda: aten._softmax_backward_data(dpsc, psc, -1, torch.float32)),
         12.0 * R * C / 8, cpu8("aten._softmax_backward_data"), len(sets))
    return 0


def gemm_workload(args):
    """The FP32 GEMMs of the config-5 GPT step (6 layers, d 384, batch 64 x 256 = 16384 rows) and
    of config 4, each timed A/B in this process against torch's own FP32 GEMM (hipBLASLt / rocBLAS
    through torch.addmm / torch.matmul, TF32 off) on the same operands: forward x.W + b, dx =
    dy.W^T (transposed view) and dW = x^T.dy (transposed view, split along K).  Cache-cold:
    launches rotate over operand copies of at least ROTATE_BYTES.  One JSON line per product."""
    import torch

    from cuda_transformer_amd import capi

    torch.backends.cuda.matmul.allow_tf32 = False
    lib = capi.lib()
    dev = torch.device("cuda", 0)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    vp = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())  # noqa: E731
    reps = max(20, args.steps)
    g = torch.Generator().manual_seed(0)
    R = 64 * 256
    shapes = [("gpt qkv", R, 384, 1152), ("gpt proj", R, 384, 384), ("gpt fc1", R, 384, 1536),
              ("gpt fc2", R, 1536, 384), ("gpt lm_head", R, 384, 65),
              ("config-4 linear", 8192, 768, 3072)]

    def copies_of(*tensors):
        nbytes = sum(t.numel() * t.element_size() for t in tensors if t is not None)
        k = rotation_copies(nbytes)
        return [tensors] + [tuple(None if t is None else t.clone() for t in tensors)
                            for _ in range(k - 1)]

    def ws_for(m_, k_, n_):
        nbytes = lib.cta_cuda_fma_workspace(1, m_, k_, n_)
        return torch.empty(max(1, nbytes // 4), device=dev) if nbytes else None

    for name, M, K, N in shapes:
        x = (torch.randn(1, M, K, generator=g) * 0.02).to(dev)
        w = (torch.randn(K, N, generator=g) * 0.02).to(dev)
        b = (torch.randn(N, generator=g) * 0.02).to(dev)
        dy = (torch.randn(1, M, N, generator=g) * 0.02).to(dev)
        zk, zn = torch.zeros(K, device=dev), torch.zeros(N, device=dev)
        s3 = capi.strides
        products = {
            # name: (ours(set), torch(set), operand set, m, k, n of the product)
            "fwd": (lambda x_, w_, b_, o_, ws_: lib.cta_cuda_fma(
                        vp(x_), s3(x_.stride()), vp(w_), s3((0, N, 1)), vp(b_), 1, 1, M, K, N, 1,
                        vp(o_), vp(ws_), st),
                    lambda x_, w_, b_, o_, ws_: torch.addmm(b_, x_[0], w_, out=o_[0]),
                    (x, w, b, torch.empty(1, M, N, device=dev), ws_for(M, K, N)), M, K, N),
            "dx": (lambda d_, w_, o_, ws_: lib.cta_cuda_fma(
                       vp(d_), s3(d_.stride()), vp(w_), s3((0, 1, N)), vp(zk), 1, 1, M, N, K, 1,
                       vp(o_), vp(ws_), st),
                   lambda d_, w_, o_, ws_: torch.matmul(d_[0], w_.t(), out=o_[0]),
                   (dy, w, torch.empty(1, M, K, device=dev), ws_for(M, N, K)), M, N, K),
            "dW": (lambda x_, d_, o_, ws_: lib.cta_cuda_fma(
                       vp(x_), s3((M * K, 1, K)), vp(d_), s3(d_.stride()), vp(zn), 1, 1, K, M, N, 1,
                       vp(o_), vp(ws_), st),
                   lambda x_, d_, o_, ws_: torch.matmul(x_[0].t(), d_[0], out=o_[0]),
                   (x, dy, torch.empty(1, K, N, device=dev), ws_for(K, M, N)), K, M, N),
        }
        for pname, (ours, theirs, operands, pm, pk, pn) in products.items():
            sets = copies_of(*operands)

            def run_ours(i, ours=ours, sets=sets):
                rc = ours(*sets[i])
                if rc != 0:
                    raise RuntimeError(lib.cta_last_error().decode())

            def run_lib(i, theirs=theirs, sets=sets):
                theirs(*sets[i])

            # Five rounds, alternating which side goes first; the median of each side's rounds.
            ts_ours, ts_lib = [], []
            for rnd in range(5):
                pair = ((run_ours, ts_ours), (run_lib, ts_lib))
                for fn, acc in (pair if rnd % 2 == 0 else pair[::-1]):
                    acc.append(_time_rotating(fn, len(sets), reps))
            t_ours, t_lib = statistics.median(ts_ours), statistics.median(ts_lib)
            fl = 2.0 * pm * pk * pn
            print(json.dumps({
                "workload": f"{name} {pname}", "m_k_n": [pm, pk, pn], "dtype": "f32",
                "ms": round(t_ours, 5), "tflops": round(fl / t_ours / 1e9, 2),
                "frac_of_peak": round(fl / t_ours / 1e9 / MFMA_FP32_PEAK_TFLOPS, 4),
                "torch_ms": round(t_lib, 5), "torch_tflops": round(fl / t_lib / 1e9, 2),
                "ours_over_torch_time": round(t_ours / t_lib, 3),
                "splitk_workspace": operands[-1] is not None,
            }), flush=True)
            del sets
        del x, w, b, dy
        torch.cuda.empty_cache()
    return 0


def gpt_workload(args):
    """Benchmark config 5: one training step (fwd + bwd + AdamW) of the small GPT on the HIP
    kernels (cuda_transformer_amd/gpt.py), batch 64 x context 256; tokens/s.  CPU baseline: the
    plain-torch model (oracle/gpt.py) on this host, batch 8, same step."""
    import torch

    from cuda_transformer_amd.gpt import GPT, GPTConfig, init_weights_, synthetic_batch
    from oracle import gpt as ogpt

    cfg, batch = GPTConfig(fused_mlp=args.gpt_mlp == "fused"), 64
    model = GPT(cfg)
    init_weights_(model, seed=0)
    model.cuda()
    opt = torch.optim.AdamW(model.parameters(), lr=6e-4, fused=args.gpt_adamw == "fused")
    batches = [synthetic_batch(cfg, batch, seed=s, device="cuda") for s in range(4)]

    def step(i, optimize=True):
        opt.zero_grad(set_to_none=True)
        _, loss = model(*batches[i % 4])
        loss.backward()
        if optimize:
            opt.step()
        return loss

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / args.steps
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i, optimize=False)
    torch.cuda.synchronize()
    ms_fb = (time.perf_counter() - t0) * 1e3 / args.steps
    tokens = batch * cfg.block_size

    cpu = None
    if not args.no_cpu_baseline:
        cores = min(16, os.cpu_count() or 1)
        torch.set_num_threads(cores)
        ref = ogpt.GPT(cfg)
        ref.load_state_dict({k: v.cpu() for k, v in model.state_dict().items()})
        ropt = torch.optim.AdamW(ref.parameters(), lr=6e-4)
        cb = 8
        idx, tgt = synthetic_batch(cfg, cb, seed=0)

        def cpu_step():
            ropt.zero_grad(set_to_none=True)
            _, l_ = ref(idx, tgt)
            l_.backward()
            ropt.step()

        cpu_s = _cpu_time(cpu_step, target_s=args.cpu_seconds)
        cpu = {"value": round(cb * cfg.block_size / cpu_s, 1), "unit": "tokens/s", "cores": cores,
               "kind": "port", "sample": f"batch {cb} x {cfg.block_size} tokens, plain-torch model "
                                         f"(oracle/gpt.py), fwd+bwd+AdamW, float32, "
                                         f"{torch.get_num_threads()} threads"}
    print(json.dumps({
        "workload": "small-GPT training step (6L 6H d384 ctx256 vocab65, batch 64), FP32",
        "value": round(tokens / (ms * 1e-3), 1), "unit": "tokens/s", "ms_per_step": round(ms, 3),
        "fwd_bwd_ms": round(ms_fb, 3), "fwd_bwd_tokens_per_s": round(tokens / (ms_fb * 1e-3), 1),
        "steps": args.steps, "mlp": args.gpt_mlp, "adamw": args.gpt_adamw,
        "model_options": {k: getattr(cfg, k) for k in ("fused_mlp", "packed_attention",
                                                       "fused_residual_ln", "cuda_embedding")},
        "cpu_baseline": cpu,
    }), flush=True)
    return 0


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}, WORLD_SIZE={world}): "
              "this build is single-GPU; multi-GPU sharding is a design note, not a benchmark.",
              file=sys.stderr)
        return 2

    if args.copy_calibration_mib:
        return copy_calibration(args.copy_calibration_mib)

    import torch

    import cuda_transformer_amd  # noqa: F401  (fails loudly if the native library is missing)

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if args.workload == "ops":
        return ops_workload(args)
    if args.workload == "fa2-sweep":
        return fa2_sweep(args)
    if args.workload == "gpt":
        return gpt_workload(args)
    if args.workload == "gemm":
        return gemm_workload(args)
    if args.workload in ("fa2-bf16", "fa2-f16"):
        return fa2_half_workload(args, args.workload[4:])
    B, H, N, D = args.batch, args.heads, args.seq, args.head_dim
    causal = not args.non_causal
    ms_step, per_kernel, flushed, (q, k, v, do), warm = fa2_timings(
        B, H, N, D, causal, args.steps, args.warmup, args.bwd_schedule,
        warm_s=args.warm_seconds)

    fwd_fl, bwd_fl = attn_flops(B, H, N, D, causal)
    value = (fwd_fl + bwd_fl) / (ms_step * 1e-3) / 1e12
    fwd_tf = fwd_fl / (per_kernel["fwd"] * 1e-3) / 1e12
    bwd_ms = sum(v_ for k_, v_ in per_kernel.items() if k_ != "fwd")
    bwd_tf = bwd_fl / (bwd_ms * 1e-3) / 1e12

    roofline = roofline_of(per_kernel, B, H, N, D, causal, flushed)
    is_config2 = (B, H, N, D, causal) == (4, 32, 4096, 64, True)
    stored_summary = ("fa2_config2_counters.md" if args.bwd_schedule == "stored"
                      else "fa2_config2_recompute_counters.md")
    roofline["traffic"] = load_traffic(roofline["kernel"], stored_summary) if is_config2 else None
    from cuda_transformer_amd import capi

    ws_full = capi.lib().cta_flash_attention_bwd_workspace(B, H, N, D, int(causal))
    ds_ws = min(ws_full, BWD_WORKSPACE_CAP) if args.bwd_schedule in ("stored", "fold") else 0

    recompute = None
    if args.bwd_schedule == "stored" and not args.no_recompute:
        # The reference's O(N)-memory schedule in the same run, after the headline's timing.
        r_ms, r_pk, r_fl, _, r_warm = fa2_timings(B, H, N, D, causal, max(3, args.steps // 2),
                                                  args.warmup, "recompute",
                                                  warm_s=args.warm_seconds)
        r_bwd = sum(v_ for k_, v_ in r_pk.items() if k_ != "fwd")
        r_roof = roofline_of(r_pk, B, H, N, D, causal, r_fl)
        r_roof["traffic"] = (load_traffic(r_roof["kernel"], "fa2_config2_recompute_counters.md")
                             if is_config2 else None)
        recompute = {
            "bwd_schedule": "recompute", "ds_workspace_bytes": 0,
            "steps": max(3, args.steps // 2), "warmup_steps_run": r_warm,
            "ms_per_step": round(r_ms, 4),
            "tflops": round((fwd_fl + bwd_fl) / (r_ms * 1e-3) / 1e12, 3),
            "fwd_tflops": round(fwd_fl / (r_pk["fwd"] * 1e-3) / 1e12, 3),
            "bwd_tflops": round(bwd_fl / (r_bwd * 1e-3) / 1e12, 3),
            "bwd_frac_of_peak": round(bwd_fl / (r_bwd * 1e-3) / 1e12 / MFMA_FP32_PEAK_TFLOPS, 4),
            "per_kernel_ms": {k_: round(v_, 4) for k_, v_ in r_pk.items()},
            "per_kernel_ms_flushed": {k_: round(v_, 4) for k_, v_ in r_fl.items()},
            "roofline": r_roof,
        }
        torch.cuda.empty_cache()

    extra = {}
    if not args.no_autograd:
        # The reference's benchmark path: CudaFlashAttention.apply, then o.backward(dO)
        # (benchmark/cuda_bench.py:44-48), through the torch operator layer and autograd.
        from cuda_autograd_fns import CudaFlashAttention

        qg, kg, vg = (t.clone().requires_grad_() for t in (q, k, v))
        for _ in range(2):
            o, _l = CudaFlashAttention.apply(qg, kg, vg, causal)
            o.backward(do)
        torch.cuda.synchronize()
        reps = max(3, args.steps // 2)
        ta = time.perf_counter()
        for _ in range(reps):
            o, _l = CudaFlashAttention.apply(qg, kg, vg, causal)
            o.backward(do)
        torch.cuda.synchronize()
        extra["autograd_ms_per_step"] = round((time.perf_counter() - ta) * 1e3 / reps, 4)

    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_steps_run": warm,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (N(0,1) Q/K/V/dO from fixed seeds)",
        "config": {"workload": f"FA2 fwd+bwd B{B} H{H} N{N} D{D} {'causal' if causal else 'non-causal'}",
                   "B": B, "H": H, "N": N, "D": D, "causal": causal,
                   "bwd_schedule": args.bwd_schedule},
        "fwd_tflops": round(fwd_tf, 3),
        "bwd_tflops": round(bwd_tf, 3),
        "fwd_frac_of_peak": round(fwd_tf / MFMA_FP32_PEAK_TFLOPS, 4),
        "bwd_frac_of_peak": round(bwd_tf / MFMA_FP32_PEAK_TFLOPS, 4),
        "per_kernel_ms": {k_: round(v_, 4) for k_, v_ in per_kernel.items()},
        "per_kernel_ms_flushed": {k_: round(v_, 4) for k_, v_ in flushed.items()},
        "roofline": roofline,
        "ds_workspace_bytes": ds_ws,
        "recompute": recompute,
        "reference_rtx5070_ms": REFERENCE_RTX5070_MS,
        "device": torch.cuda.get_device_name(0),
        "host": host_info(),
        "torch": torch.__version__,
        **extra,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_reference_path(B, H, N, D, causal)
        if args.cpu_port:
            line["cpu_baseline_port"] = cpu_port_baseline(B, H, N, D, causal, args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

#!/usr/bin/env python3
"""Headline benchmark: causal attention fwd+bwd TFLOP/s on one MI355X.

One step = one forward + backward of the attention op (the public autograd op
``flash_cuda.attn`` -- what nanolab's mixer calls) over one batch of the
BASELINE headline configuration (causal B16 H12 S1024 D64 bf16, seeded
synthetic inputs already resident in HBM). ``value`` is the algorithmic
14*B*H*D*N_vis FLOPs per step divided by the measured step time.

Also reported on the same JSON line:
  * ``roofline``: the dominant kernel (largest average launch time), its
    algorithmic FLOPs per launch over its average duration, measured here with
    HIP events bracketing back-to-back launches on the stream it runs on;
  * ``cpu_baseline``: the reference's CPU attention path (transpose +
    repeat_interleave + SDPA, fp32 -- oracle/cpu_path.py) timed on this host's
    cores on a bounded sample (a batch slice) of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--config board]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import torch

from machinelearning_amd import _capi, perf
from machinelearning_amd import flash_cuda as fc
from machinelearning_amd.inputs import CONFIGS, make_inputs

DT_NAME = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}
ELEM = {torch.bfloat16: 2, torch.float16: 2, torch.float32: 4}


def _events_ms(fn, n: int) -> float:
    """Average ms per call of ``fn`` over n back-to-back calls, bracketed by HIP events."""
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(n):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / n


def kernel_times(cfg, q, k, v, do, n: int = 20) -> dict:
    """Average duration of each kernel of the path, one C-ABI launch at a time."""
    lib = _capi.load()
    B, S, H, D = q.shape
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[q.dtype]
    shp = _capi.shape(B, S, H, k.shape[2], D, cfg.causal, cfg.window, cfg.scale, code,
                      cfg.sinks, cfg.block)
    sp = ctypes.byref(shp)
    st = torch.cuda.current_stream().cuda_stream
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=q.device, dtype=torch.float32)
    delta = lse.new_empty(_capi.workspace_floats(shp))
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    calls = {
        "attn_fwd": lambda: lib.mi_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                            o.data_ptr(), lse.data_ptr(), sp, st),
        "attn_bwd_delta": lambda: lib.mi_attn_bwd_delta(o.data_ptr(), do.data_ptr(), lse.data_ptr(),
                                                        None, delta.data_ptr(), sp, st),
        "attn_bwd_dkdv": lambda: lib.mi_attn_bwd_dkdv(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                      do.data_ptr(), lse.data_ptr(),
                                                      delta.data_ptr(), dk.data_ptr(),
                                                      dv.data_ptr(), sp, st),
        "attn_bwd_dq": lambda: lib.mi_attn_bwd_dq(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                  do.data_ptr(), lse.data_ptr(),
                                                  delta.data_ptr(), dq.data_ptr(), sp, st),
    }
    out = {}
    for name, fn in calls.items():          # order matters: each stage feeds the next
        _capi.check(fn())
        for _ in range(3):
            fn()
        out[name] = _events_ms(fn, n)
    return out


def profile_kernels(cfg, iters: int) -> None:
    """Launch every kernel of the path `iters` times, then one plain copy.

    For rocprofv3: the kernel-trace summary gives each kernel's average
    duration, and FETCH_SIZE / WRITE_SIZE of the copy (256 MiB read, 256 MiB
    written) calibrate the same counters read on the attention kernels.
    """
    q, k, v, do = make_inputs(cfg, "cuda")
    with torch.no_grad():
        kernel_times(cfg, q, k, v, do, iters)
        src = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profiled {cfg.name}: {iters} launches per kernel + one 256 MiB copy", flush=True)


def load_traffic(cfg, kernel: str):
    """HBM bytes per launch of `kernel` measured by rocprofv3 (profiles/), or None.

    profiles/traffic_<config>.txt holds 'kernel: bytes' lines written from two
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) scaled by the copy
    calibration; the derivation is recorded in the same file.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        f"traffic_{cfg.name}.txt")
    try:
        with open(path) as f:
            for line in f:
                name, _, val = line.partition(":")
                if name.strip() == kernel:
                    return float(val.split()[0])
    except (OSError, ValueError, IndexError):
        return None
    return None


def cpu_baseline(cfg, seconds: float = 10.0) -> dict:
    """The reference's CPU attention path, fp32, on a batch slice of the workload."""
    from oracle.cpu_path import cpu_attention

    torch.set_num_threads(max(1, torch.get_num_threads()))
    cores = torch.get_num_threads()
    Bs = 1
    q, k, v, do = (t.float() for t in make_inputs(cfg, "cpu", B=Bs))
    q.requires_grad_()
    k.requires_grad_()
    v.requires_grad_()

    def step():
        y = cpu_attention(q, k, v, cfg.scale, cfg.causal, cfg.window, cfg.sinks, cfg.block)
        torch.autograd.grad(y, (q, k, v), do)

    step()                                   # warmup
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 50):
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    fl = perf.flops(Bs, cfg.H, cfg.S, cfg.D, cfg.causal, cfg.window, sinks=cfg.sinks,
                    block=cfg.block)
    return {"value": round(fl / med / 1e12, 5), "unit": "TFLOP/s", "cores": cores,
            "kind": "port",
            "sample": (f"fwd+bwd of batch slice B={Bs} of the {cfg.name} workload "
                       f"(H{cfg.H} S{cfg.S} D{cfg.D}, fp32 SDPA path), median of "
                       f"{len(times)} iterations, {med * 1e3:.1f} ms each")}


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=200,
                   help="untimed steps first; ~200 bring the GPU to its steady clock")
    p.add_argument("--config", default="board", choices=sorted(CONFIGS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--kernel-iters", type=int, default=20)
    p.add_argument("--mode", default="bench", choices=("bench", "kernels"),
                   help="kernels: only launch each kernel --kernel-iters times (for rocprofv3)")
    args = p.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the op shards over (batch, head) with no exchange; see DESIGN.md). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    if not fc.is_available():
        print(f"library unavailable: {fc.unavailable_reason()}", file=sys.stderr)
        return 1

    cfg = CONFIGS[args.config]
    if args.mode == "kernels":
        profile_kernels(cfg, args.kernel_iters)
        return 0
    q, k, v, do = make_inputs(cfg, "cuda")
    q.requires_grad_()
    k.requires_grad_()
    v.requires_grad_()

    def step():
        o, _ = fc.attn(q, k, v, cfg.causal, cfg.window, cfg.scale, sinks=cfg.sinks,
                       block=cfg.block)
        torch.autograd.grad(o, (q, k, v), do)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        step()
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    total_flops = perf.flops(cfg.B, cfg.H, cfg.S, cfg.D, cfg.causal, cfg.window,
                             sinks=cfg.sinks, block=cfg.block)
    tflops = total_flops / (ms * 1e-3) / 1e12
    dtn = DT_NAME[cfg.dtype]
    peak = perf.PEAK_TFLOPS[dtn]

    with torch.no_grad():
        kt = kernel_times(cfg, q.detach(), k.detach(), v.detach(), do, args.kernel_iters)
    mfma = {n: t for n, t in kt.items() if n in perf.KERNEL_FLOPS_PER_PAIR_D}
    dom = max(mfma, key=mfma.get)
    kfl = perf.kernel_flops(dom, cfg.B, cfg.H, cfg.S, cfg.D, cfg.causal, cfg.window,
                            cfg.sinks, cfg.block)
    achieved = kfl / (kt[dom] * 1e-3) / 1e12
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2), "peak": peak,
                "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                "traffic": load_traffic(cfg, dom),
                "avg_launch_ms": round(kt[dom], 5),
                "kernels_ms": {n: round(t, 5) for n, t in kt.items()}}

    cpu = None if args.no_cpu_baseline else cpu_baseline(cfg, args.cpu_seconds)

    line = {
        "metric": "attn fwd+bwd TFLOP/s & % bf16 MFMA peak (causal B16 H12 S1024 D64)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "frac_of_peak": round(tflops / peak, 4),
        "dtype": dtn,
        "data": "synthetic (seeded N(0,1) q/k/v, dO~N(0,1e-2) for the headline)",
        "config": {"workload": cfg.name, **cfg.describe(),
                   "flops_per_step": total_flops},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

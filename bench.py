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
       python bench.py --mode decode|prologue|gate   (the widened rows' measurements)
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
    # The launches the autograd step makes: with the output residual where the op
    # keeps it (16-bit, D = 128).
    o_res = torch.empty_like(q) if fc._wants_residual(q, cfg.sinks, None, cfg.window) else None
    if o_res is None:
        fwd = lambda: lib.mi_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                      lse.data_ptr(), sp, st)
    else:
        fwd = lambda: lib.mi_attn_fwd_res(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                          o_res.data_ptr(), lse.data_ptr(), sp, st)
    calls = {
        "attn_fwd": fwd,
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
    # The whole backward as one call, as the autograd op runs it (16-bit: the
    # delta pass fused into dQ, then dK/dV).
    if o_res is None:
        calls["attn_bwd_call"] = lambda: lib.mi_attn_bwd(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), do.data_ptr(), lse.data_ptr(),
            None, delta.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), sp, st)
    else:
        calls["attn_bwd_call"] = lambda: lib.mi_attn_bwd_res(
            q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), o_res.data_ptr(),
            do.data_ptr(), lse.data_ptr(), None, delta.data_ptr(), dq.data_ptr(), dk.data_ptr(),
            dv.data_ptr(), sp, st)
    out = {}
    for name, fn in calls.items():          # order matters: each stage feeds the next
        _capi.check(fn())
        for _ in range(3):
            fn()
        out[name] = _events_ms(fn, n)
    return out


def step_kernel_times(cfg, q, k, v, do, n: int = 20) -> dict:
    """Kernel durations inside the step's own launch order, HIP events between launches.

    Each of n iterations enqueues, on one stream: the forward and the whole backward
    as the autograd op calls them (mi_attn_fwd / _res, then mi_attn_bwd / _res: at 16
    bits dQ with the delta pass fused in, then dK/dV), then the stages dK/dV and dQ
    once more on the planes that backward wrote. An event is recorded before and
    after every launch, so each duration is that kernel's own time in the step's
    cache and clock state (the per-launch averages; the sum of the first two is
    the step's GPU time without the host's autograd gap). Returns ms per launch:
    attn_fwd, attn_bwd_call (dQ + delta and dK/dV), attn_bwd_dkdv, attn_bwd_dq
    (the stage without the fused delta pass) and attn_bwd_dq+delta (the call minus
    dK/dV).
    """
    lib = _capi.load()
    B, S, H, D = q.shape
    code = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}[q.dtype]
    shp = _capi.shape(B, S, H, k.shape[2], D, cfg.causal, cfg.window, cfg.scale, code,
                      cfg.sinks, cfg.block)
    sp = ctypes.byref(shp)
    st = torch.cuda.current_stream().cuda_stream
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=q.device, dtype=torch.float32)
    ws = lse.new_empty(_capi.workspace_floats(shp))
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    o_res = torch.empty_like(q) if fc._wants_residual(q, cfg.sinks, None, cfg.window) else None
    P = lambda t: t.data_ptr()
    if o_res is None:
        fwd = lambda: lib.mi_attn_fwd(P(q), P(k), P(v), P(o), P(lse), sp, st)
        bwd = lambda: lib.mi_attn_bwd(P(q), P(k), P(v), P(o), P(do), P(lse), None, P(ws), P(dq),
                                      P(dk), P(dv), sp, st)
    else:
        fwd = lambda: lib.mi_attn_fwd_res(P(q), P(k), P(v), P(o), P(o_res), P(lse), sp, st)
        bwd = lambda: lib.mi_attn_bwd_res(P(q), P(k), P(v), P(o), P(o_res), P(do), P(lse), None,
                                          P(ws), P(dq), P(dk), P(dv), sp, st)
    seq = (("attn_fwd", fwd), ("attn_bwd_call", bwd),
           ("attn_bwd_dkdv", lambda: lib.mi_attn_bwd_dkdv(P(q), P(k), P(v), P(do), P(lse), P(ws),
                                                          P(dk), P(dv), sp, st)),
           ("attn_bwd_dq", lambda: lib.mi_attn_bwd_dq(P(q), P(k), P(v), P(do), P(lse), P(ws),
                                                      P(dq), sp, st)))
    for _, fn in seq:                       # order matters: each stage feeds the next
        _capi.check(fn())
    torch.cuda.synchronize()
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in seq] for _ in range(n + 3)]
    for it in range(n + 3):                 # 3 untimed iterations first
        for (name, fn), (e0, e1) in zip(seq, ev[it]):
            e0.record()
            fn()
            e1.record()
    torch.cuda.synchronize()
    out = {name: sum(ev[it][j][0].elapsed_time(ev[it][j][1]) for it in range(3, n + 3)) / n
           for j, (name, _) in enumerate(seq)}
    out["attn_bwd_dq+delta"] = out["attn_bwd_call"] - out["attn_bwd_dkdv"]
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
    """(HBM bytes per launch of `kernel`, source) measured by rocprofv3, or (None, None).

    profiles/traffic_<config>.txt holds 'kernel: bytes' lines written from two
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) scaled by the copy
    calibration; the derivation and the build it was measured on ('# build:'
    line) are recorded in the same file. The figure is read from that file, not
    measured in this run.
    """
    rel = os.path.join("profiles", f"traffic_{cfg.name}.txt")
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), rel)
    val, build = None, None
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("# build:"):
                    build = line.split(":", 1)[1].strip()
                    continue
                name, _, rest = line.partition(":")
                if name.strip() == kernel and val is None:
                    val = float(rest.split()[0])
    except (OSError, ValueError, IndexError):
        return None, None
    if val is None:
        return None, None
    return val, {"file": rel, "build": build, "measured_in_this_run": False}


def host_info() -> dict:
    """The host's CPU model and the CPUs this process may run on."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    quota = None
    try:   # cgroup v2 CPU quota ("max" or "<quota> <period>")
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, per = f.read().split()
            if q != "max":
                quota = round(int(q) / int(per), 2)
    except (OSError, ValueError):
        pass
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cpus": affinity,
            "cgroup_cpu_quota": quota}


def cpu_baseline(cfg, seconds: float = 10.0) -> dict:
    """The reference's CPU attention path, fp32, on a batch slice of the workload.

    Threads: every CPU this process may run on (its affinity mask), capped by a
    cgroup CPU quota when one is set (threads beyond the quota only time-slice).
    """
    from oracle.cpu_path import cpu_attention

    host = host_info()
    threads = host["affinity_cpus"]
    if host["cgroup_cpu_quota"]:
        threads = max(1, min(threads, int(host["cgroup_cpu_quota"])))
    torch.set_num_threads(threads)
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
    while len(times) < 3 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    fl = perf.flops(Bs, cfg.H, cfg.S, cfg.D, cfg.causal, cfg.window, sinks=cfg.sinks,
                    block=cfg.block)
    return {"value": round(fl / med / 1e12, 5), "unit": "TFLOP/s", "cores": cores,
            "threads": cores, **host,
            "kind": "port",
            "sample": (f"fwd+bwd of batch slice B={Bs} of the {cfg.name} workload "
                       f"(H{cfg.H} S{cfg.S} D{cfg.D}, fp32 SDPA path), median of "
                       f"{len(times)} iterations, {med * 1e3:.1f} ms each")}


def sdpa_same_gpu(n: int, cfg, ms_step: float) -> dict:
    """torch SDPA on this GPU, as context (never the target): what nanolab runs
    without the kernel (``flash_cuda.sdpa_reference``: transpose, repeat_interleave
    for GQA, SDPA with is_causal), forward and forward + backward, timed with HIP
    events over n back-to-back calls like the step, at the headline config and at
    the reference's E17 GQA shape (B8 H12/Hkv4 S1024 D32 bf16,
    ``nanolab/flash_cuda.py:319-378``), beside this build's step on the same
    inputs. ``speedup`` is SDPA's fwd+bwd time over this build's."""
    out = {}
    for name in dict.fromkeys((cfg.name, "gqa")):
        c = CONFIGS[name]
        if c.window or c.sinks or c.block:
            continue
        q, k, v, do = make_inputs(c, "cuda")
        xs = [t.detach().requires_grad_() for t in (q, k, v)]

        def sd_fwd():
            return fc.sdpa_reference(*xs, c.scale, c.causal)

        def sd_step():
            torch.autograd.grad(sd_fwd(), xs, do)
        with torch.no_grad():
            t_fwd = _best_us(sd_fwd, n) / 1e3
        t_all = _best_us(sd_step, n) / 1e3
        step = _Step(c)
        ours = ms_step if name == cfg.name else _best_us(step, n, warm=30) / 1e3
        ours_fwd = _best_us(step.forward, n) / 1e3
        fl = perf.flops(c.B, c.H, c.S, c.D, c.causal, c.window)
        out[name] = {
            "config": c.describe(), "backend": fc.sdpa_backend(q, k, v, c.scale, c.causal),
            "sdpa_fwd_ms": round(t_fwd, 5), "sdpa_fwd_bwd_ms": round(t_all, 5),
            "sdpa_fwd_bwd_tflops": round(fl / (t_all * 1e-3) / 1e12, 1),
            "ours_fwd_ms": round(ours_fwd, 5), "ours_fwd_bwd_ms": round(ours, 5),
            "speedup_fwd": round(t_fwd / ours_fwd, 2), "speedup": round(t_all / ours, 2)}
        del q, k, v, do, xs, step
    return out


def _best_us(fn, n: int, reps: int = 3, warm: int = 10) -> float:
    """Minimum over `reps` of the average us per call of n back-to-back calls."""
    for _ in range(warm):
        fn()
    return min(_events_ms(fn, n) for _ in range(reps)) * 1e3


# KV-cached decode workloads (bf16): name -> (B, T, H, Hkv, D, cached, causal).
# One step = one attention step of nanolab's Attention.forward_cached
# (nanolab/mixers.py:372-467) for T active queries against `cached` committed
# keys: one-token decoding at the board model's shape, long caches, a
# block-diffusion draft (bidirectional block of 32) and a self-speculation
# verify (causal block of 32) with GQA.
DECODE_CASES = {
    "decode_board": (16, 1, 12, 12, 64, 1024, True),
    "decode_long": (16, 1, 12, 12, 64, 8192, True),
    "decode_b1_32k": (1, 1, 12, 12, 64, 32768, True),
    "decode_gqa_d128": (8, 1, 32, 8, 128, 8192, True),
    "draft_block32": (16, 32, 12, 12, 64, 1024, False),
    "verify_block32_gqa": (8, 32, 32, 8, 128, 4096, True),
}


def _torch_cached_step(q, k, v, ck, cv, causal, scale):
    """The reference's step on the GPU: cat + repeat_interleave + masked SDPA (mixers.py:401-458)."""
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    kf = torch.cat([ck, k.transpose(1, 2)], 2)
    vf = torch.cat([cv, v.transpose(1, 2)], 2)
    mask = None
    if causal:
        Lk = kf.shape[2]
        mask = torch.cat([torch.ones(T, Lk - T, dtype=torch.bool, device=q.device),
                          torch.tril(torch.ones(T, T, dtype=torch.bool, device=q.device))],
                         1)[None, None]
    if Hkv != H:
        kf = kf.repeat_interleave(H // Hkv, 1)
        vf = vf.repeat_interleave(H // Hkv, 1)
    y = torch.nn.functional.scaled_dot_product_attention(q.transpose(1, 2), kf, vf,
                                                         attn_mask=mask, scale=scale)
    return y.transpose(1, 2)


def bench_decode(iters: int, cases=None) -> None:
    """One JSON line per decode workload: the step through the C ABI (kernel time incl.
    the split merge), the public ``attn_cached`` call, and the reference's torch step."""
    from machinelearning_amd.decode import attn_cached
    lib = _capi.load()
    gen = torch.Generator(device="cuda").manual_seed(0)
    for name, (B, T, H, Hkv, D, Lc, causal) in DECODE_CASES.items():
        if cases and name not in cases:
            continue
        dt = torch.bfloat16

        def rnd(*shape):
            return torch.randn(*shape, device="cuda", generator=gen).to(dt)
        q, k, v = rnd(B, T, H, D), rnd(B, T, Hkv, D), rnd(B, T, Hkv, D)
        ck, cv = rnd(B, Hkv, Lc, D), rnd(B, Hkv, Lc, D)
        out = torch.empty_like(q)
        lse = torch.empty(B, H, T, device="cuda", dtype=torch.float32)
        scale = D ** -0.5
        shp = _capi.MiDecodeShape(B, T, H, Hkv, D, Lc, Lc, int(causal), 0, 0, scale,
                                  _capi.MI_BF16, ck.stride(0), ck.stride(1), cv.stride(0),
                                  cv.stride(1))
        nws = _capi.decode_workspace_floats(shp)
        ws = torch.empty(max(nws, 1), device="cuda", dtype=torch.float32)
        st = torch.cuda.current_stream().cuda_stream

        def step():
            return lib.mi_attn_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), ck.data_ptr(),
                                      cv.data_ptr(), None, None, out.data_ptr(), lse.data_ptr(),
                                      ws.data_ptr(), ctypes.byref(shp), st)
        _capi.check(step())
        cache = {"k": ck, "v": cv}
        with torch.no_grad():
            us = _best_us(step, iters)
            api_us = _best_us(lambda: attn_cached(q, k, v, cache, False, causal), iters)
            ref_us = _best_us(lambda: _torch_cached_step(q, k, v, ck, cv, causal, scale), iters)
            ref = _torch_cached_step(q, k, v, ck, cv, causal, scale)
            err = float((out.float() - ref.float()).abs().max())
        nbytes = 2 * B * Hkv * (Lc + T) * D * 2 + 2 * B * T * H * D * 2 + B * H * T * 4
        gbps = nbytes / (us * 1e-6) / 1e9
        print(json.dumps({
            "mode": "decode", "case": name, "dtype": "bf16",
            "config": {"B": B, "T": T, "H": H, "Hkv": Hkv, "D": D, "cached": Lc,
                       "causal": causal, "splits_workspace_floats": nws},
            "us_per_step": round(us, 2), "api_us_per_step": round(api_us, 2),
            "torch_ref_us_per_step": round(ref_us, 2), "speedup_vs_torch": round(ref_us / us, 2),
            "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": 8000.0,
                         "unit": "GB/s", "frac": round(gbps / 8000.0, 4),
                         "algorithmic_bytes": nbytes},
            "max_abs_diff_vs_torch": err}), flush=True)


def bench_prologue(iters: int) -> None:
    """Fused QK-norm + RoPE (qk_norm_rope) vs the reference's torch chain, board-shape q."""
    import torch.nn.functional as F
    from machinelearning_amd.prologue import qk_norm_rope
    B, T, H, D = 16, 1024, 12, 64
    gen = torch.Generator(device="cuda").manual_seed(0)
    x16 = torch.randn(B, T, H, D, device="cuda", generator=gen).to(torch.bfloat16)
    gr = torch.randn(B, T, H, D, device="cuda", generator=gen).to(torch.bfloat16)
    w = torch.ones(D, device="cuda").requires_grad_()
    inv = 10000.0 ** (-torch.arange(0, D, 2, device="cuda", dtype=torch.float32) / D)
    ang = torch.arange(T, device="cuda", dtype=torch.float32)[:, None] * inv[None, :]
    c, s = torch.cat([ang.cos(), ang.cos()], -1), torch.cat([ang.sin(), ang.sin()], -1)

    def fused_fwd():
        with torch.no_grad():
            qk_norm_rope(x16, w, c, s, 1e-6, torch.bfloat16)

    def fused():
        xg = x16.detach().requires_grad_()
        torch.autograd.grad(qk_norm_rope(xg, w, c, s, 1e-6, torch.bfloat16), (xg, w), gr)

    def chain(x):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            y = F.rms_norm(x, (D,), w, 1e-6)
            x1, x2 = y[..., : D // 2], y[..., D // 2:]
            return (y * c[None, :, None, :] + torch.cat((-x2, x1), -1) * s[None, :, None, :]
                    ).to(torch.bfloat16)

    def ref_fwd():
        with torch.no_grad():
            chain(x16)

    def ref():
        xg = x16.detach().requires_grad_()
        torch.autograd.grad(chain(xg), (xg, w), gr)
    res = {n: round(_best_us(f, iters), 2) for n, f in (
        ("fused_fwd_us", fused_fwd), ("fused_fwd_bwd_us", fused), ("torch_fwd_us", ref_fwd),
        ("torch_fwd_bwd_us", ref))}
    print(json.dumps({"mode": "prologue", "config": {"B": B, "T": T, "H": H, "D": D,
                                                     "dtype": "bf16"}, **res}), flush=True)


def bench_gate(cfg, iters: int) -> None:
    """fwd+bwd step: ungated, the gate fused in the kernels, and ungated + the torch gate."""
    q, k, v, do = make_inputs(cfg, "cuda")
    q.requires_grad_()
    k.requires_grad_()
    v.requires_grad_()
    z = torch.randn(cfg.B, cfg.S, cfg.H, device="cuda", requires_grad=True)

    def plain():
        o, _ = fc.attn(q, k, v, cfg.causal, cfg.window, cfg.scale)
        torch.autograd.grad(o, (q, k, v), do)

    def fused():
        y, _ = fc.attn(q, k, v, cfg.causal, cfg.window, cfg.scale, gate=z)
        torch.autograd.grad(y, (q, k, v, z), do)

    def torch_gate():
        o, _ = fc.attn(q, k, v, cfg.causal, cfg.window, cfg.scale)
        y = o * torch.sigmoid(z).unsqueeze(-1).to(o.dtype)
        torch.autograd.grad(y, (q, k, v, z), do)
    res = {n: round(_best_us(f, iters, warm=30), 2) for n, f in (
        ("ungated_us", plain), ("fused_gate_us", fused), ("torch_gate_us", torch_gate))}
    print(json.dumps({"mode": "gate", "config": {"workload": cfg.name}, **res}), flush=True)


class _Step:
    """One fwd+bwd step of the public autograd op on fixed, HBM-resident inputs."""

    def __init__(self, cfg):
        self.cfg = cfg
        q, k, v, do = make_inputs(cfg, "cuda")
        self.inputs = (q.requires_grad_(), k.requires_grad_(), v.requires_grad_(), do)

    def __call__(self):
        cfg = self.cfg
        q, k, v, do = self.inputs
        o, _ = fc.attn(q, k, v, cfg.causal, cfg.window, cfg.scale, sinks=cfg.sinks,
                       block=cfg.block)
        torch.autograd.grad(o, (q, k, v), do)

    def forward(self):
        cfg = self.cfg
        q, k, v, _ = self.inputs
        with torch.no_grad():
            fc.attn(q, k, v, cfg.causal, cfg.window, cfg.scale, sinks=cfg.sinks, block=cfg.block)


def time_steps(cfg, steps: int, warmup: int, settle_s: float):
    """(ms per step, settle steps, the step) over exactly `steps` timed steps.

    Before the `warmup` untimed steps, steps run for `settle_s` seconds of wall
    time (synchronised every 10 steps): an idle MI355X needs some tens of ms of
    sustained work to reach its steady clock, and a short warmup alone measured
    the same kernels ~8% slower. The timed region is bracketed by
    torch.cuda.synchronize() and HIP events on the current stream.
    """
    step = _Step(cfg)
    settle_steps = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < settle_s:
        for _ in range(10):
            step()
        torch.cuda.synchronize()
        settle_steps += 10
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        step()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, settle_steps, step


# Row-length study at the board's heads and head dim: (B, S) with the board's
# visible-pair count at S = 1024, 2048 and 4096, and S = 2048 at twice the pairs.
LENGTH_CASES = ((16, 1024), (4, 2048), (1, 4096), (8, 2048))


def bench_lengths(kernel_iters: int, settle_s: float) -> None:
    """One JSON line per (B, S): the forward and the whole backward (C-ABI launches,
    HIP events, best of 3) and their cost per visible pair. At a fixed pair count the
    per-pair cost falls as rows get longer: the per-workgroup and per-wave fixed costs
    (prologue, diagonal tile, epilogue) are spread over more key / query tiles."""
    import dataclasses
    base = CONFIGS["board"]
    for i, (B, S) in enumerate(LENGTH_CASES):
        cfg = dataclasses.replace(base, name=f"board_B{B}_S{S}", B=B, S=S)
        q, k, v, do = make_inputs(cfg, "cuda")
        with torch.no_grad():
            if i == 0:                        # reach the steady clock first
                t_end = time.perf_counter() + settle_s
                while time.perf_counter() < t_end:
                    kernel_times(cfg, q, k, v, do, 20)
            kt = [kernel_times(cfg, q, k, v, do, kernel_iters) for _ in range(3)]
        fwd = min(t["attn_fwd"] for t in kt)
        bwd = min(t["attn_bwd_call"] for t in kt)
        pairs = perf.nvis(S, True) * B * cfg.H
        print(json.dumps({"mode": "lengths", "B": B, "S": S, "H": cfg.H, "D": cfg.D,
                          "visible_pairs": pairs, "fwd_ms": round(fwd, 5), "bwd_ms": round(bwd, 5),
                          "fwd_ps_per_pair": round(fwd * 1e9 / pairs, 3),
                          "bwd_ps_per_pair": round(bwd * 1e9 / pairs, 3)}), flush=True)


def bench_configs(names, steps: int, warmup: int, settle_s: float, kernel_iters: int) -> None:
    """One JSON line per workload: the fwd+bwd step, the forward alone, each kernel."""
    for name in names:
        cfg = CONFIGS[name]
        ms, settle_steps, step = time_steps(cfg, steps, warmup, settle_s)
        fwd_ms = _best_us(step.forward, steps) / 1e3
        q, k, v, do = step.inputs
        with torch.no_grad():
            kt = kernel_times(cfg, q.detach(), k.detach(), v.detach(), do, kernel_iters)
        fl = perf.flops(cfg.B, cfg.H, cfg.S, cfg.D, cfg.causal, cfg.window, sinks=cfg.sinks,
                        block=cfg.block)
        fl_fwd = perf.flops(cfg.B, cfg.H, cfg.S, cfg.D, cfg.causal, cfg.window, bwd=False,
                            sinks=cfg.sinks, block=cfg.block)
        peak = perf.PEAK_TFLOPS[DT_NAME[cfg.dtype]]
        kern = {}
        for kname, t in kt.items():
            entry = {"ms": round(t, 5)}
            if kname in perf.KERNEL_FLOPS_PER_PAIR_D:
                tf = perf.kernel_flops(kname, cfg.B, cfg.H, cfg.S, cfg.D, cfg.causal,
                                       cfg.window, cfg.sinks, cfg.block) / (t * 1e-3) / 1e12
                entry.update(tflops=round(tf, 1), frac=round(tf / peak, 4))
            kern[kname] = entry
        nbytes = perf.compulsory_bytes(cfg.B, cfg.S, cfg.H, cfg.D, ELEM[cfg.dtype])
        print(json.dumps({
            "mode": "configs", "workload": name, "config": cfg.describe(),
            "ms_per_step": round(ms, 5), "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
            "frac_of_peak": round(fl / (ms * 1e-3) / 1e12 / peak, 4),
            "fwd_ms": round(fwd_ms, 5), "fwd_tflops": round(fl_fwd / (fwd_ms * 1e-3) / 1e12, 1),
            "compulsory_bytes": nbytes,
            "hbm_frac_of_step": round(nbytes / (ms * 1e-3) / (perf.PEAK_HBM_GBS * 1e9), 4),
            "steps": steps, "warmup": warmup, "clock_settle_steps": settle_steps,
            "kernels": kern}), flush=True)


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=200,
                   help="untimed steps before the timed ones (after the clock settle)")
    p.add_argument("--settle", type=float, default=0.5,
                   help="seconds of untimed steps before the warmup, to reach the steady clock")
    p.add_argument("--config", default="board", choices=sorted(CONFIGS))
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-sdpa", action="store_true",
                   help="skip the torch SDPA timing on the same GPU (context only)")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--kernel-iters", type=int, default=20)
    p.add_argument("--mode", default="bench",
                   choices=("bench", "kernels", "configs", "decode", "prologue", "gate",
                            "lengths"),
                   help="kernels: only launch each kernel --kernel-iters times (for rocprofv3); "
                        "decode / prologue / gate: the KV-cached decode step, the fused q/k "
                        "prologue and the fused output gate, one JSON line per workload; "
                        "lengths: fwd / bwd cost per visible pair against the row length")
    p.add_argument("--cases", nargs="*", default=None,
                   help="decode workloads, or the configs of --mode configs (default all)")
    args = p.parse_args(argv)

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the op shards over (batch, head) with no exchange). "
              "Run with --gpus 1.", file=sys.stderr)
        return 2
    if not fc.is_available():
        print(f"library unavailable: {fc.unavailable_reason()}", file=sys.stderr)
        return 1

    cfg = CONFIGS[args.config]
    if args.mode == "kernels":
        profile_kernels(cfg, args.kernel_iters)
        return 0
    if args.mode == "configs":
        bench_configs(args.cases or [n for n in CONFIGS if n != "smoke"], args.steps,
                      args.warmup, args.settle, args.kernel_iters)
        return 0
    if args.mode == "decode":
        bench_decode(max(args.kernel_iters, 50), args.cases)
        return 0
    if args.mode == "lengths":
        bench_lengths(args.kernel_iters, args.settle)
        return 0
    if args.mode == "prologue":
        bench_prologue(max(args.kernel_iters, 50))
        return 0
    if args.mode == "gate":
        bench_gate(cfg, 100)
        return 0
    ms, settle_steps, step = time_steps(cfg, args.steps, args.warmup, args.settle)
    q, k, v, do = step.inputs
    total_flops = perf.flops(cfg.B, cfg.H, cfg.S, cfg.D, cfg.causal, cfg.window,
                             sinks=cfg.sinks, block=cfg.block)
    tflops = total_flops / (ms * 1e-3) / 1e12
    dtn = DT_NAME[cfg.dtype]
    peak = perf.PEAK_TFLOPS[dtn]

    with torch.no_grad():
        kt = step_kernel_times(cfg, q.detach(), k.detach(), v.detach(), do, args.kernel_iters)
    mfma = {n: t for n, t in kt.items() if n in perf.KERNEL_FLOPS_PER_PAIR_D}
    dom = max(mfma, key=mfma.get)
    kfl = perf.kernel_flops(dom, cfg.B, cfg.H, cfg.S, cfg.D, cfg.causal, cfg.window,
                            cfg.sinks, cfg.block)
    achieved = kfl / (kt[dom] * 1e-3) / 1e12
    traffic, traffic_src = load_traffic(cfg, dom)
    gpu_step = kt["attn_fwd"] + kt["attn_bwd_call"]
    roofline = {"bound": "mfma", "kernel": dom, "achieved": round(achieved, 2), "peak": peak,
                "unit": "TFLOP/s", "frac": round(achieved / peak, 4),
                "traffic": traffic, "traffic_source": traffic_src,
                "avg_launch_ms": round(kt[dom], 5),
                "kernels_ms": {n: round(t, 5) for n, t in kt.items()},
                # The step's kernels timed in the step's own launch order (fwd, then the
                # backward call), right after the timed steps: their sum against
                # ms_per_step, whose excess is the host's autograd hand-off between the
                # forward and the backward (negative: the clock or cache state moved).
                "step_kernel_sum_ms": round(gpu_step, 5),
                "step_minus_kernel_sum_ms": round(ms - gpu_step, 5)}

    cpu = None if args.no_cpu_baseline else cpu_baseline(cfg, args.cpu_seconds)
    sdpa = None if args.no_sdpa else sdpa_same_gpu(args.kernel_iters, cfg, ms)

    line = {
        "metric": "attn fwd+bwd TFLOP/s & % bf16 MFMA peak (causal B16 H12 S1024 D64)",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "clock_settle_steps": settle_steps,
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
        "sdpa_same_gpu": sdpa,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

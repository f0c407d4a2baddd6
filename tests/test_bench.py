"""bench.py's output contract: one JSON line with the metric, the one-GPU value, the
roofline of the dominant kernel and the configuration it was measured on.

The CPU test checks the refusal of more than one GPU (before anything touches a
device); the GPU test runs a short headline bench in a child process (no CPU baseline,
no SDPA leg) and checks every field a reader of the line relies on."""

from __future__ import annotations

import json
import math
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def _bench(*args, timeout=240):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], cwd=ROOT,
                          capture_output=True, text=True, timeout=timeout)


def test_more_than_one_gpu_is_refused():
    r = _bench("--gpus", "2", timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and "--gpus 1" in r.stderr
    assert r.stdout.strip() == ""


@pytest.mark.gpu
def test_headline_line_contract():
    r = _bench("--steps", "4", "--warmup", "2", "--settle", "0.1", "--no-cpu-baseline",
               "--no-sdpa")
    assert r.returncode == 0, r.stderr[-2000:]
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("{")]
    assert len(lines) == 1, r.stdout[-2000:]
    d = json.loads(lines[0])
    assert d["metric"].startswith("attn fwd+bwd TFLOP/s")
    assert d["unit"] == "TFLOP/s" and d["higher_is_better"] is True
    assert d["n_gpus"] == 1 and d["steps"] == 4 and d["warmup"] == 2
    assert d["scaling"] == "weak" and d["vs_baseline"] is None
    assert d["dtype"] == "bf16" and d["data"].startswith("synthetic")
    cfg = d["config"]
    assert cfg["workload"] == "board"
    assert (cfg["B"], cfg["S"], cfg["H"], cfg["D"]) == (16, 1024, 12, 64) and cfg["causal"]
    # value is the algorithmic FLOPs of one step over its time: 14 * D per visible pair.
    pairs = cfg["B"] * cfg["H"] * cfg["S"] * (cfg["S"] + 1) // 2
    assert cfg["flops_per_step"] == 14 * cfg["D"] * pairs
    tflops = cfg["flops_per_step"] / (d["ms_per_step"] * 1e-3) / 1e12
    assert math.isclose(d["value"], tflops, rel_tol=2e-3)
    assert math.isclose(d["frac_of_peak"], d["value"] / 2516.6, rel_tol=2e-3)
    roof = d["roofline"]
    assert roof["bound"] in ("mfma", "hbm") and roof["unit"] in ("TFLOP/s", "GB/s")
    assert math.isclose(roof["frac"], roof["achieved"] / roof["peak"], rel_tol=1e-3)
    assert roof["traffic"] is None or roof["traffic"] > 0
    assert "cpu_baseline" not in d or d["cpu_baseline"] is None

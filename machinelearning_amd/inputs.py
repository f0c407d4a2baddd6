"""Seeded synthetic inputs for the benchmark / parity configurations.

Recipe (identical bits on CPU and GPU): ``torch.manual_seed(seed)`` (0 by
default, as ``nanolab/tests.py:262`` and ``nanolab/flash_cuda.py:339``), draw
q, k, v, dO in that order on the CPU in float32, then cast to the config dtype
and move to the target device. Scale is 1/sqrt(D) everywhere.

Config-specific draws:
  * "board" (headline): dO ~ N(0, 1e-2) read as standard deviation 1e-2.
  * "long": q is drawn N(0,1) then multiplied by 2 (sharper softmax).
  * "recall": k[b,t,h] = proto[b,h,t mod 64] + 0.1 * N(0,1) with
    proto ~ N(0,1) of shape [B,H,64,D] (peaked, associative-recall-like scores).
"""

from __future__ import annotations

import dataclasses
import math

import torch


@dataclasses.dataclass(frozen=True)
class Config:
    name: str
    B: int
    S: int
    H: int
    Hkv: int
    D: int
    dtype: torch.dtype
    causal: bool = True
    window: int = 0
    sinks: int = 0
    block: int = 0
    q_mult: float = 1.0
    do_std: float = 1.0
    proto_keys: bool = False

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.D)

    def describe(self) -> dict:
        return {"B": self.B, "S": self.S, "H": self.H, "Hkv": self.Hkv, "D": self.D,
                "dtype": str(self.dtype).replace("torch.", ""), "causal": self.causal,
                "window": self.window, "sinks": self.sinks, "block": self.block}


CONFIGS = {
    # nanolab cpu_smoke-scale attention, fp32
    "smoke": Config("smoke", 4, 256, 4, 4, 64, torch.float32),
    # board-shape causal attention, the headline
    "board": Config("board", 16, 1024, 12, 12, 64, torch.bfloat16, do_std=1e-2),
    # sliding-window causal (SWA mixer, sinks=0)
    "swa": Config("swa", 8, 4096, 16, 16, 64, torch.bfloat16, window=256),
    # nanolab's default `swa` mixer, SWA(64, 4) (nanolab/config.py:133-134), at the
    # board shape: the sliding window plus StreamingLLM attention sinks
    "swa_sinks": Config("swa_sinks", 16, 1024, 12, 12, 64, torch.bfloat16, window=64, sinks=4),
    # wide-head long-context causal, Q scaled by 2
    "long": Config("long", 2, 8192, 16, 16, 128, torch.bfloat16, q_mult=2.0),
    # non-causal full attention with prototype (recall-like) keys
    "recall": Config("recall", 32, 2048, 8, 8, 64, torch.bfloat16, causal=False,
                     proto_keys=True),
    # Not a BASELINE config: the shape of the reference's only published
    # measurement of this path (E17, B8 T1024 H12 / Hkv4 D32 bf16, the defaults of
    # its self-check, nanolab/flash_cuda.py:319-327), which times the in-kernel
    # GQA group sum of dK/dV.
    "gqa": Config("gqa", 8, 1024, 12, 4, 32, torch.bfloat16),
}


def make_inputs(cfg: Config, device="cpu", seed: int = 0, B: int | None = None):
    """Return (q, k, v, do) for ``cfg``, drawn at batch size ``B`` (default cfg.B).

    Seeded and deterministic: the same (cfg, B, seed) always gives the same bits.
    """
    Bn = cfg.B if B is None else B
    g = torch.Generator(device="cpu").manual_seed(seed)
    q = torch.randn(Bn, cfg.S, cfg.H, cfg.D, generator=g) * cfg.q_mult
    if cfg.proto_keys:
        proto = torch.randn(Bn, cfg.Hkv, 64, cfg.D, generator=g)
        idx = torch.arange(cfg.S) % 64
        k = proto[:, :, idx, :].permute(0, 2, 1, 3) + 0.1 * torch.randn(
            Bn, cfg.S, cfg.Hkv, cfg.D, generator=g)
    else:
        k = torch.randn(Bn, cfg.S, cfg.Hkv, cfg.D, generator=g)
    v = torch.randn(Bn, cfg.S, cfg.Hkv, cfg.D, generator=g)
    do = torch.randn(Bn, cfg.S, cfg.H, cfg.D, generator=g) * cfg.do_std
    out = tuple(t.to(cfg.dtype).contiguous().to(device) for t in (q, k, v, do))
    return out

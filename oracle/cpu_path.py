"""The reference's CPU attention path, restated -- TEST INFRASTRUCTURE ONLY.

This is what nanolab runs for attention when it is not on CUDA, and what the
bench reports as ``cpu_baseline`` (kind "port"): it is timed, never shipped.

* ``cpu_attention`` follows ``nanolab/mixers.py:311-338``: transpose
  [B,T,H,D] -> [B,H,T,D], ``repeat_interleave`` the KV heads for GQA, then
  ``F.scaled_dot_product_attention`` (``is_causal`` for plain causal /
  non-causal). A sliding window goes through the exact chunked path when
  ``swa_auto_chunk`` says so (``mixers.py:322-335``), else a dense mask.
* ``swa_auto_chunk`` restates the chunking rule of ``mixers.py:138-165``
  (chunk when T >= 4*window, at max(256, window)).
* ``swa_chunked`` restates ``mixers.py:168-200`` with sinks=0: queries
  [s0, e0) only ever see keys [s0 - window + 1, e0), so the out-of-window
  scores are never formed.

The reference runs this path in float32 off-CUDA (``nanolab/utils.py:33-35``;
autocast is CUDA-only, ``nanolab/train.py:228-230``), so callers pass fp32.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def swa_auto_chunk(T: int, window: int) -> int:
    """Chunk size for the exact chunked window path, or 0 for the dense mask."""
    if window <= 0 or T <= 0:
        return 0
    if T < 4 * window:
        return 0
    return max(256, window)


def swa_chunked(q, k, v, window: int, scale: float, chunk: int) -> torch.Tensor:
    """Exact causal sliding-window attention on [B,H,T,D], chunk by chunk (sinks=0)."""
    B, H, T, D = q.shape
    out = q.new_empty(B, H, T, D)
    pos = torch.arange(T, device=q.device)
    for s0 in range(0, T, chunk):
        e0 = min(s0 + chunk, T)
        lo = max(0, s0 - window + 1)
        kpos = pos[lo:e0]
        qpos = pos[s0:e0]
        keep = (kpos[None, :] <= qpos[:, None]) & (kpos[None, :] > qpos[:, None] - window)
        out[:, :, s0:e0] = F.scaled_dot_product_attention(
            q[:, :, s0:e0], k[:, :, lo:e0], v[:, :, lo:e0], attn_mask=keep[None, None],
            scale=scale)
    return out


def cpu_attention(q, k, v, scale: float, causal: bool = True, window: int = 0) -> torch.Tensor:
    """[B,T,H,D] attention the way nanolab's mixer computes it without the kernel."""
    T = q.shape[1]
    qs, ks, vs = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if ks.shape[1] != qs.shape[1]:
        rep = qs.shape[1] // ks.shape[1]
        ks = ks.repeat_interleave(rep, dim=1)
        vs = vs.repeat_interleave(rep, dim=1)
    if window and window > 0:
        if not causal:
            raise ValueError("a sliding window is causal-only")
        chunk = swa_auto_chunk(T, window)
        if chunk:
            y = swa_chunked(qs, ks, vs, window, scale, chunk)
        else:
            i = torch.arange(T)
            keep = (i[None, :] <= i[:, None]) & (i[None, :] > i[:, None] - window)
            y = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=keep[None, None], scale=scale)
    else:
        y = F.scaled_dot_product_attention(qs, ks, vs, is_causal=causal, scale=scale)
    return y.transpose(1, 2).contiguous()

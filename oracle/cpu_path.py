"""The reference's CPU attention path, restated -- TEST INFRASTRUCTURE ONLY.

This is what nanolab runs for attention when it is not on CUDA, and what the
bench reports as ``cpu_baseline`` (kind "port"): it is timed, never shipped.

* ``cpu_attention`` follows ``nanolab/mixers.py:311-338``: transpose
  [B,T,H,D] -> [B,H,T,D], ``repeat_interleave`` the KV heads for GQA, then
  ``F.scaled_dot_product_attention`` (``is_causal`` for plain causal /
  non-causal; the block-causal mask of ``mixers.py:76-93`` as an explicit
  mask, ``mixers.py:318-320``). A sliding window goes through the exact chunked path when
  ``swa_auto_chunk`` says so (``mixers.py:322-335``), else a dense mask.
* ``swa_auto_chunk`` restates the chunking rule of ``mixers.py:138-165``
  (chunk when T >= 4*window, at max(256, window)).
* ``swa_chunked`` restates ``mixers.py:168-200``: queries [s0, e0) only
  ever see keys [s0 - (window - sinks) + 1, e0) plus the first ``sinks``
  keys, so the out-of-window scores are never formed.

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


def swa_chunked(q, k, v, window: int, scale: float, chunk: int, sinks: int = 0) -> torch.Tensor:
    """Exact causal SWA(window, sinks) attention on [B,H,T,D], chunk by chunk."""
    B, H, T, D = q.shape
    span = window - sinks
    out = q.new_empty(B, H, T, D)
    pos = torch.arange(T, device=q.device)
    for s0 in range(0, T, chunk):
        e0 = min(s0 + chunk, T)
        lo = max(0, s0 - span + 1)
        if lo <= sinks:                   # the sink keys and the span's keys touch
            kidx = pos[:e0]
        else:
            kidx = torch.cat([pos[:sinks], pos[lo:e0]])
        qpos = pos[s0:e0]
        keep = ((kidx[None, :] <= qpos[:, None])
                & ((kidx[None, :] > qpos[:, None] - span) | (kidx[None, :] < sinks)))
        out[:, :, s0:e0] = F.scaled_dot_product_attention(
            q[:, :, s0:e0], k[:, :, kidx], v[:, :, kidx], attn_mask=keep[None, None],
            scale=scale)
    return out


def dense_window_mask(T: int, window: int, sinks: int = 0) -> torch.Tensor:
    """[T, T] keep-mask of SWA(window, sinks) (mixers.py:117-131)."""
    i = torch.arange(T)
    causal = i[None, :] <= i[:, None]
    keep = causal & (i[None, :] > i[:, None] - (window - sinks))
    if sinks:
        keep = keep | (causal & (i[None, :] < sinks))
    return keep


def cpu_attention(q, k, v, scale: float, causal: bool = True, window: int = 0,
                  sinks: int = 0, block: int = 0) -> torch.Tensor:
    """[B,T,H,D] attention the way nanolab's mixer computes it without the kernel."""
    T = q.shape[1]
    qs, ks, vs = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if ks.shape[1] != qs.shape[1]:
        rep = qs.shape[1] // ks.shape[1]
        ks = ks.repeat_interleave(rep, dim=1)
        vs = vs.repeat_interleave(rep, dim=1)
    if block and block > 1:               # semi-AR: causal across blocks, dense within
        blk = torch.arange(T) // block
        keep = blk[:, None] >= blk[None, :]
        y = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=keep[None, None], scale=scale)
    elif window and window > 0:
        if not causal:
            raise ValueError("a sliding window is causal-only")
        chunk = swa_auto_chunk(T, window)
        if chunk:
            y = swa_chunked(qs, ks, vs, window, scale, chunk, sinks)
        else:
            keep = dense_window_mask(T, window, sinks)
            y = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=keep[None, None], scale=scale)
    else:
        y = F.scaled_dot_product_attention(qs, ks, vs, is_causal=causal, scale=scale)
    return y.transpose(1, 2).contiguous()

"""KV-cached attention for incremental decoding.

This is the attention section of nanolab's ``Attention.forward_cached``
(``nanolab/mixers.py:372-467``). It serves semi-autoregressive / block-diffusion
sampling and self-speculative decoding (``nanolab/diffusion.py:304-490``), and
the reasoning harness's cached decoder (``nanolab/reason.py:340-375``). Each
step attends a block of T new queries to every committed key plus the block's
own keys.

The reference keeps a per-layer cache dict. ``"k"`` / ``"v"`` hold the
committed keys / values as (B, Hkv, L, D); once a sliding window evicts rows,
``"pos"`` holds their absolute positions and ``"end"`` the next position. Each
step, the reference:

- concatenates the cache with the block's K / V (``torch.cat``,
  ``mixers.py:404-405``);
- builds the step's boolean mask (``mixers.py:407-433``);
- repeats K / V for GQA and runs SDPA (``mixers.py:452-458``);
- on ``commit``, stores the concatenation, or with a window only its live rows
  (``mixers.py:435-450``).

``attn_cached`` keeps that contract: the same dict, keys, shapes and error
behaviour, so callers and tests that read ``cache["k"].shape[2]`` see what they
saw before. The step itself runs through ``mi_attn_decode``
(``csrc/attn_decode.hip``). That kernel reads the cache and the block in place,
and the heads of a GQA group share one read of their kv head. Without a window,
the committed rows live in a capacity buffer, with ``cache["k"]`` a view of it.
A commit at the end of that view writes only the block's rows, instead of
copying the whole prefix every step.

Inference only: no gradient flows through the step. With autograd recording
and an input that requires grad, this raises rather than silently dropping
the gradient. There is no CPU fallback: without the library it raises
``RuntimeError``.
"""

from __future__ import annotations

import ctypes
import math

import torch

from . import _capi
from . import flash_cuda as _fc

# Private cache-dict entries: the capacity buffers behind cache["k"] /
# cache["v"], each stored as (buffer, [rows handed out]). The row count lives
# in a list shared by every shallow copy of the dict, so once one copy appends
# to the buffer, another copy still holding the old front sees the mismatch
# and reallocates instead of overwriting rows the first copy now exposes.
_KBUF, _VBUF = "_mi_kbuf", "_mi_vbuf"
_ROW_ALIGN = 64          # capacity granularity (rows)

# Split-partial workspaces, one per (device, stream), grown on demand, for
# the _WS_STREAMS most recently used streams. Steps of one stream run in
# order, so they can share one; this saves an allocation per step. Dropping a
# workspace is safe while a step still uses it: torch's caching allocator
# hands a freed block out again only to allocations on the stream it was
# allocated on (the step's own stream), which run after that step.
_WORKSPACES: dict = {}
_WS_MIN_FLOATS = 1 << 16
_WS_STREAMS = 8


# Shape structs and their workspace sizes by shape key: a sampler repeats
# each block's shape over its denoising steps (the library only reads the
# struct).
_SHAPES: dict = {}
_SHAPES_MAX = 4096


def _shape(key: tuple):
    hit = _SHAPES.get(key)
    if hit is None:
        shp = _capi.MiDecodeShape(*key)
        hit = (shp, _capi.decode_workspace_floats(shp))
        if len(_SHAPES) >= _SHAPES_MAX:
            _SHAPES.clear()
        _SHAPES[key] = hit
    return hit


def _dense(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    if t.dtype != dtype:
        t = t.to(dtype)
    return t if t.is_contiguous() else t.contiguous()


def _workspace(dev: torch.device, stream: int, floats: int) -> torch.Tensor:
    key = (dev.index, stream)
    ws = _WORKSPACES.pop(key, None)
    if ws is None or ws.numel() < floats:
        ws = torch.empty(max(floats, _WS_MIN_FLOATS), dtype=torch.float32, device=dev)
    _WORKSPACES[key] = ws                        # most recent last
    while len(_WORKSPACES) > _WS_STREAMS:
        del _WORKSPACES[next(iter(_WORKSPACES))]
    return ws


def _cache_tensor(t, B, Hkv, D, dtype, device, who, name):
    if t.dim() != 4 or t.shape[0] != B or t.shape[1] != Hkv or t.shape[3] != D:
        raise ValueError(f"{who}: cache[{name!r}] must be (B, Hkv, L, D) = ({B}, {Hkv}, L, {D}), "
                         f"got {tuple(t.shape)}")
    if t.dtype != dtype or t.device != device:
        t = t.to(device=device, dtype=dtype)
    # Rows D elements apart, batch / head strides in whole 16-byte chunks.
    chunk = 16 // t.element_size()
    if (t.stride(3) != 1 or t.stride(2) != D or t.stride(0) % chunk or t.stride(1) % chunk
            or t.data_ptr() % 16):
        t = t.contiguous()
    return t


def _commit_append(cache, key, bufkey, old, new_rows, Lc, T):
    """cache[key] <- cat(old, new_rows) along dim 2, appending in place when
    ``old`` is exactly the handed-out front of the capacity buffer."""
    B, Hkv, _, D = new_rows.shape
    held = cache.get(bufkey)
    buf, front = held if isinstance(held, tuple) else (None, None)
    in_place = (buf is not None and old is not None and front[0] == Lc
                and old.data_ptr() == buf.data_ptr() and old.stride() == buf.stride()
                and old.dtype == buf.dtype and old.device == buf.device
                and buf.shape[2] >= Lc + T)
    if not in_place:
        cap = max(_ROW_ALIGN, 2 * (Lc + T))
        cap = (cap + _ROW_ALIGN - 1) // _ROW_ALIGN * _ROW_ALIGN
        buf = torch.empty(B, Hkv, cap, D, dtype=new_rows.dtype, device=new_rows.device)
        front = [0]
        if Lc:
            buf[:, :, :Lc].copy_(old)
    buf[:, :, Lc:Lc + T].copy_(new_rows)
    front[0] = Lc + T
    cache[bufkey] = (buf, front)
    cache[key] = buf[:, :, :Lc + T]


def attn_cached(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cache: dict, commit: bool,
                causal: bool = False, *, window: int = 0, sinks: int = 0,
                scale: float | None = None, gate: torch.Tensor | None = None,
                return_lse: bool = False):
    """One cached attention step: (B, T, H, D) queries of the active block.

    ``k`` / ``v`` are the block's keys / values (B, T, Hkv, D), after RoPE and
    the value residual, as the mixer computes them (``mixers.py:387-400``). The
    queries attend to the whole cache and to the block: bidirectionally
    (``causal=False``, block diffusion) or lower-triangularly
    (``causal=True``). With ``window`` > 0 (causal only) and ``sinks``, the
    reference's sliding-window mask applies to absolute positions. ``gate``
    (B, T, H) applies the output gate ``sigmoid(gate)`` (``mixers.py:460-462``).

    ``commit=True`` stores the block into ``cache`` as the reference does.
    Without a window the cache grows by T rows. With one, only the sinks and
    the ``window - sinks - 1`` most recent positions stay. Returns the
    (B, T, H, D) output in the inputs' dtype, and the (B, H, T) float32 LSE too
    when ``return_lse``.
    """
    who = "attn_cached"
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.dim() != 4 or not t.is_cuda:
            raise ValueError(f"{who}: {name} must be a 4-D GPU tensor, got "
                             f"{tuple(t.shape)} on {t.device}")
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    if (k.shape[:2] != (B, T) or v.shape != k.shape or k.shape[3] != D or Hkv == 0
            or H % Hkv):
        raise ValueError(f"{who}: need q (B, T, H, D) and k, v (B, T, Hkv, D) with H a multiple "
                         f"of Hkv, got {tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if D not in _fc.SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{who}: head_dim must be one of {_fc.SUPPORTED_HEAD_DIMS}, got {D}")
    dtype = _fc.effective_dtype(q, k, v)
    if dtype not in _fc.SUPPORTED_DTYPES:
        raise ValueError(f"{who}: unsupported dtypes {q.dtype}/{k.dtype}/{v.dtype}")
    window, sinks = int(window or 0), int(sinks or 0)
    if window < 0:
        raise ValueError(f"{who}: window must be >= 0, got {window}")
    if window and not causal:
        # the reference's refusal (mixers.py:410-414)
        raise ValueError(
            "cached SWA decode requires causal=True. A window is defined "
            "on distance to the query, so a bidirectional block has no "
            "windowed reading -- the diffusion path is not SWA-compatible.")
    if window and not 0 <= sinks < window:
        raise ValueError(f"{who}: sinks must satisfy 0 <= sinks < window, "
                         f"got sinks={sinks} window={window}")
    if not window:
        sinks = 0
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if not (math.isfinite(scale) and scale > 0):
        raise ValueError(f"{who}: scale must be finite and > 0, got {scale}")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise RuntimeError(f"{who}: the cached step is inference-only (no backward); call it "
                           f"under torch.no_grad() or with detached inputs")
    if _fc._load() is None:
        raise RuntimeError(f"{who}: the library is unavailable ({_fc.unavailable_reason()})")
    dev = q.device
    q, k, v = (_dense(t, dtype) for t in (q, k, v))

    ck, cv = cache.get("k"), cache.get("v")
    if (ck is None) != (cv is None):
        raise ValueError(f"{who}: cache holds only one of 'k' / 'v'")
    Lc = 0 if ck is None else int(ck.shape[2])
    if ck is not None:
        ck = _cache_tensor(ck, B, Hkv, D, dtype, dev, who, "k")
        cv = _cache_tensor(cv, B, Hkv, D, dtype, dev, who, "v")
        if cv.shape[2] != Lc:
            raise ValueError(f"{who}: cache 'k' and 'v' lengths differ: {Lc} vs {cv.shape[2]}")
    start, cpos = Lc, None
    if window:
        start = int(cache.get("end", 0))
        cpos = cache.get("pos")
        if cpos is None:
            if Lc != start:
                raise ValueError(f"{who}: cache holds {Lc} rows but ends at position {start} "
                                 f"and has no 'pos'")
        else:
            cpos = cpos.to(device=dev, dtype=torch.int64).contiguous()
            if cpos.shape != (Lc,):
                raise ValueError(f"{who}: cache 'pos' must be ({Lc},), got {tuple(cpos.shape)}")

    g = None
    if gate is not None:
        if tuple(gate.shape) == (B, T, H, 1):
            gate = gate.squeeze(-1)
        if tuple(gate.shape) != (B, T, H):
            raise ValueError(f"{who}: gate logits must be (B, T, H) = {(B, T, H)}, got "
                             f"{tuple(gate.shape)}")
        g = gate.to(device=dev, dtype=torch.float32).contiguous()

    out = torch.empty(B, T, H, D, dtype=dtype, device=dev)
    lse = torch.empty(B, H, T, dtype=torch.float32, device=dev) if return_lse else None
    key = (B, T, H, Hkv, D, Lc, start, 1 if causal else 0, window, sinks, scale,
           _fc._DTYPE_CODE[dtype],
           ck.stride(0) if ck is not None else 0, ck.stride(1) if ck is not None else 0,
           cv.stride(0) if cv is not None else 0, cv.stride(1) if cv is not None else 0)
    shp, nws = _shape(key)
    lib = _capi.load()

    def ptr(t):
        return None if t is None else t.data_ptr()

    with _fc._on_device(q):
        stream = _fc._stream(q)
        ws = _workspace(dev, stream, nws) if nws > 0 else None
        st = lib.mi_attn_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), ptr(ck), ptr(cv),
                                ptr(cpos), ptr(g), out.data_ptr(), ptr(lse), ptr(ws),
                                ctypes.byref(shp), stream)
    _capi.check(st)

    if commit:
        kt, vt = k.transpose(1, 2), v.transpose(1, 2)          # (B, Hkv, T, D) views
        if window:
            # Keep the sinks plus the tail the next block can still reach
            # (mixers.py:437-448): positions < sinks or >= end - (w - s - 1).
            end = start + T
            tail = window - sinks - 1
            apos = torch.arange(start, end, device=dev, dtype=torch.int64)
            kpos = apos if Lc == 0 else torch.cat(
                [cpos if cpos is not None else torch.arange(start, device=dev), apos])
            live = (kpos < sinks) | (kpos >= end - tail)
            k_full = kt if Lc == 0 else torch.cat([ck, kt], dim=2)
            v_full = vt if Lc == 0 else torch.cat([cv, vt], dim=2)
            cache["k"] = k_full[:, :, live].detach()
            cache["v"] = v_full[:, :, live].detach()
            cache["pos"] = kpos[live]
            cache["end"] = end
        else:
            _commit_append(cache, "k", _KBUF, ck, kt, Lc, T)
            _commit_append(cache, "v", _VBUF, cv, vt, Lc, T)
    return (out, lse) if return_lse else out

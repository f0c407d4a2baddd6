"""CPU oracle for the KV-cached decode step -- TEST INFRASTRUCTURE ONLY.

Only ``tests/`` may import this module, and only as the checker; the product
path (``machinelearning_amd.decode``) never calls it.

What it restates (reference paths relative to bharathvbcr/MachineLearning):
the attention section of ``Attention.forward_cached``
(``nanolab/mixers.py:372-467``), in float64 numpy:

* ``step_mask``: the step's boolean mask (``mixers.py:407-433``). Without a
  window, ``causal=False`` is all-true (bidirectional block) and
  ``causal=True`` is ``[ones(T, Lc) | tril(T, T)]``. With a window
  (``causal`` required, else ``ValueError``), the mask is
  ``kpos <= apos & (kpos > apos - (w - s) | kpos < s)`` over absolute
  positions, with the cache's ``pos`` (``arange(end)`` before any eviction)
  followed by ``end .. end + T - 1``.
* ``cached_attention``: concatenate the cache with the block's K / V
  (``mixers.py:402-405``), repeat the kv heads for GQA, then masked softmax
  attention (``mixers.py:452-458``, SDPA's math). The optional output gate is
  applied as ``mixers.py:460-462`` does.
* ``commit``: the cache update (``mixers.py:435-450``). Without a window it
  keeps the concatenation. With one it keeps the live rows (positions
  ``< sinks`` or ``>= end - (w - s - 1)``) and sets ``pos`` and ``end``.

Pinning (``tests/test_decode.py``, CPU): a block-by-block cached run with
``commit`` reproduces ``oracle.attention.forward`` over the whole sequence.
That holds for causal blocks (== causal attention), for bidirectional blocks
of length L (== the block-causal mask with block = L, the cache invariant
``nanolab/diffusion.py:331`` rests on), and for SWA(12, 3) in blocks of 8, the
shape of the reference's ``swa_cached_decode_matches_the_uncached_window``
(``nanolab/tests.py:3420-3455``). The cache there stays within w - 1 rows and
stops growing. Also checked: the mask's closed forms, the refusal of a
bidirectional windowed step, and planted mistakes (an eviction tail one row
short, a window bound off by one), each caught. No function here is "parity
unpinned".
"""

from __future__ import annotations

import math

import numpy as np


def step_mask(Lc: int, T: int, causal: bool, window: int = 0, sinks: int = 0, cpos=None,
              start: int | None = None):
    """(T, Lc + T) keep-mask of one cached step, and the key positions (window only)."""
    if window:
        if not causal:
            raise ValueError("cached SWA decode requires causal=True")
        start = Lc if start is None else int(start)
        cp = np.arange(start) if cpos is None else np.asarray(cpos, dtype=np.int64)
        apos = np.arange(start, start + T)
        kpos = np.concatenate([cp, apos])
        keep = ((kpos[None, :] <= apos[:, None])
                & ((kpos[None, :] > apos[:, None] - (window - sinks)) | (kpos[None, :] < sinks)))
        return keep, kpos
    if causal:
        left = np.ones((T, Lc), dtype=bool)
        right = np.tril(np.ones((T, T), dtype=bool))
        return np.concatenate([left, right], axis=1), None
    return np.ones((T, Lc + T), dtype=bool), None


def cached_attention(q, k, v, cache: dict, causal: bool, window: int = 0, sinks: int = 0,
                     scale: float | None = None, gate=None):
    """One step: q [B,T,H,D], k/v [B,T,Hkv,D], cache {"k","v": [B,Hkv,Lc,D], "pos", "end"}.

    Returns (y [B,T,H,D], lse [B,H,T]) in float64.
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    B, T, H, D = q.shape
    Hkv = k.shape[2]
    rep = H // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    kt, vt = k.transpose(0, 2, 1, 3), v.transpose(0, 2, 1, 3)          # (B,Hkv,T,D)
    ck, cv = cache.get("k"), cache.get("v")
    k_full = kt if ck is None else np.concatenate([np.asarray(ck, np.float64), kt], axis=2)
    v_full = vt if cv is None else np.concatenate([np.asarray(cv, np.float64), vt], axis=2)
    Lc = k_full.shape[2] - T
    start = int(cache.get("end", 0)) if window else Lc
    keep, _ = step_mask(Lc, T, causal, window, sinks, cache.get("pos") if window else None,
                        start)
    kk = np.repeat(k_full, rep, axis=1)
    vv = np.repeat(v_full, rep, axis=1)
    qh = q.transpose(0, 2, 1, 3)                                        # (B,H,T,D)
    s = np.einsum("bhtd,bhjd->bhtj", qh, kk) * scale
    s = np.where(keep[None, None], s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    den = e.sum(axis=-1, keepdims=True)
    y = np.einsum("bhtj,bhjd->bhtd", e / den, vv).transpose(0, 2, 1, 3)
    lse = (m + np.log(den))[..., 0]
    if gate is not None:
        y = y / (1.0 + np.exp(-np.asarray(gate, np.float64)))[..., None]
    return y, lse


def commit(cache: dict, k, v, window: int = 0, sinks: int = 0) -> None:
    """Store the block's K / V into ``cache`` as ``mixers.py:435-450`` does."""
    kt = np.asarray(k, np.float64).transpose(0, 2, 1, 3)
    vt = np.asarray(v, np.float64).transpose(0, 2, 1, 3)
    T = kt.shape[2]
    ck, cv = cache.get("k"), cache.get("v")
    k_full = kt if ck is None else np.concatenate([ck, kt], axis=2)
    v_full = vt if cv is None else np.concatenate([cv, vt], axis=2)
    if window:
        start = int(cache.get("end", 0))
        cpos = cache.get("pos")
        cpos = np.arange(start) if cpos is None else np.asarray(cpos)
        kpos = np.concatenate([cpos, np.arange(start, start + T)])
        end = start + T
        tail = window - sinks - 1
        live = (kpos < sinks) | (kpos >= end - tail)
        cache["k"], cache["v"] = k_full[:, :, live], v_full[:, :, live]
        cache["pos"], cache["end"] = kpos[live], end
    else:
        cache["k"], cache["v"] = k_full, v_full


def decode_blocks(q, k, v, blocks, causal, window: int = 0, sinks: int = 0,
                  scale: float | None = None):
    """Run a whole sequence block by block through the cache (commit every block).

    q [B,S,H,D], k/v [B,S,Hkv,D]; ``blocks`` lists the block lengths (sum S).
    Returns the concatenated outputs [B,S,H,D] and the cache sizes after each commit.
    """
    cache: dict = {}
    outs, sizes, p0 = [], [], 0
    for n in blocks:
        y, _ = cached_attention(q[:, p0:p0 + n], k[:, p0:p0 + n], v[:, p0:p0 + n], cache,
                                causal, window, sinks, scale)
        commit(cache, k[:, p0:p0 + n], v[:, p0:p0 + n], window, sinks)
        outs.append(y)
        sizes.append(cache["k"].shape[2])
        p0 += n
    return np.concatenate(outs, axis=1), sizes

"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker. The product path
(``machinelearning_amd``) never calls it and has no CPU fallback.

What it restates (reference paths relative to bharathvbcr/MachineLearning):

* ``forward``  -- the brute-force reference the reference verifies its kernel
  against, ``nanolab/csrc/flash_attn_sim.py:193-212`` (``reference_attention``):
  materialise the dense score matrix, mask it, logsumexp + softmax, with GQA by
  repeating KV heads (head h reads KV head h // (H/Hkv), ``cu:8-14``).
  Extended by the masks the north star and the SWA mixer add: the sliding
  window SWA(w, s) of ``nanolab/mixers.py:96-135`` (key j visible to query i
  iff j <= i and (j > i - (w - s) or j < s): the w - s most recent keys plus s
  StreamingLLM sinks; s = 0 is the plain window i - w < j <= i) and
  non-causal (all keys).
* ``forward_gated`` / ``backward_gated`` -- the per-head output gate of
  gated attention (``mixers.py:340-344``: y = O * sigmoid(gate(x))), with
  dgate = (1 - sigmoid) * rowsum(dy * y).
* ``backward`` -- the closed-form gradient algebra of
  ``nanolab/csrc/flash_attn_cuda.cu:8-14``: p = exp(s*scale - L),
  Delta = rowsum(dO*O), dS = p*(dP - Delta), dQ = scale*dS K, dK = scale*dS^T Q
  (summed over the GQA group), dV = p^T dO. An LSE gradient enters as
  Delta -= dLSE (d LSE_i / d s_ij = p_ij).

Everything is float64 numpy, one (batch, head) at a time so a large shape
costs O(S^2) memory, not O(B*H*S^2).

Pinning (tests/test_oracle.py): ``backward`` is checked against torch
autograd of ``forward`` (an independent derivation), ``forward`` against
torch's SDPA math backend and a pure-Python triple loop, and both against the
invariants and special cases that the mathematics fixes (rows of P sum to 1,
sum_j dK_j = 0, sum dV = sum dO, S=1, Q=0, window=1, window >= S == causal,
causal row 0), and ``visible_mask`` position by position against the sets of
the reference's ``swa_mask_is_causal_local_and_keeps_the_sinks``
(``nanolab/tests.py:2993-3018``). ``forward_gated`` / ``backward_gated`` (the
per-head output gate of ``mixers.py:340-344``) are checked against torch
autograd of the gated composition, dgate included. ``round_operand`` is
checked against torch's own bfloat16 / float16 conversions (ties, subnormals,
the largest finite values), and ``backward(operand_dtype=...)`` against a
torch restatement that rounds P and dS with those conversions; without
``operand_dtype`` it is bit for bit the plain backward. ``backward(magnitudes=
True)`` is checked against a pure-Python sum of |terms| and the triangle
inequality. No function here is "parity unpinned".
"""

from __future__ import annotations

import math

import numpy as np


def visible_mask(S: int, causal: bool = True, window: int = 0, sinks: int = 0,
                 block: int = 0) -> np.ndarray:
    """[S_q, S_k] boolean keep-mask. Rows are queries, columns keys.

    Causal is ``tril`` (flash_attn_sim.py:206-207); with ``block`` > 1 it is
    the block-causal mask of ``block_causal_mask`` (mixers.py:76-93): query
    block >= key block. The window keeps ``k > q - (window - sinks)`` on top of
    causal, plus the causal part of the first ``sinks`` keys (mixers.py:117-131),
    0 <= sinks < window.
    """
    i = np.arange(S)[:, None]
    j = np.arange(S)[None, :]
    keep = np.ones((S, S), dtype=bool)
    block = int(block or 0)
    if block > 1:
        if not causal or (window and window > 0):
            raise ValueError("block-causal needs causal and no window")
        return (i // block) >= (j // block)
    if causal:
        keep &= j <= i
    sinks = int(sinks or 0)
    if window and window > 0:
        if not causal:
            raise ValueError("a sliding window is causal-only")
        if not 0 <= sinks < window:
            raise ValueError(f"sinks must satisfy 0 <= sinks < window, got {sinks}, {window}")
        keep &= (j > i - (window - sinks)) | (j < sinks)
    elif sinks:
        raise ValueError("sinks need a sliding window")
    return keep


def _as64(x) -> np.ndarray:
    if hasattr(x, "detach"):           # torch tensor -> numpy without importing torch here
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, dtype=np.float64)


def _check(q, k, v):
    if q.ndim != 4 or k.ndim != 4 or v.ndim != 4:
        raise ValueError("expected [B,S,H,D] / [B,S,Hkv,D]")
    B, S, H, D = q.shape
    if k.shape != v.shape or k.shape[0] != B or k.shape[1] != S or k.shape[3] != D:
        raise ValueError(f"shape mismatch q{q.shape} k{k.shape} v{v.shape}")
    if k.shape[2] <= 0 or H % k.shape[2]:
        raise ValueError("n_head must be a positive multiple of n_kv_head")
    return B, S, H, k.shape[2], D


def forward(q, k, v, scale: float | None = None, causal: bool = True, window: int = 0,
            sinks: int = 0, block: int = 0):
    """Brute-force attention. q [B,S,H,D], k/v [B,S,Hkv,D] -> (O [B,S,H,D], LSE [B,H,S]).

    float64 throughout; LSE is the natural-log logsumexp of the masked, scaled
    scores (the taped L of cu:8-14).
    """
    q, k, v = _as64(q), _as64(k), _as64(v)
    B, S, H, Hkv, D = _check(q, k, v)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    group = H // Hkv
    keep = visible_mask(S, causal, window, sinks, block)
    o = np.zeros((B, S, H, D))
    lse = np.zeros((B, H, S))
    for b in range(B):
        for h in range(H):
            hk = h // group
            s = (q[b, :, h, :] @ k[b, :, hk, :].T) * scale
            s = np.where(keep, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            e = np.exp(s - m)
            den = e.sum(axis=1, keepdims=True)
            lse[b, h] = (m + np.log(den))[:, 0]
            o[b, :, h, :] = (e / den) @ v[b, :, hk, :]
    return o, lse


def round_operand(x: np.ndarray, kind: str) -> np.ndarray:
    """``x`` rounded to a 16-bit MMA operand format and back to float64.

    ``kind`` "bfloat16": the float32 value's upper 16 bits, rounded to nearest
    with ties to even (bf16 is the top half of an IEEE binary32: 8 exponent and
    7 stored mantissa bits). "float16": IEEE binary16 via numpy's conversion
    (round to nearest even, subnormals kept). Finite inputs only.
    """
    x32 = np.asarray(x, dtype=np.float32)
    if kind == "float16":
        return x32.astype(np.float16).astype(np.float64)
    if kind != "bfloat16":
        raise ValueError(kind)
    u = x32.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def backward(q, k, v, o, lse, do, scale: float | None = None, causal: bool = True,
             window: int = 0, dlse=None, sinks: int = 0, block: int = 0,
             operand_dtype: str | None = None, magnitudes: bool = False):
    """Closed-form gradients (cu:8-14) -> (dQ, dK, dV), float64.

    ``o`` and ``lse`` are the forward's outputs (the tape); ``dlse`` is an
    optional incoming gradient of LSE [B,H,S].

    ``operand_dtype`` ("bfloat16" / "float16"): P and dS are rounded to that
    format before the products that consume them, as the reference's 16-bit
    MMA backward packs them into its mma.sync operands (``pack_a_from_acc``:
    dS for dQ += dS K at ``cu:945``, dS and P for dK += dS^T Q and
    dV += P^T dO at ``cu:1153-1154``). Everything else stays float64.

    ``magnitudes``: the same three products over absolute values,
    scale * |dS| |K|, scale * |dS|^T |Q| and |P|^T |dO| -- per gradient element
    the sum of its terms' magnitudes, which bounds the effect of a relative
    rounding u of every term by u times that sum.
    """
    q, k, v, o, lse, do = (_as64(t) for t in (q, k, v, o, lse, do))
    B, S, H, Hkv, D = _check(q, k, v)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    group = H // Hkv
    keep = visible_mask(S, causal, window, sinks, block)
    dl = None if dlse is None else _as64(dlse)
    dq = np.zeros_like(q)
    dk = np.zeros_like(k)
    dv = np.zeros_like(v)
    for b in range(B):
        for h in range(H):
            hk = h // group
            qh, kh, vh, doh = q[b, :, h], k[b, :, hk], v[b, :, hk], do[b, :, h]
            s = (qh @ kh.T) * scale
            p = np.where(keep, np.exp(s - lse[b, h][:, None]), 0.0)
            delta = (doh * o[b, :, h]).sum(axis=1)
            if dl is not None:
                delta = delta - dl[b, h]
            dp = doh @ vh.T
            ds = p * (dp - delta[:, None])
            if operand_dtype is not None:
                p, ds = round_operand(p, operand_dtype), round_operand(ds, operand_dtype)
            if magnitudes:
                p, ds, kh, qh, doh = (np.abs(t) for t in (p, ds, kh, qh, doh))
            dq[b, :, h] = scale * (ds @ kh)
            dk[b, :, hk] += scale * (ds.T @ qh)
            dv[b, :, hk] += p.T @ doh
    return dq, dk, dv


def delta(o, do, dlse=None):
    """Delta[b,h,i] = sum_d dO*O (- dLSE) -> [B,H,S] (flash_delta_kernel, cu:1231-1262)."""
    o, do = _as64(o), _as64(do)
    d = (o * do).sum(axis=-1).transpose(0, 2, 1)
    if dlse is not None:
        d = d - _as64(dlse)
    return d



def sigmoid(z):
    z = _as64(z)
    return 1.0 / (1.0 + np.exp(-z))


def forward_gated(q, k, v, gate, scale=None, causal=True, window=0, sinks=0):
    """Gated attention (mixers.py:340-344): y = sigmoid(gate)[..., None] * O.

    gate: logits [B, S, H]. Returns (y, lse) with lse of the ungated attention.
    """
    o, lse = forward(q, k, v, scale, causal, window, sinks)
    return o * sigmoid(gate)[..., None], lse


def backward_gated(q, k, v, gate, y, lse, dy, scale=None, causal=True, window=0, dlse=None,
                   sinks=0):
    """Gradients of ``forward_gated`` -> (dq, dk, dv, dgate).

    dO_attn = sigmoid(z) * dy feeds the ungated backward (whose Delta,
    rowsum(dO_attn * O), equals rowsum(dy * y)); dgate = sigmoid'(z) *
    rowsum(dy * O) = (1 - sigmoid(z)) * rowsum(dy * y).
    """
    sg = sigmoid(gate)[..., None]
    y, dy = _as64(y), _as64(dy)
    o = y / sg
    dq, dk, dv = backward(q, k, v, o, lse, sg * dy, scale, causal, window, dlse, sinks)
    dgate = (1.0 - sg[..., 0]) * (dy * y).sum(axis=-1)
    return dq, dk, dv, dgate

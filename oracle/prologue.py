"""CPU oracle for the fused attention prologue -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py`` may import this
module, and only as the checker. The product path never calls it.

What it restates (reference paths relative to bharathvbcr/MachineLearning):

* ``rms_norm`` -- ``RMSNorm.forward`` (``nanolab/mixers.py:46-56``):
  ``F.rms_norm(x, (D,), weight, eps)`` = x / sqrt(mean(x^2) + eps) * weight,
  over the last (head) dimension, eps = 1e-6 by default.
* ``rope_cache`` -- ``build_rope_cache`` (``mixers.py:59-65``): inv_freq =
  base^(-2i/D), angles t * inv_freq, duplicated to D columns (cat(f, f)).
* ``apply_rope`` -- ``apply_rope`` (``mixers.py:68-75``): x*cos + rot(x)*sin
  with rot(x) = cat(-x[D/2:], x[:D/2]).
* ``prologue`` -- the attention block's q / k path (``mixers.py:282-292``):
  q_norm / k_norm (when qk_norm) then RoPE (when cos is given).
* ``prologue_backward`` -- closed-form gradients of that composition:
  RoPE^T (the rotation's transpose: dy = g*cos + rot^T(g*sin) with
  rot^T(u) = cat(u[D/2:], -u[:D/2])), then the RMSNorm backward
  dx = rstd * (dn - n * mean(dn * n)) with n = x * rstd, dn = dy * weight, and
  dweight = sum over rows of dy * n.

float64 numpy throughout. Pinning (tests/test_oracle.py): the forward against
a torch float64 restatement with torch's own ``F.rms_norm``, the backward
against torch autograd of that forward, the rope cache against the closed
form at hand-picked entries, and invariants (RoPE is an isometry per pair,
RMSNorm output has mean square weight^2 per element on average, rotating by
t then reading position 0 is the identity). No function here is
"parity unpinned".
"""

from __future__ import annotations

import numpy as np


def _as64(x) -> np.ndarray:
    if hasattr(x, "detach"):
        x = x.detach().cpu().double().numpy()
    return np.asarray(x, dtype=np.float64)


def rope_cache(T: int, D: int, base: float = 10000.0):
    """(cos, sin), each [T, D], float64 (mixers.py:59-65 before its dtype cast)."""
    inv_freq = 1.0 / (base ** (np.arange(0, D, 2, dtype=np.float64) / D))
    freqs = np.outer(np.arange(T, dtype=np.float64), inv_freq)
    emb = np.concatenate([freqs, freqs], axis=-1)
    return np.cos(emb), np.sin(emb)


def rot(x: np.ndarray) -> np.ndarray:
    """cat(-x2, x1) over the last dimension."""
    d = x.shape[-1] // 2
    return np.concatenate([-x[..., d:], x[..., :d]], axis=-1)


def rot_t(u: np.ndarray) -> np.ndarray:
    """Transpose of ``rot``: <rot(x), u> = <x, rot_t(u)>."""
    d = u.shape[-1] // 2
    return np.concatenate([u[..., d:], -u[..., :d]], axis=-1)


def rms_norm(x, weight, eps: float = 1e-6):
    """x / sqrt(mean(x^2, -1) + eps) * weight -> (y, rstd[..., 0])."""
    x, w = _as64(x), _as64(weight)
    rstd = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * rstd * w, rstd[..., 0]


def apply_rope(x, cos, sin):
    """x: [B, T, H, D]; cos / sin: [T, D]."""
    x, c, s = _as64(x), _as64(cos), _as64(sin)
    return x * c[None, :, None, :] + rot(x) * s[None, :, None, :]


def prologue(x, weight, cos, sin, eps: float = 1e-6, norm: bool = True):
    """RMSNorm (optional) then RoPE on x [B, T, H, D] -> (out, rstd [B, T, H])."""
    x = _as64(x)
    if norm:
        y, rstd = rms_norm(x, weight, eps)
    else:
        y, rstd = x, np.ones(x.shape[:-1])
    return apply_rope(y, cos, sin), rstd


def prologue_backward(g, x, weight, cos, sin, eps: float = 1e-6, norm: bool = True):
    """Gradients of ``prologue`` for the incoming gradient g -> (dx, dweight)."""
    g, x, w = _as64(g), _as64(x), _as64(weight)
    c, s = _as64(cos)[None, :, None, :], _as64(sin)[None, :, None, :]
    dy = g * c + rot_t(g * s)
    if not norm:
        return dy, None
    rstd = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    n = x * rstd
    dn = dy * w
    dx = rstd * (dn - n * np.mean(dn * n, axis=-1, keepdims=True))
    dw = (dy * n).reshape(-1, x.shape[-1]).sum(axis=0)
    return dx, dw

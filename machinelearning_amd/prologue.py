"""Fused q / k prologue of nanolab's attention block: QK-norm + RoPE in one pass.

nanolab's attention (``nanolab/mixers.py:282-292``) turns each projected head
row into the attention kernel's input with a chain of torch ops:
``RMSNorm`` (``F.rms_norm``, ``mixers.py:46-56``) when ``qk_norm`` is on, then
``apply_rope`` (``x*cos + cat(-x2, x1)*sin``, ``mixers.py:68-75``). Under
autocast that chain runs in fp32, and ``flash_cuda``'s autocast bridge casts
the result back to bf16. ``qk_norm_rope`` does the whole chain in one
HIP pass per tensor (``csrc/qk_prologue.hip`` through the C ABI,
``mi_qk_prologue_fwd`` / ``mi_qk_prologue_bwd``) and writes ``out_dtype``
directly. It is an autograd op: gradients flow to ``x`` and to the norm
``weight`` (cos / sin are constants, as in the reference's rope cache).

There is no CPU fallback: without the library this raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes

import torch

from . import _capi
from . import flash_cuda as _fc

SUPPORTED_HEAD_DIMS = (32, 64, 128)
_CODE = {torch.float32: _capi.MI_F32, torch.float16: _capi.MI_F16,
         torch.bfloat16: _capi.MI_BF16}


def _shape(x, out_dtype, norm, rope, eps):
    B, T, H, D = x.shape
    return _capi.MiPrologueShape(B, T, H, D, _CODE[x.dtype], _CODE[out_dtype], int(norm),
                                 int(rope), float(eps))


def _ptr(t):
    return None if t is None else t.data_ptr()


class _ProFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, cos, sin, eps, out_dtype):
        lib = _capi.load()
        norm, rope = weight is not None, cos is not None
        out = torch.empty(x.shape, dtype=out_dtype, device=x.device)
        rstd = torch.empty(x.shape[:-1], dtype=torch.float32, device=x.device) if norm else None
        shp = _shape(x, out_dtype, norm, rope, eps)
        with _fc._on_device(x):
            st = lib.mi_qk_prologue_fwd(x.data_ptr(), _ptr(weight), _ptr(cos), _ptr(sin),
                                        out.data_ptr(), _ptr(rstd), ctypes.byref(shp),
                                        _fc._stream(x))
        _capi.check(st)
        ctx.save_for_backward(x, weight, cos, sin, rstd)
        ctx.eps, ctx.out_dtype, ctx.norm, ctx.rope = eps, out_dtype, norm, rope
        return out

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, g):
        lib = _capi.load()
        x, weight, cos, sin, rstd = ctx.saved_tensors
        g = g.to(ctx.out_dtype).contiguous()
        dx = torch.empty_like(x)
        dw = None
        shp = _shape(x, ctx.out_dtype, ctx.norm, ctx.rope, ctx.eps)
        if ctx.norm:
            dw = torch.zeros(x.shape[-1], dtype=torch.float32, device=x.device)
        n = ctypes.c_longlong(0)
        _capi.check(lib.mi_qk_prologue_workspace(ctypes.byref(shp), ctypes.byref(n)))
        ws = torch.empty(max(n.value, 1), dtype=torch.float32, device=x.device)
        with _fc._on_device(x):
            st = lib.mi_qk_prologue_bwd(g.data_ptr(), x.data_ptr(), _ptr(weight), _ptr(cos),
                                        _ptr(sin), _ptr(rstd), dx.data_ptr(), _ptr(dw),
                                        ws.data_ptr(), ctypes.byref(shp), _fc._stream(x))
        _capi.check(st)
        return dx, dw, None, None, None, None


def qk_norm_rope(x: torch.Tensor, weight: torch.Tensor | None, cos: torch.Tensor | None,
                 sin: torch.Tensor | None, eps: float = 1e-6,
                 out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """rope(rms_norm(x) * weight) on x [B, T, H, D] in one pass.

    ``weight`` [D] is the RMSNorm weight (None: no norm, the reference's
    ``qk_norm=False``); ``cos`` / ``sin`` [T, D] are the rope cache rows of the
    sequence positions (None: no RoPE, the reference's ``cos is None``).
    ``out_dtype`` defaults to ``x.dtype``; pass ``torch.bfloat16`` to feed the
    16-bit attention kernel directly. Raises ``ValueError`` for unsupported
    inputs and ``RuntimeError`` when the library cannot run.
    """
    if x.dim() != 4 or not x.is_cuda:
        raise ValueError(f"qk_norm_rope: x must be a 4-D GPU tensor [B, T, H, D], got "
                         f"{tuple(x.shape)} on {x.device}")
    B, T, H, D = x.shape
    if D not in SUPPORTED_HEAD_DIMS or x.dtype not in _CODE:
        raise ValueError(f"qk_norm_rope: head_dim must be one of {SUPPORTED_HEAD_DIMS} and the "
                         f"dtype float32 / float16 / bfloat16, got {D} / {x.dtype}")
    out_dtype = x.dtype if out_dtype is None else out_dtype
    if out_dtype not in _CODE:
        raise ValueError(f"qk_norm_rope: unsupported out_dtype {out_dtype}")
    if (cos is None) != (sin is None):
        raise ValueError("qk_norm_rope: cos and sin go together")
    if weight is not None and tuple(weight.shape) != (D,):
        raise ValueError(f"qk_norm_rope: weight must be [{D}], got {tuple(weight.shape)}")
    if cos is not None and (tuple(cos.shape) != (T, D) or tuple(sin.shape) != (T, D)):
        raise ValueError(f"qk_norm_rope: cos / sin must be [{T}, {D}], got "
                         f"{tuple(cos.shape)} / {tuple(sin.shape)}")
    if not (eps >= 0.0) or eps == float("inf"):
        raise ValueError(f"qk_norm_rope: eps must be finite and >= 0, got {eps}")
    if _fc._load() is None:
        raise RuntimeError(f"qk_norm_rope: the library is unavailable ({_fc.unavailable_reason()})")
    x = x.contiguous()
    w = None if weight is None else weight.to(device=x.device, dtype=torch.float32).contiguous()
    c = None if cos is None else cos.to(device=x.device, dtype=torch.float32).contiguous()
    s = None if sin is None else sin.to(device=x.device, dtype=torch.float32).contiguous()
    if x.numel() == 0:
        out = x.to(out_dtype)
        return out if w is None else out + 0.0 * w.sum().to(out_dtype)
    return _ProFn.apply(x, w, c, s, float(eps), out_dtype)

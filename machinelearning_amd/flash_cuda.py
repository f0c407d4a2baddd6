"""MI355X flash attention: the drop-in for nanolab's opt-in ``flash_cuda`` op.

Same module surface as ``nanolab/flash_cuda.py`` (names, argument meaning,
error behaviour), so ``nanolab/mixers.py:347-370`` and ``nanolab/model.py``
call it unchanged:

    from machinelearning_amd import flash_cuda
    if flash_cuda.supports(q, k, v):          # dtype / head_dim / layout
        y = flash_cuda.flash_attn(q, k, v, scale)

and two extensions the north star asks for, keyword-only on the old entry
point so the positional ``flash_attn(q, k, v, scale)`` call keeps binding
``scale`` (``nanolab/mixers.py:364``):

    y = flash_cuda.flash_attn(q, k, v, scale, causal=False)
    y = flash_cuda.flash_attn(q, k, v, scale, window=256)
    out, lse = flash_cuda.attn(q, k, v, causal, window, scale)   # LSE returned

Below this module is ``libmi_attn.so`` (hand-written HIP for gfx950, C ABI in
``include/mi_attn.h``), prebuilt in-tree by ``build_ext``, loaded with ctypes.
There is no CPU fallback in here: when the library cannot run, ``is_available``
is False with a reason, and ``flash_attn`` raises ``RuntimeError`` -- the
caller's fallback (the mixer's SDPA path) is the caller's business.

Paths
-----
* 16-bit (f16/bf16): MFMA ``v_mfma_f32_32x32x16_{bf16,f16}`` forward and
  backward at every supported head dim ("mma" in the reference's vocabulary).
* float32: the same kernels on ``v_mfma_f32_32x32x2f32`` (fp32 in, fp32 out).
* ``use_mma=False`` on 16-bit inputs runs the float32 kernels on upcast copies
  (fp32 arithmetic end to end, P and dS never rounded), then casts O back --
  the role the reference's FMA kernels play (``flash_cuda.py:244-256``).

``NANOLAB_FLASH_CUDA=0`` refuses the library, as in the reference
(``flash_cuda.py:103-105``).
"""

from __future__ import annotations

import ctypes
import logging
import math
import os

import torch

from . import _capi

log = logging.getLogger("machinelearning_amd.flash_cuda")

SUPPORTED_HEAD_DIMS = (32, 64, 128)
SUPPORTED_DTYPES = (torch.float32, torch.float16, torch.bfloat16)
MMA_DTYPES = (torch.float16, torch.bfloat16)
# The MFMA backward covers every supported head dim (the reference stopped its
# tensor-core backward at 64 for register pressure, flash_cuda.py:46-49).
MMA_BWD_HEAD_DIMS = (32, 64, 128)
# Head dims at which a 16-bit forward that will be differentiated also keeps the
# output's rounding residual, so the backward's Delta = rowsum(dO * O) sees O to
# ~16 bits. At D = 128 on long rows (the S = 8192 workload) Delta from the
# bf16-rounded O alone put dK up to 3e-2 off; at D <= 64 the BASELINE shapes stay
# within 0.74 of the 2e-2 bound without it, and the headline keeps its traffic.
RESIDUAL_HEAD_DIMS = (128,)
TARGET_ARCH = "gfx950"

_DTYPE_CODE = {torch.float32: _capi.MI_F32, torch.float16: _capi.MI_F16,
               torch.bfloat16: _capi.MI_BF16}

_lib = None
_load_error: str | None = None
_load_attempted = False
_mma_ok = False
_mma_error: str | None = None
_f32_ok = False
_f32_error: str | None = None


def _probe_mfma(lib, dtype: torch.dtype) -> tuple[bool, str]:
    """Check the kernels' MFMA register layout against the hardware.

    Multiplies seeded matrices through the exact fragment helpers the attention
    kernels use and compares with a plain matmul of the same rounded inputs. A
    wrong layout is wrong by O(1), so the 1e-2 bar is not a close call. Fails
    closed (mirrors ``_probe_mma``, ``nanolab/flash_cuda.py:59-88``).
    """
    try:
        code = _DTYPE_CODE[dtype]
        kp = lib.mi_mfma_probe_k(code)
        g = torch.Generator(device="cpu").manual_seed(0)
        a = torch.randn(32, kp, generator=g).to(dtype).cuda()
        b = torch.randn(kp, 32, generator=g).to(dtype).cuda()
        d = torch.empty(32, 32, dtype=torch.float32, device="cuda")
        st = lib.mi_mfma_probe(a.data_ptr(), b.data_ptr(), d.data_ptr(), code,
                               torch.cuda.current_stream().cuda_stream)
        if st:
            return False, _capi.error_string(st)
        torch.cuda.synchronize()
        want = a.float() @ b.float()
        err = (d - want).abs().max().item()
        if not err < 1e-2:
            return False, (f"MFMA layout probe failed for {dtype}: "
                           f"max |mfma - matmul| = {err:.3e}")
        return True, ""
    except Exception as e:  # noqa: BLE001 - any failure closes the gate
        return False, f"{type(e).__name__}: {e}"


def _load():
    """Load the prebuilt library and run the layout probes, once.

    Returns the ctypes library or None with ``_load_error`` set. Never raises:
    callers gate on ``is_available()``.
    """
    global _lib, _load_error, _load_attempted, _mma_ok, _mma_error, _f32_ok, _f32_error
    if _load_attempted:
        return _lib
    _load_attempted = True
    if os.environ.get("NANOLAB_FLASH_CUDA", "1") == "0":
        _load_error = "disabled by NANOLAB_FLASH_CUDA=0"
        return None
    if not torch.cuda.is_available():
        _load_error = "no GPU device"
        return None
    try:
        arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    except Exception:  # noqa: BLE001
        arch = "unknown"
    if arch != TARGET_ARCH:
        _load_error = f"libmi_attn.so is built for {TARGET_ARCH}; this device is {arch}"
        return None
    try:
        lib = _capi.load()
    except OSError as e:
        _load_error = f"OSError: {e}"
        log.warning("libmi_attn.so did not load (%s)", _load_error)
        return None
    _lib = lib
    _mma_ok, _mma_error = True, None
    for dt in MMA_DTYPES:
        ok, why = _probe_mfma(lib, dt)
        if not ok:
            _mma_ok, _mma_error = False, why
            log.warning("16-bit MFMA path off (%s)", why)
            break
    _f32_ok, _f32_error = _probe_mfma(lib, torch.float32)
    if not _f32_ok:
        log.warning("float32 MFMA path off (%s)", _f32_error)
    return _lib


def is_available() -> bool:
    """Whether libmi_attn.so loaded on a gfx950 device (the first call loads it)."""
    return _load() is not None


def unavailable_reason() -> str:
    """The load failure recorded by the one load attempt; '' after a successful load."""
    _load()
    return "" if _lib is not None else (_load_error or "unknown")


def mma_available() -> bool:
    """Whether the bf16/f16 MFMA kernels may run: library loaded, fragment probe passed."""
    return _load() is not None and _mma_ok


def mma_unavailable_reason() -> str:
    """The load failure, else the failed 16-bit probe's message; '' when the path is on."""
    if _load() is None:
        return unavailable_reason()
    return "" if _mma_ok else (_mma_error or "unknown")


def effective_dtype(q: torch.Tensor, k: torch.Tensor,
                    v: torch.Tensor) -> torch.dtype | None:
    """Arithmetic dtype for (q, k, v): the GPU autocast dtype while autocast is on,
    else their shared dtype, else None (mixed dtypes outside autocast).

    The autocast case matters because a custom autograd op is not cast by
    autocast itself, and nanolab's mixer passes fp32 q/k (after RoPE) with a
    bf16 v under autocast (``nanolab/flash_cuda.py:161-177``).
    """
    if q.is_cuda and torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    if q.dtype == k.dtype == v.dtype:
        return q.dtype
    return None


def supports(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """Shape, dtype and device test for (q, k, v); the library is not touched.

    Checks 4-D [B, S, heads, D] tensors on the GPU with a supported effective
    dtype and head dim, matching B / S / D, and query heads a multiple of the
    kv heads (``nanolab/flash_cuda.py:180-202``). Strides do not matter: the
    entry points cast and make contiguous copies as needed.
    """
    return _supported_dtype(q, k, v) is not None


def _supported_dtype(q, k, v):
    """supports()'s test, returning the effective dtype when it passes (else None).
    Shapes are compared as plain int tuples (cheaper than torch.Size slices)."""
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        return None
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        return None
    dtype = effective_dtype(q, k, v)
    if dtype not in SUPPORTED_DTYPES:
        return None
    (B, S, H, D), (Bk, Sk, Hk, Dk), (Bv, Sv, Hv, Dv) = (tuple(q.shape), tuple(k.shape),
                                                        tuple(v.shape))
    if D not in SUPPORTED_HEAD_DIMS:
        return None
    if (Bk, Sk) != (B, S) or (Bv, Sv) != (B, S):
        return None
    if Hk != Hv or Dk != D or Dv != D:
        return None
    if Hk == 0 or H % Hk != 0:
        return None
    return dtype


# ---------------------------------------------------------------------------
# raw launches through the C ABI (caller-allocated outputs, current stream)
# ---------------------------------------------------------------------------
_SHAPES = _capi.ShapeCache()


def _shape_of(q, k, causal, window, sinks, scale, block=0):
    """(struct, byref pointer, backward workspace floats) for this call's shape."""
    B, S, H, D = q.shape
    return _SHAPES.get((B, S, H, k.shape[2], D, causal, window, scale, _DTYPE_CODE[q.dtype],
                        sinks, block))


def _stream(t: torch.Tensor) -> int:
    """Raw handle of the current HIP stream of t's device."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


class _on_device:
    """Make ``t``'s device current for the duration of a C-ABI call."""

    def __init__(self, t: torch.Tensor):
        self.idx = t.get_device()
        self.prev = None

    def __enter__(self):
        cur = torch.cuda.current_device()
        if cur != self.idx:
            self.prev = cur
            torch.cuda.set_device(self.idx)

    def __exit__(self, *exc):
        if self.prev is not None:
            torch.cuda.set_device(self.prev)


def _wants_residual(q, sinks, gate, window: int = 0) -> bool:
    """Whether a differentiated forward keeps O's rounding residual: 16-bit, no
    gate, and either a RESIDUAL_HEAD_DIMS head dim or sinks (which the 16-bit
    window kernels fold) that some row sees beyond its span (window - sinks < S).
    A sink key's dK sums dS = P (dP - Delta) over every row from the key on, with P
    of order 1 / span on each: the 8-bit rounding of a 16-bit O in Delta =
    rowsum(dO * O) then accumulates over the sequence (dK off by 1.2x the bound at
    S 2048, SWA(8, 4)); with the residual Delta carries O to ~16 bits."""
    if q.dtype not in MMA_DTYPES or gate is not None:
        return False
    folded = sinks > 0 and window - sinks < q.shape[1]
    return q.shape[-1] in RESIDUAL_HEAD_DIMS or folded


def _fwd(q, k, v, causal, window, sinks, scale, gate=None, block=0, residual=False):
    """(o, lse, o_res); o_res is None unless `residual` (mi_attn_fwd_res)."""
    lib = _capi.load()
    B, S, H, D = q.shape
    o = torch.empty_like(q)
    o_res = torch.empty_like(q) if residual else None
    lse = torch.empty((B, H, S), dtype=torch.float32, device=q.device)
    _, sp, _ = _shape_of(q, k, causal, window, sinks, scale, block)
    with _on_device(q):
        if residual:
            st = lib.mi_attn_fwd_res(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                     o_res.data_ptr(), lse.data_ptr(), sp, _stream(q))
        elif gate is None:
            st = lib.mi_attn_fwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                 lse.data_ptr(), sp, _stream(q))
        else:
            st = lib.mi_attn_fwd_gated(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       gate.data_ptr(), o.data_ptr(), lse.data_ptr(), sp,
                                       _stream(q))
    if st:
        _capi.check(st)
    return o, lse, o_res


def _bwd(do, dlse, q, k, v, o, lse, causal, window, sinks, scale, gate=None, block=0,
         o_res=None):
    lib = _capi.load()
    if do.dtype != q.dtype:
        do = do.to(q.dtype)
    if not do.is_contiguous():
        do = do.contiguous()
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    if dlse is not None:
        dlse = dlse.to(torch.float32).contiguous()
    _, sp, nws = _shape_of(q, k, causal, window, sinks, scale, block)
    # [2,B,H,S] planes (+ float32's sink partials, or the split dK/dV partials of
    # small 16-bit GQA grids)
    delta = lse.new_empty(nws)
    dgate = None
    with _on_device(q):
        if o_res is not None:
            st = lib.mi_attn_bwd_res(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                     o_res.data_ptr(), do.data_ptr(), lse.data_ptr(),
                                     None if dlse is None else dlse.data_ptr(), delta.data_ptr(),
                                     dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), sp, _stream(q))
        elif gate is None:
            st = lib.mi_attn_bwd(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                 do.data_ptr(), lse.data_ptr(),
                                 None if dlse is None else dlse.data_ptr(), delta.data_ptr(),
                                 dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), sp, _stream(q))
        else:
            do_attn = torch.empty_like(do)          # sigmoid(gate) * do, the kernels' input
            dgate = torch.empty_like(gate)
            st = lib.mi_attn_bwd_gated(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       gate.data_ptr(), o.data_ptr(), do.data_ptr(),
                                       lse.data_ptr(), None if dlse is None else dlse.data_ptr(),
                                       delta.data_ptr(), do_attn.data_ptr(), dq.data_ptr(),
                                       dk.data_ptr(), dv.data_ptr(), dgate.data_ptr(), sp,
                                       _stream(q))
    if st:
        _capi.check(st)
    return dq, dk, dv, dgate


class _AttnFn(torch.autograd.Function):
    """Attention on [B,S,H,D] returning (O, LSE); both outputs differentiable.

    The LSE tape [B,H,S] is saved for the backward, like the reference's
    ``_FlashAttnFn`` (``nanolab/flash_cuda.py:205-230``); its incoming
    gradient folds into Delta inside the library.
    """

    @staticmethod
    def forward(ctx, q, k, v, causal, window, sinks, scale, gate=None, block=0):
        residual = any(ctx.needs_input_grad[:3]) and _wants_residual(q, sinks, gate, window)
        o, lse, o_res = _fwd(q, k, v, causal, window, sinks, scale, gate, block, residual)
        ctx.save_for_backward(q, k, v, o, lse, gate, o_res)
        ctx.causal, ctx.window, ctx.sinks, ctx.scale, ctx.block = causal, window, sinks, scale, block
        ctx.set_materialize_grads(False)
        return o, lse

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, do, dlse):
        q, k, v, o, lse, gate, o_res = ctx.saved_tensors
        if do is None:
            do = torch.zeros_like(o)
        dq, dk, dv, dgate = _bwd(do, dlse, q, k, v, o, lse, ctx.causal, ctx.window, ctx.sinks,
                                 ctx.scale, gate, ctx.block, o_res)
        return dq, dk, dv, None, None, None, None, dgate, None


def _prepare(q, k, v, causal, window, sinks, scale, use_mma, who, block=0):
    dtype = _supported_dtype(q, k, v)
    if dtype is None:
        raise ValueError(
            f"{who}: unsupported inputs "
            f"(q={tuple(q.shape)}/{q.dtype}, k={tuple(k.shape)}/{k.dtype}, "
            f"v={tuple(v.shape)}/{v.dtype}); head_dim must be one of "
            f"{SUPPORTED_HEAD_DIMS} and the effective dtype one of {SUPPORTED_DTYPES}")
    window = int(window or 0)
    if window < 0:
        raise ValueError(f"{who}: window must be >= 0, got {window}")
    if window > 0 and not causal:
        raise ValueError(f"{who}: a sliding window is causal-only")
    sinks = int(sinks or 0)
    if sinks < 0 or (sinks > 0 and sinks >= window):
        # the same contract as sliding_window_mask (nanolab/mixers.py:117-120)
        raise ValueError(f"{who}: sinks must satisfy 0 <= sinks < window, "
                         f"got sinks={sinks} window={window}")
    block = int(block or 0)
    if block < 0:
        raise ValueError(f"{who}: block must be >= 0, got {block}")
    if block > 1 and (not causal or window > 0):
        # the reference refuses block-causal with SWA as well (mixers.py:300-304)
        raise ValueError(f"{who}: block-causal attention (block={block}) is causal across "
                         f"blocks and exclusive with a sliding window")
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    scale = float(scale)
    if not math.isfinite(scale):
        raise ValueError(f"{who}: scale must be finite, got {scale}")
    if q.dtype != dtype or not q.is_contiguous():
        q = q.to(dtype).contiguous()
    if k.dtype != dtype or not k.is_contiguous():
        k = k.to(dtype).contiguous()
    if v.dtype != dtype or not v.is_contiguous():
        v = v.to(dtype).contiguous()
    if use_mma is None:
        use_mma = dtype in MMA_DTYPES and mma_available()
    elif use_mma:
        if dtype not in MMA_DTYPES:
            raise ValueError(f"{who}: use_mma=True but the effective dtype is {dtype}; "
                             f"the 16-bit MFMA path exists only for {MMA_DTYPES}")
        if not mma_available():
            raise RuntimeError(f"{who}: use_mma=True but the MFMA path is unavailable "
                               f"({mma_unavailable_reason()})")
    if _load() is None:
        raise RuntimeError(f"machinelearning_amd flash attention is unavailable "
                           f"({unavailable_reason()})")
    return q, k, v, bool(causal), window, sinks, scale, dtype, bool(use_mma), block


def _positive_scale(q, scale):
    """Map scale <= 0 onto the library's scale > 0 contract, exactly.

    softmax(scale * q k^T) is unchanged by (q, scale) -> (-q, -scale), and for
    scale == 0 every score is 0 = (0 * q) k^T at any positive scale. Both
    rewrites are autograd ops on q, so dQ picks up the sign (or the zero) and
    dK = scale' * dS^T q' is already the true gradient.
    """
    if scale > 0:
        return q, scale
    if scale < 0:
        return -q, -scale
    return q * 0, 1.0


def _run(q, k, v, causal, window, sinks, scale, dtype, use_mma, gate=None, block=0):
    q, scale = _positive_scale(q, scale)
    if dtype in MMA_DTYPES and not use_mma:
        # fp32 arithmetic end to end on upcast copies; the casts are autograd ops.
        if not _f32_ok:
            raise RuntimeError(f"float32 path unavailable ({_f32_error})")
        o, lse = _AttnFn.apply(q.float(), k.float(), v.float(), causal, window, sinks, scale,
                               gate, block)
        return o.to(dtype), lse
    if dtype == torch.float32 and not _f32_ok:
        raise RuntimeError(f"float32 path unavailable ({_f32_error})")
    return _AttnFn.apply(q, k, v, causal, window, sinks, scale, gate, block)


def _gate_of(gate, q, who):
    """Gate logits as a contiguous fp32 [B, S, H] tensor on q's device (autograd-safe)."""
    if gate is None:
        return None
    B, S, H, _ = q.shape
    if tuple(gate.shape) == (B, S, H, 1):
        gate = gate.squeeze(-1)
    if tuple(gate.shape) != (B, S, H):
        raise ValueError(f"{who}: gate logits must be [B, S, H] = {(B, S, H)}, got "
                         f"{tuple(gate.shape)}")
    return gate.to(device=q.device, dtype=torch.float32).contiguous()


def attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, causal: bool = True,
         window: int = 0, scale: float | None = None,
         use_mma: bool | None = None, *,
         sinks: int = 0, gate: torch.Tensor | None = None,
         block: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """GQA flash attention. q [B,S,H,D], k/v [B,S,Hkv,D] -> (O [B,S,H,D], LSE [B,H,S] fp32).

    ``causal``: key j visible to query i iff j <= i (else every key).
    ``window`` > 0 (causal only): the reference's SWA(window, sinks) mask
    (``nanolab/mixers.py:96-135``): j > i - (window - sinks), or j < sinks
    (StreamingLLM attention sinks, 0 <= sinks < window).
    ``gate``: optional gate logits [B, S, H] (or [B, S, H, 1]); the output
    becomes O * sigmoid(gate), the per-head output gate of nanolab's gated
    attention (``mixers.py:340-344``), applied on O inside the kernel, with
    its gradient returned to ``gate``. LSE stays that of the ungated attention.
    ``block`` > 1 (causal, no window): the block-causal (semi-autoregressive)
    mask of ``nanolab/mixers.py:76-93``, key j visible to query i iff
    j // block <= i // block.
    ``scale`` defaults to 1/sqrt(D). LSE is the natural-log logsumexp of the
    masked, scaled scores and is differentiable. Raises ValueError for
    unsupported inputs and RuntimeError when the library cannot run.
    """
    q, k, v, causal, window, sinks, scale, dtype, use_mma, block = _prepare(
        q, k, v, causal, window, sinks, scale, use_mma, "flash_cuda.attn", block)
    return _run(q, k, v, causal, window, sinks, scale, dtype, use_mma,
                _gate_of(gate, q, "flash_cuda.attn"), block)


def flash_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
               scale: float | None = None, use_mma: bool | None = None, *,
               causal: bool = True, window: int = 0, sinks: int = 0,
               gate: torch.Tensor | None = None, block: int = 0) -> torch.Tensor:
    """Flash attention returning O only -- ``nanolab/flash_cuda.py:233-279``'s signature.

    ``flash_attn(q, k, v, scale)`` is the reference's causal call unchanged;
    ``causal``, ``window``, ``sinks``, ``gate`` and ``block`` (see ``attn``) are
    keyword-only extensions. ``use_mma``: None
    takes the 16-bit MFMA kernels whenever the dtype is 16-bit, True demands
    them (ValueError on fp32, RuntimeError if the probe failed), False forces
    fp32 arithmetic.
    """
    q, k, v, causal, window, sinks, scale, dtype, use_mma, block = _prepare(
        q, k, v, causal, window, sinks, scale, use_mma, "flash_cuda.flash_attn", block)
    return _run(q, k, v, causal, window, sinks, scale, dtype, use_mma,
                _gate_of(gate, q, "flash_cuda.flash_attn"), block)[0]


def sdpa_reference(q, k, v, scale, causal: bool = True, window: int = 0, sinks: int = 0,
                   block: int = 0):
    """What nanolab does without the kernel: widen KV heads, transpose, SDPA.

    Mirrors ``nanolab/flash_cuda.py:282-294`` (``repeat_interleave`` included)
    and adds the window, sinks included, as a dense mask
    (``nanolab/mixers.py:96-135`` and ``mixers.py:331-335``).
    """
    import torch.nn.functional as F
    group = q.shape[2] // k.shape[2]
    qs = q.transpose(1, 2)
    ks = k.repeat_interleave(group, dim=2).transpose(1, 2)
    vs = v.repeat_interleave(group, dim=2).transpose(1, 2)
    if block and block > 1:
        T = q.shape[1]
        blk = torch.arange(T, device=q.device) // block
        keep = blk[:, None] >= blk[None, :]                    # mixers.py:88-89
        y = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=keep[None, None], scale=scale)
    elif window and window > 0:
        T = q.shape[1]
        i = torch.arange(T, device=q.device)
        causal_keep = i[None, :] <= i[:, None]
        keep = causal_keep & (i[None, :] > i[:, None] - (window - sinks))
        if sinks:
            keep = keep | (causal_keep & (i[None, :] < sinks))
        y = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=keep[None, None], scale=scale)
    else:
        y = F.scaled_dot_product_attention(qs, ks, vs, is_causal=causal, scale=scale)
    return y.transpose(1, 2).contiguous()


def sdpa_backend(q, k, v, scale, causal: bool = True, window: int = 0, sinks: int = 0,
                 block: int = 0) -> str:
    """Name of the SDPA backend torch runs for ``sdpa_reference`` on these inputs:
    the first of its priority order (flash, memory-efficient, math) that accepts
    them, tried one at a time under ``torch.nn.attention.sdpa_kernel``."""
    from torch.nn.attention import SDPBackend, sdpa_kernel
    for name, be in (("flash", SDPBackend.FLASH_ATTENTION),
                     ("efficient", SDPBackend.EFFICIENT_ATTENTION), ("math", SDPBackend.MATH)):
        try:
            with sdpa_kernel([be]), torch.no_grad():
                sdpa_reference(q, k, v, scale, causal, window, sinks, block)
            return name
        except RuntimeError:
            continue
    return "none"


def _timed_ms(fn, iters: int) -> float:
    """Mean ms per call over ``iters`` calls queued back to back (HIP events), after
    a few untimed calls; one synchronisation at each end."""
    for _ in range(3):
        fn()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(iters):
        fn()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / iters


def main(argv=None) -> int:
    """Self-check of the kernels on one shape: errors against an fp32 reference, then speed.

    Keeps the reference CLI's flags (``nanolab/flash_cuda.py:319-327``) and adds
    --window / --sinks / --noncausal. Every path this build can run on the
    inputs ("mfma" at 16 bits, "fp32" arithmetic via ``use_mma=False``) is
    compared with ``sdpa_reference`` evaluated in float32 on the same rounded
    inputs, and timed forward alone and forward + backward. A last path,
    "sdpa", times ``sdpa_reference`` itself in the inputs' dtype on the same GPU
    (what nanolab runs without the kernel; the reference's harness times SDPA
    beside its kernel the same way, ``nanolab/flash_cuda.py:353-378``) and names
    the backend torch picked. The report is one JSON object per path (errors as
    max-abs and relative to the reference's max, times in ms, throughput in
    TFLOP/s of the algorithmic 4*D / 14*D flops per visible pair).
    """
    import argparse
    import json

    from . import perf

    ap = argparse.ArgumentParser(description="flash attention self-check (errors, then speed)")
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--seq", type=int, default=1024)
    ap.add_argument("--heads", type=int, default=12)
    ap.add_argument("--kv_heads", type=int, default=4)
    ap.add_argument("--head_dim", type=int, default=32)
    ap.add_argument("--dtype", default="bf16", choices=("fp32", "fp16", "bf16"))
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--window", type=int, default=0)
    ap.add_argument("--sinks", type=int, default=0)
    ap.add_argument("--noncausal", action="store_true")
    a = ap.parse_args(argv)

    if not is_available():
        print(json.dumps({"available": False, "reason": unavailable_reason()}))
        return 1
    dtype = {"fp32": torch.float32, "fp16": torch.float16, "bf16": torch.bfloat16}[a.dtype]
    causal = not a.noncausal
    gen = torch.Generator(device="cpu").manual_seed(0)

    def draw(heads):
        return torch.randn(a.batch, a.seq, heads, a.head_dim, generator=gen).to(dtype).cuda()
    q, k, v = draw(a.heads), draw(a.kv_heads), draw(a.kv_heads)
    dy = draw(a.heads)
    scale = a.head_dim ** -0.5
    # The comparison target: the mixer's own SDPA path, in float32, on the same bits.
    ref_in = [t.float().requires_grad_() for t in (q, k, v)]
    y_ref = sdpa_reference(*ref_in, scale, causal, a.window, a.sinks)
    g_ref = torch.autograd.grad(y_ref, ref_in, dy.float())

    paths = {"fp32": False}
    if dtype in MMA_DTYPES and mma_available():
        paths = {"mfma": True, "fp32": False}
    fl_fwd = perf.flops(a.batch, a.heads, a.seq, a.head_dim, causal, a.window, bwd=False,
                        sinks=a.sinks)
    fl_all = perf.flops(a.batch, a.heads, a.seq, a.head_dim, causal, a.window, sinks=a.sinks)
    for name, mma in paths.items():
        xs = [t.detach().requires_grad_() for t in (q, k, v)]

        def fwd():
            return flash_attn(*xs, scale, use_mma=mma, causal=causal, window=a.window,
                              sinks=a.sinks)
        y = fwd()
        grads = torch.autograd.grad(y, xs, dy)
        errs = {}
        for tname, got, want in zip(("out", "dq", "dk", "dv"), (y,) + grads, (y_ref,) + g_ref):
            e = (got.float() - want.float()).abs().max().item()
            errs[tname] = {"max_abs": e, "rel": e / max(want.abs().max().item(), 1e-30)}
        with torch.no_grad():
            t_fwd = _timed_ms(fwd, a.iters)
        t_all = _timed_ms(lambda: torch.autograd.grad(fwd(), xs, dy), a.iters)
        print(json.dumps({
            "path": name, "shape": {"B": a.batch, "T": a.seq, "H": a.heads,
                                    "Hkv": a.kv_heads, "D": a.head_dim, "dtype": a.dtype,
                                    "causal": causal, "window": a.window, "sinks": a.sinks},
            "errors_vs_fp32_sdpa": errs,
            "fwd_ms": round(t_fwd, 4), "fwd_bwd_ms": round(t_all, 4),
            "fwd_tflops": round(fl_fwd / t_fwd / 1e9, 1),
            "fwd_bwd_tflops": round(fl_all / t_all / 1e9, 1)}), flush=True)
    # SDPA on the same GPU, in the inputs' dtype: timing context, never a target.
    xs = [t.detach().requires_grad_() for t in (q, k, v)]

    def sdpa_fwd():
        return sdpa_reference(*xs, scale, causal, a.window, a.sinks)
    with torch.no_grad():
        t_fwd = _timed_ms(sdpa_fwd, a.iters)
    t_all = _timed_ms(lambda: torch.autograd.grad(sdpa_fwd(), xs, dy), a.iters)
    backend = sdpa_backend(q, k, v, scale, causal, a.window, a.sinks)
    print(json.dumps({
        "path": "sdpa", "backend": backend,
        "shape": {"B": a.batch, "T": a.seq, "H": a.heads, "Hkv": a.kv_heads, "D": a.head_dim,
                  "dtype": a.dtype, "causal": causal, "window": a.window, "sinks": a.sinks},
        "fwd_ms": round(t_fwd, 4), "fwd_bwd_ms": round(t_all, 4),
        "fwd_tflops": round(fl_fwd / t_fwd / 1e9, 1),
        "fwd_bwd_tflops": round(fl_all / t_all / 1e9, 1)}), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

"""mi_attn_bwd_noalloc (the backward whose workspace is a static device array)
against mi_attn_bwd with a caller-owned workspace, through the C ABI.

Both run the same kernels, so the results must agree bit for bit. Two calls in
a row, the second on a smaller input, so the second call reads the array after
the first left its contents there; sink shapes (float32's sink pass uses the
partial-sum region after the two planes); and a shape too large for the array,
which must be
refused before anything runs. One exception to bitwise agreement: a GQA shape
whose split dK/dV partials do not fit the array runs the unsplit dK/dV kernel
there, which sums the group's heads in another fp32 order (within one bf16
rounding of mi_attn_bwd's split result).
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from machinelearning_amd import _capi
from machinelearning_amd import flash_cuda as fc

pytestmark = pytest.mark.gpu

MI_ERR_SCRATCH = 10
SCRATCH_FLOATS = 4 << 20


@pytest.fixture(scope="module", autouse=True)
def _library():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert fc.is_available(), fc.unavailable_reason()
    yield


def _inputs(B, T, H, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    mk = lambda h: torch.randn(B, T, h, D, generator=g).to(dtype).cuda()
    return mk(H), mk(Hkv), mk(Hkv), mk(H)


def _both(B, T, H, Hkv, D, dtype, window=0, sinks=0, seed=0):
    """(mi_attn_bwd grads, mi_attn_bwd_noalloc grads) for one shape."""
    lib = _capi.load()
    code = {torch.float32: _capi.MI_F32, torch.float16: _capi.MI_F16,
            torch.bfloat16: _capi.MI_BF16}[dtype]
    shp = _capi.shape(B, T, H, Hkv, D, True, window, D ** -0.5, code, sinks)
    sp = ctypes.byref(shp)
    st = torch.cuda.current_stream().cuda_stream
    q, k, v, do = _inputs(B, T, H, Hkv, D, dtype, seed)
    P = lambda t: t.data_ptr()
    o = torch.empty_like(q)
    lse = torch.empty(B, H, T, device="cuda")
    _capi.check(lib.mi_attn_fwd(P(q), P(k), P(v), P(o), P(lse), sp, st))
    outs = []
    for noalloc in (False, True):
        dq, dk, dv = (torch.full_like(t, float("nan")) for t in (q, k, v))
        if noalloc:
            _capi.check(lib.mi_attn_bwd_noalloc(P(q), P(k), P(v), P(o), P(do), P(lse), None,
                                                 P(dq), P(dk), P(dv), sp, st))
        else:
            ws = torch.empty(_capi.workspace_floats(shp), device="cuda")
            _capi.check(lib.mi_attn_bwd(P(q), P(k), P(v), P(o), P(do), P(lse), None, P(ws),
                                        P(dq), P(dk), P(dv), sp, st))
        torch.cuda.synchronize()
        outs.append((dq, dk, dv))
    return outs


def _assert_same(outs, tag):
    for name, a, b in zip(("dQ", "dK", "dV"), *outs):
        assert torch.isfinite(b).all(), f"{tag}: {name} not fully written"
        assert torch.equal(a, b), f"{tag}: {name} differs from mi_attn_bwd"


def test_two_calls_second_smaller():
    """Board-like causal bf16 shape, then a smaller GQA shape on the same array."""
    _assert_same(_both(2, 1024, 12, 12, 64, torch.bfloat16, seed=1), "call 1 (B2 T1024 H12 D64)")
    _assert_same(_both(1, 200, 4, 2, 32, torch.bfloat16, seed=2), "call 2 (B1 T200 H4/2 D32)")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_sink_shapes(dtype):
    """90-wide window with 65 sinks and SWA(17, 4): float32's separate sink pass keeps
    per-chunk partial sums after the two planes; 16-bit folds the sinks (two sink tiles
    at 65) and keeps none."""
    _assert_same(_both(2, 300, 4, 2, 64, dtype, window=90, sinks=65, seed=3), f"sinks {dtype}")
    _assert_same(_both(1, 130, 2, 1, 32, dtype, window=17, sinks=4, seed=4), f"sinks 4 {dtype}")


def test_gqa_split_partials_beyond_the_array_run_unsplit():
    """The reference's E17 shape (B8 T1024 H12/Hkv4 D32): mi_attn_bwd splits the dK/dV
    walk per query head (fp32 partials, 6.3M floats), which the static array cannot
    hold; the no-alloc call runs the unsplit kernel instead of refusing."""
    B, T, H, Hkv, D = 8, 1024, 12, 4, 32
    shp = _capi.shape(B, T, H, Hkv, D, True, 0, D ** -0.5, _capi.MI_BF16)
    assert _capi.workspace_floats(shp) > SCRATCH_FLOATS > 2 * B * H * T
    (dq0, dk0, dv0), (dq1, dk1, dv1) = _both(B, T, H, Hkv, D, torch.bfloat16, seed=5)
    assert torch.equal(dq0, dq1), "dQ does not depend on the dK/dV split"
    for name, a, b in (("dK", dk0, dk1), ("dV", dv0, dv1)):
        assert torch.isfinite(b).all(), f"{name} not fully written"
        a32, b32 = a.float(), b.float()
        # One bf16 rounding apart at most: |a - b| <= 2^-7 * max(|a|, |b|) (+ a floor for
        # values near zero, where the fp32 sums differ by a few ulps of their terms).
        tol = 2.0 ** -7 * torch.maximum(a32.abs(), b32.abs()) + 1e-6 * a32.abs().max()
        bad = (a32 - b32).abs() > tol
        assert not bad.any(), (f"{name}: split and unsplit differ by "
                               f"{(a32 - b32).abs().max().item():.3g} at {bad.nonzero()[0].tolist()}")
        assert (a32 != b32).float().mean().item() < 0.05, f"{name}: too many elements differ"


def test_too_large_is_refused_before_any_launch():
    lib = _capi.load()
    B, T, H = 4, 8200, 64                    # 2*B*H*T = 4,198,400 floats > 4 << 20
    assert 2 * B * H * T > SCRATCH_FLOATS
    shp = _capi.shape(B, T, H, H, 64, True, 0, 0.125, _capi.MI_BF16)
    # Full-size buffers (so that even a wrongly accepted call would stay in bounds).
    x = torch.empty(B, T, H, 64, device="cuda", dtype=torch.bfloat16)
    lse = torch.empty(B, H, T, device="cuda")
    sentinel = torch.full_like(x, 7.0)
    P = lambda t: t.data_ptr()
    st = lib.mi_attn_bwd_noalloc(P(x), P(x), P(x), P(x), P(x), P(lse), None, P(sentinel),
                                 P(sentinel), P(sentinel), ctypes.byref(shp),
                                 torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert st == MI_ERR_SCRATCH, st
    assert "scratch" in _capi.error_string(st)
    assert bool((sentinel == 7.0).all())

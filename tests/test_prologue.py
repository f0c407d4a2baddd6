"""The fused q / k prologue (QK-norm + RoPE): oracle pinning on the CPU, and
parity of the HIP kernels through the C ABI on the GPU.

Reference: ``RMSNorm`` (``nanolab/mixers.py:46-56``), ``build_rope_cache``
(``mixers.py:59-65``), ``apply_rope`` (``mixers.py:68-75``), applied to q and
k at ``mixers.py:282-292``. Tolerances: float32 outputs within 1e-5 of the
float64 oracle; 16-bit outputs within the output format's rounding (2^-8
relative to the row's largest value, plus 1e-3 absolute) -- both written in
``_tol``.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import prologue as orp


def _rand(B, T, H, D, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, H, D, generator=g, dtype=torch.float64) * 1.7
    w = 1.0 + 0.3 * torch.randn(D, generator=g, dtype=torch.float64)
    gr = torch.randn(B, T, H, D, generator=g, dtype=torch.float64)
    return x, w, gr


def _rope_complex(x, t0, base=10000.0):
    """RoPE as a rotation of the pairs (x_i, x_{i+D/2}) by angle t * base^(-2i/D)."""
    B, T, H, D = x.shape
    half = D // 2
    inv = base ** (-torch.arange(0, D, 2, dtype=torch.float64) / D)
    ang = (torch.arange(T, dtype=torch.float64) + t0)[:, None] * inv[None, :]   # [T, D/2]
    z = torch.complex(x[..., :half], x[..., half:]) * torch.polar(
        torch.ones_like(ang), ang)[None, :, None, :]
    return torch.cat([z.real, z.imag], dim=-1)


# ---------------------------------------------------------------- oracle pins (CPU)
def test_rope_cache_closed_form():
    c, s = orp.rope_cache(3, 4, 10000.0)
    # inv_freq = [1, 0.01]; angles at t = 2: [2, 0.02, 2, 0.02]
    assert np.allclose(c[2], np.cos([2.0, 0.02, 2.0, 0.02]), atol=0, rtol=1e-15)
    assert np.allclose(s[2], np.sin([2.0, 0.02, 2.0, 0.02]), atol=0, rtol=1e-15)
    assert np.array_equal(c[0], np.ones(4)) and np.array_equal(s[0], np.zeros(4))


def test_rms_norm_matches_torch():
    x, w, _ = _rand(2, 5, 3, 64, seed=1)
    y, rstd = orp.rms_norm(x, w, 1e-6)
    ref = F.rms_norm(x, (64,), w, 1e-6)
    assert np.abs(y - ref.numpy()).max() < 1e-13
    assert np.abs(rstd - 1 / torch.sqrt((x * x).mean(-1) + 1e-6).numpy()).max() < 1e-13


def test_apply_rope_is_a_pair_rotation():
    x, _, _ = _rand(2, 9, 3, 32, seed=2)
    c, s = orp.rope_cache(9, 32)
    got = orp.apply_rope(x, c, s)
    assert np.abs(got - _rope_complex(x, 0).numpy()).max() < 1e-13
    # an isometry per row, and relative: <rope(q)_t1, rope(k)_t2> depends on t1 - t2 only
    assert np.abs(np.linalg.norm(got, axis=-1) - np.linalg.norm(x.numpy(), axis=-1)).max() < 1e-12
    q, k = x[:, :1], x[:, 1:2]
    c2, s2 = orp.rope_cache(12, 32)
    a = (orp.apply_rope(q, c2[3:4], s2[3:4]) * orp.apply_rope(k, c2[1:2], s2[1:2])).sum(-1)
    b = (orp.apply_rope(q, c2[7:8], s2[7:8]) * orp.apply_rope(k, c2[5:6], s2[5:6])).sum(-1)
    assert np.abs(a - b).max() < 1e-12


@pytest.mark.parametrize("norm", [True, False])
def test_backward_matches_autograd(norm):
    x, w, gr = _rand(2, 7, 3, 64, seed=3)
    c, s = orp.rope_cache(7, 64)
    xa, wa = x.clone().requires_grad_(), w.clone().requires_grad_()
    y = F.rms_norm(xa, (64,), wa, 1e-6) if norm else xa
    out = _rope_complex(y, 0)
    (out * gr).sum().backward()
    o, _ = orp.prologue(x, w, c, s, 1e-6, norm)
    dx, dw = orp.prologue_backward(gr, x, w, c, s, 1e-6, norm)
    assert np.abs(o - out.detach().numpy()).max() < 1e-12
    assert np.abs(dx - xa.grad.numpy()).max() < 1e-12
    if norm:
        assert np.abs(dw - wa.grad.numpy()).max() < 1e-11


def test_planted_rope_transpose_sign_is_caught(monkeypatch):
    x, w, gr = _rand(1, 5, 2, 32, seed=4)
    c, s = orp.rope_cache(5, 32)
    monkeypatch.setattr(orp, "rot_t", orp.rot)          # wrong: rot instead of its transpose
    dx, _ = orp.prologue_backward(gr, x, w, c, s, 1e-6, True)
    xa, wa = x.clone().requires_grad_(), w.clone().requires_grad_()
    (_rope_complex(F.rms_norm(xa, (32,), wa, 1e-6), 0) * gr).sum().backward()
    assert np.abs(dx - xa.grad.numpy()).max() > 1e-3


# ---------------------------------------------------------------- host checks (CPU)
def test_prologue_shape_validation():
    from machinelearning_amd import _capi
    lib = _capi.load()

    def st(**kw):
        base = dict(B=2, T=8, H=3, D=64, dtype_in=2, dtype_out=2, norm=1, rope=1, eps=1e-6)
        base.update(kw)
        n = ctypes.c_longlong(-1)
        return lib.mi_qk_prologue_workspace(ctypes.byref(_capi.MiPrologueShape(**base)),
                                            ctypes.byref(n)), n.value
    assert st()[0] == 0 and st()[1] > 0
    assert st(norm=0) == (0, 0)
    assert st(D=48)[0] == 4
    assert st(dtype_out=9)[0] == 3
    assert st(eps=float("nan"))[0] == 9
    assert st(B=-1)[0] == 2
    shp = _capi.MiPrologueShape(2, 8, 3, 64, 2, 2, 1, 1, 1e-6)
    assert lib.mi_qk_prologue_fwd(None, None, None, None, None, None, ctypes.byref(shp), None) == 1


# ---------------------------------------------------------------- GPU parity
def _tol(ref: np.ndarray, dtype) -> float:
    if dtype == torch.float32:
        return 1e-5 * max(1.0, float(np.abs(ref).max()))
    return 2.0 ** -8 * float(np.abs(ref).max()) + 1e-3


def _gpu(x, w, gr, cos, sin, dt_in, dt_out, norm=True, rope=True):
    from machinelearning_amd.prologue import qk_norm_rope
    xg = x.to(dt_in).cuda().requires_grad_()
    wg = w.float().cuda().requires_grad_() if norm else None
    c = torch.as_tensor(cos).float().cuda() if rope else None
    s = torch.as_tensor(sin).float().cuda() if rope else None
    out = qk_norm_rope(xg, wg, c, s, 1e-6, dt_out)
    grads = torch.autograd.grad(out, [xg] + ([wg] if norm else []), gr.to(dt_out).cuda())
    torch.cuda.synchronize()
    res = [out.detach().double().cpu().numpy(), grads[0].double().cpu().numpy()]
    res.append(grads[1].double().cpu().numpy() if norm else None)
    return res


def _check(got, x, w, gr, cos, sin, dt_in, dt_out, norm, rope, tag):
    xr = x.to(dt_in).double()                     # the kernel's actual input values
    grr = gr.to(dt_out).double()
    if rope:
        c, s = cos, sin
    else:
        c, s = np.ones((x.shape[1], x.shape[3])), np.zeros((x.shape[1], x.shape[3]))
    ref, _ = orp.prologue(xr, w.float().double(), c, s, 1e-6, norm)
    rdx, rdw = orp.prologue_backward(grr, xr, w.float().double(), c, s, 1e-6, norm)
    pairs = [("out", got[0], ref, dt_out), ("dx", got[1], rdx, dt_in)]
    if norm:
        pairs.append(("dw", got[2], rdw, torch.float32))
    for name, a, b, dt in pairs:
        tol = _tol(b, dt) if name != "dw" else 1e-4 * max(1.0, float(np.abs(b).max()))
        err = float(np.abs(a - b).max())
        print(f"{tag} {name}: max|err|={err:.3e} tol={tol:.2e}", flush=True)
        assert err < tol, f"{tag}: {name} {err:.3e} >= {tol:.2e}"


DTYPES = [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
          (torch.float16, torch.float16), (torch.float32, torch.bfloat16)]


@pytest.mark.gpu
@pytest.mark.parametrize("dts", DTYPES, ids=lambda d: f"{d[0]}->{d[1]}".replace("torch.", ""))
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("mode", ["norm+rope", "rope", "norm"])
def test_prologue_parity(dts, D, mode):
    dt_in, dt_out = dts
    norm, rope = "norm" in mode, "rope" in mode
    x, w, gr = _rand(2, 37, 3, D, seed=D)
    cos, sin = orp.rope_cache(37, D)
    got = _gpu(x, w, gr, cos, sin, dt_in, dt_out, norm, rope)
    _check(got, x, w, gr, cos, sin, dt_in, dt_out, norm, rope, f"{mode} D{D} {dts}")


@pytest.mark.gpu
def test_prologue_board_shape_and_determinism():
    """q at the board shape (B16 T1024 H12 D64, bf16), sampled rows + bitwise repeat."""
    x, w, gr = _rand(16, 1024, 12, 64, seed=9)
    cos, sin = orp.rope_cache(1024, 64)
    a = _gpu(x, w, gr, cos, sin, torch.bfloat16, torch.bfloat16)
    b = _gpu(x, w, gr, cos, sin, torch.bfloat16, torch.bfloat16)
    assert all(np.array_equal(p, q) for p, q in zip(a, b)), "not bitwise reproducible"
    _check(a, x, w, gr, cos, sin, torch.bfloat16, torch.bfloat16, True, True, "board")


@pytest.mark.gpu
def test_prologue_feeds_attention():
    """The fused prologue then the attention op == the reference chain then SDPA."""
    from machinelearning_amd import flash_cuda as fc
    from machinelearning_amd.prologue import qk_norm_rope
    B, T, H, D = 2, 100, 4, 64
    g = torch.Generator().manual_seed(5)
    q = torch.randn(B, T, H, D, generator=g).cuda()
    k = torch.randn(B, T, H, D, generator=g).cuda()
    v = torch.randn(B, T, H, D, generator=g).cuda()
    wq = (1 + 0.2 * torch.randn(D, generator=g)).cuda()
    wk = (1 + 0.2 * torch.randn(D, generator=g)).cuda()
    c, s = (torch.as_tensor(t).float().cuda() for t in orp.rope_cache(T, D))
    qr = qk_norm_rope(q, wq, c, s, 1e-6, torch.bfloat16)
    kr = qk_norm_rope(k, wk, c, s, 1e-6, torch.bfloat16)
    y = fc.flash_attn(qr, kr, v.to(torch.bfloat16), 1 / math.sqrt(D))
    # reference chain in fp32 on the same device
    def ref_rope(x):
        x1, x2 = x[..., : D // 2], x[..., D // 2:]
        return x * c[None, :, None, :] + torch.cat((-x2, x1), -1) * s[None, :, None, :]
    qf = ref_rope(F.rms_norm(q, (D,), wq, 1e-6))
    kf = ref_rope(F.rms_norm(k, (D,), wk, 1e-6))
    yr = F.scaled_dot_product_attention(qf.transpose(1, 2), kf.transpose(1, 2),
                                        v.transpose(1, 2), is_causal=True,
                                        scale=1 / math.sqrt(D)).transpose(1, 2)
    assert (y.float() - yr).abs().max().item() < 3e-2

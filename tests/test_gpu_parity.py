"""Parity of the HIP kernels (through the C ABI) against the float64 oracle.

Tolerances (applied in ``tests/_parity.py``): float32
inputs within 1e-5 max-abs on O, dQ, dK, dV and 1e-4 on LSE; 16-bit inputs
within 2e-2 of the oracle evaluated on the same rounded inputs (an "upcast"
reference), element by element, plus the output format's own half-ulp at
that element; LSE 1e-4. At the board config, whose dO ~ N(0, 1e-2) makes the
gradients ~1e-2, a relative bound (max|err| / max|ref| <= 2e-2) is added so a
zero gradient cannot pass, and the board shape is also run with dO ~ N(0, 1).

Shapes mirror the reference's own device tests (``nanolab/tests.py:352-482``:
T = 100, 37, 33 tails, GQA groups 1/2/4, D 32/64/128) plus the BASELINE
configs: the fp32 smoke config in full, the four 16-bit configs at full size
with the oracle run on sampled heads and size-independent invariants checked
on every head, and every head and element of them against the float32 upcast
reference computed on the GPU.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from machinelearning_amd import flash_cuda as fc
from machinelearning_amd.inputs import CONFIGS, make_inputs
from oracle import attention as orc
from tests import _parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _library():
    # Fail (not skip) on a GPU box where the native library does not load:
    # a GPU test must never pass on a fallback.
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert fc.is_available(), fc.unavailable_reason()
    yield


def _gpu(q, k, v, do, causal=True, window=0, scale=None, use_mma=None, sinks=0):
    qg, kg, vg = (t.detach().cuda().requires_grad_() for t in (q, k, v))
    o, lse = fc.attn(qg, kg, vg, causal, window, scale, use_mma=use_mma, sinks=sinks)
    dq, dk, dv = torch.autograd.grad(o, (qg, kg, vg), do.cuda())
    torch.cuda.synchronize()
    return [t.detach().double().cpu().numpy() for t in (o, lse, dq, dk, dv)]


def _ref(q, k, v, do, causal=True, window=0, scale=None, sinks=0):
    o, lse = orc.forward(q, k, v, scale, causal, window, sinks=sinks)
    dq, dk, dv = orc.backward(q, k, v, o, lse, do, scale, causal, window, sinks=sinks)
    return [o, lse, dq, dk, dv]


def _compare(got, want, dtype, tag, rel_grad=None):
    """Every tensor at the bar of its dtype; rel_grad adds the relative bound on dQ/dK/dV."""
    names = ("O", "LSE", "dQ", "dK", "dV")
    for name, a, b in zip(names, got, want):
        rel = rel_grad if name in ("dQ", "dK", "dV") else None
        _parity.check(tag, name, a, b, dtype, rel=rel)


def _rand(B, T, H, Hkv, D, dtype, seed=0, do_std=1.0):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, T, H, D, generator=g).to(dtype)
    k = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
    v = torch.randn(B, T, Hkv, D, generator=g).to(dtype)
    do = torch.randn(B, T, H, D, generator=g).mul(do_std).to(dtype)
    return q, k, v, do


# ---------------------------------------------------------------------------
def test_mfma_layout_probe():
    assert fc.mma_available(), fc.mma_unavailable_reason()
    assert fc._f32_ok, fc._f32_error


def test_smoke_config_fp32_full():
    """fp32 B4 H4 S256 D64 causal, every head, 1e-5."""
    cfg = CONFIGS["smoke"]
    q, k, v, do = make_inputs(cfg)
    _compare(_gpu(q, k, v, do, True, 0, cfg.scale), _ref(q, k, v, do, True, 0, cfg.scale),
             torch.float32, "smoke-fp32")


SHAPES = [  # (B, T, H, Hkv, D): the reference's device/mirror test shapes
    (2, 100, 4, 2, 32),
    (1, 37, 2, 2, 32),
    (1, 33, 2, 1, 32),
    (1, 64, 4, 1, 64),
    (1, 80, 2, 1, 128),
    (2, 130, 4, 4, 64),
    (1, 257, 2, 2, 128),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B%dT%dH%d/%dD%d" % s)
@pytest.mark.parametrize("mode", ["causal", "noncausal", "window"])
def test_small_shapes(shape, dtype, mode):
    B, T, H, Hkv, D = shape
    q, k, v, do = _rand(B, T, H, Hkv, D, dtype, seed=T + D)
    causal = mode != "noncausal"
    window = 17 if mode == "window" else 0
    scale = 1.0 / math.sqrt(D)
    _compare(_gpu(q, k, v, do, causal, window, scale), _ref(q, k, v, do, causal, window, scale),
             dtype, f"{mode} {shape} {dtype}")


@pytest.mark.parametrize("T,W", [(300, 64), (129, 1), (200, 128), (64, 200), (513, 256)])
def test_window_cases(T, W):
    q, k, v, do = _rand(1, T, 2, 1, 64, torch.float32, seed=W)
    _compare(_gpu(q, k, v, do, True, W), _ref(q, k, v, do, True, W), torch.float32,
             f"window T{T} W{W}")


def test_window_geq_seq_is_causal_bitwise():
    q, k, v, do = _rand(1, 100, 2, 2, 64, torch.bfloat16, seed=3)
    a = _gpu(q, k, v, do, True, 100)
    b = _gpu(q, k, v, do, True, 0)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_window_one_is_identity():
    q, k, v, do = _rand(1, 70, 2, 2, 32, torch.float32, seed=5)
    o = _gpu(q, k, v, do, True, 1)[0]
    assert np.abs(o - v.double().numpy()).max() < 1e-6


def _sample_heads(cfg, q, k, v, do, got, heads, rel_grad=None):
    """Oracle on selected (b, kv head) of a full-size run, with the kv head's whole
    group of query heads (GQA: query heads [hk*grp, (hk+1)*grp) share kv head hk)."""
    grp = cfg.H // cfg.Hkv
    for b, hk in heads:
        qs = slice(hk * grp, (hk + 1) * grp)
        kv = lambda t: t[b:b + 1, :, hk:hk + 1]
        qh = lambda t: t[b:b + 1, :, qs]
        ref = _ref(qh(q), kv(k), kv(v), qh(do), cfg.causal, cfg.window, cfg.scale, cfg.sinks)
        mine = [got[0][b:b + 1, :, qs], got[1][b:b + 1, qs],
                got[2][b:b + 1, :, qs], got[3][b:b + 1, :, hk:hk + 1],
                got[4][b:b + 1, :, hk:hk + 1]]
        _compare(mine, ref, cfg.dtype, f"{cfg.name} b{b} kvh{hk}", rel_grad)


def _invariants(cfg, q, k, do, got):
    """Size-independent checks on every head: sum_j dK_j = 0, sum_j dV_j = sum_i dO_i,
    sum_i <q_i, dQ_i> = sum_j <k_j, dK_j> (query sums taken over each GQA group)."""
    o, lse, dq, dk, dv = got
    B, S, H, D = dq.shape
    Hkv = dk.shape[2]
    grp = H // Hkv
    don = do.double().numpy().reshape(B, S, Hkv, grp, D)
    dos = don.sum(axis=(1, 3))                               # [B, Hkv, D]
    dvs = dv.sum(axis=1)
    scale_v = np.abs(don).sum(axis=(1, 3)).max() + 1e-30
    assert np.abs(dvs - dos).max() / scale_v < 1e-2, "sum dV != sum dO"
    dks = dk.sum(axis=1)
    scale_k = np.abs(dk).sum(axis=1).max() + 1e-30
    assert np.abs(dks).max() / scale_k < 1e-2, "sum dK != 0"
    # sum_i <q_i, dQ_i> = sum_j <k_j, dK_j> per (b, kv head): both equal scale * sum_ij
    # dS_ij q_i.k_j (the derivative of the loss along q -> (1+e) q equals that along
    # k -> (1+e) k).
    qd = (q.double().numpy() * dq).reshape(B, S, Hkv, grp, D)
    lhs = qd.sum(axis=(1, 3, 4))                              # [B, Hkv]
    rhs = (k.double().numpy() * dk).sum(axis=(1, 3))
    scale_qk = np.abs(qd).sum(axis=(1, 3, 4)).max() + 1e-30
    assert np.abs(lhs - rhs).max() / scale_qk < 1e-2, "sum <q, dQ> != sum <k, dK>"
    assert np.isfinite(o).all() and np.isfinite(lse).all()


# (batch, kv head) groups compared with the float64 oracle per full-size config: the
# corners, the middle, then seeded picks. The oracle's cost grows with S^2 * D, so the
# long config (S 8192, D 128) keeps two.
_N_HEADS = {"long": 2, "swa": 4, "recall": 4}


def _heads_of(cfg, n):
    B, Hk = cfg.B, cfg.Hkv
    picks = [(0, 0), (B - 1, Hk - 1), (B // 2, Hk // 2)]
    rng = np.random.default_rng(1000 + cfg.S + B)
    while len(set(picks)) < min(n, B * Hk):
        picks.append((int(rng.integers(B)), int(rng.integers(Hk))))
    return list(dict.fromkeys(picks))[:n]


@pytest.mark.parametrize("name", ["board", "board_do1", "swa", "swa_sinks", "long", "recall",
                                  "gqa"])
def test_baseline_configs_full_size(name):
    """Each BASELINE config at full size: the oracle on sampled heads, invariants on all.

    "board" keeps the config's dO ~ N(0, 1e-2) and adds the relative gradient bound
    (its gradients are ~1e-2, inside the absolute 2e-2); "board_do1" is the same
    shape and Q/K/V with dO ~ N(0, 1), where the absolute bound has teeth.
    """
    import dataclasses
    if name == "board_do1":
        cfg = dataclasses.replace(CONFIGS["board"], name="board_do1", do_std=1.0)
    else:
        cfg = CONFIGS[name]
    q, k, v, do = make_inputs(cfg)
    got = _gpu(q, k, v, do, cfg.causal, cfg.window, cfg.scale, sinks=cfg.sinks)
    _sample_heads(cfg, q, k, v, do, got, _heads_of(cfg, _N_HEADS.get(name, 8)),
                  rel_grad=_parity.REL_GRAD if name.startswith("board") else None)
    _invariants(cfg, q, k, do, got)


def _fp32_reference_all_heads(cfg, q, k, v, do):
    """Every head of a full-size config in float32 on the GPU: the north star's
    "fp32-upcast reference" (the same rounded 16-bit inputs, widened), forward
    and closed-form backward (Delta = rowsum(dO*O), dS = P*(dO V^T - Delta),
    dQ = scale dS K, dK = scale dS^T Q, dV = P^T dO, summed over each GQA group)
    under the oracle's visibility mask. A few kv heads at a time keep the
    [heads, S, S] score blocks near 256 MB."""
    B, S, H, D = q.shape
    Hkv = k.shape[2]
    grp = H // Hkv
    keep = torch.from_numpy(orc.visible_mask(S, cfg.causal, cfg.window, cfg.sinks,
                                             cfg.block)).cuda()
    qf, kf, vf, dof = (t.cuda().float() for t in (q, k, v, do))
    o = torch.empty_like(qf)
    lse = torch.empty(B, H, S, device="cuda")
    dq, dk, dv = torch.empty_like(qf), torch.empty_like(kf), torch.empty_like(vf)
    chunk = max(1, (1 << 26) // (grp * S * S))          # kv heads per block
    for b in range(B):
        for h0 in range(0, Hkv, chunk):
            h1 = min(Hkv, h0 + chunk)
            n = h1 - h0
            # [n, grp, S, D] query-side and [n, 1, S, D] key-side operands, contiguous.
            Q = qf[b, :, h0 * grp:h1 * grp].reshape(S, n, grp, D).permute(1, 2, 0, 3).contiguous()
            dO = dof[b, :, h0 * grp:h1 * grp].reshape(S, n, grp, D).permute(1, 2, 0, 3).contiguous()
            Kt = kf[b, :, h0:h1].permute(1, 0, 2).contiguous().unsqueeze(1)
            Vt = vf[b, :, h0:h1].permute(1, 0, 2).contiguous().unsqueeze(1)
            s = torch.matmul(Q, Kt.transpose(-1, -2).contiguous()) * cfg.scale
            s = s.masked_fill(~keep, float("-inf"))
            L = torch.logsumexp(s, dim=-1)
            p = torch.exp(s - L.unsqueeze(-1))
            O = torch.matmul(p, Vt)
            delta = (dO * O).sum(-1, keepdim=True)
            dp = torch.matmul(dO, Vt.transpose(-1, -2).contiguous())
            ds = p * (dp - delta)
            dQ = torch.matmul(ds, Kt) * cfg.scale
            dK = torch.matmul(ds.transpose(-1, -2).contiguous(), Q).sum(1) * cfg.scale
            dV = torch.matmul(p.transpose(-1, -2).contiguous(), dO).sum(1)
            o[b, :, h0 * grp:h1 * grp] = O.permute(2, 0, 1, 3).reshape(S, n * grp, D)
            lse[b, h0 * grp:h1 * grp] = L.reshape(n * grp, S)
            dq[b, :, h0 * grp:h1 * grp] = dQ.permute(2, 0, 1, 3).reshape(S, n * grp, D)
            dk[b, :, h0:h1] = dK.permute(1, 0, 2)
            dv[b, :, h0:h1] = dV.permute(1, 0, 2)
            del s, p, dp, ds
    torch.cuda.synchronize()
    return [t.double().cpu().numpy() for t in (o, lse, dq, dk, dv)]


@pytest.mark.parametrize("name", ["board", "board_do1", "swa", "swa_sinks", "long", "recall",
                                  "gqa", "board-f16", "swa-f16", "long-f16", "recall-f16",
                                  "gqa-f16"])
def test_baseline_configs_all_heads_fp32(name):
    """Each 16-bit BASELINE config at full size, every head and every element, against
    the float32 upcast reference computed on the GPU, at the same element-wise bound
    (and, at the board config, the same relative gradient bound) as the oracle checks.
    "-f16": the same workload with float16 inputs (the bound then carries float16's
    half-ulp)."""
    import dataclasses
    if name == "board_do1":
        cfg = dataclasses.replace(CONFIGS["board"], name="board_do1", do_std=1.0)
    elif name.endswith("-f16"):
        cfg = dataclasses.replace(CONFIGS[name[:-4]], dtype=torch.float16)
    else:
        cfg = CONFIGS[name]
    q, k, v, do = make_inputs(cfg)
    got = _gpu(q, k, v, do, cfg.causal, cfg.window, cfg.scale, sinks=cfg.sinks)
    ref = _fp32_reference_all_heads(cfg, q, k, v, do)
    torch.cuda.empty_cache()
    _compare(got, ref, cfg.dtype, f"allheads-fp32 {name}",
             rel_grad=_parity.REL_GRAD if name.startswith("board") else None)


def test_fp32_reference_matches_oracle():
    """The float32 GPU reference used above, against the float64 oracle on a small
    GQA window-with-sinks case: it must sit far inside the 16-bit bound it serves."""
    import dataclasses
    cfg = dataclasses.replace(CONFIGS["swa_sinks"], B=2, S=200, H=6, Hkv=2, window=37, sinks=3)
    q, k, v, do = _rand(cfg.B, cfg.S, cfg.H, cfg.Hkv, cfg.D, torch.bfloat16, seed=21)
    ref32 = _fp32_reference_all_heads(cfg, q, k, v, do)
    ref64 = _ref(q, k, v, do, cfg.causal, cfg.window, cfg.scale, cfg.sinks)
    for name, a, b in zip(("O", "LSE", "dQ", "dK", "dV"), ref32, ref64):
        assert np.abs(a - b).max() < 1e-4, f"fp32 reference {name} off the oracle"


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("jump", ["rescale", "overflow"])
def test_forward_late_max_jump(D, dtype, jump):
    """A key late in the row whose score towers over every earlier one, so the
    forward's lazy rescale must move the running max mid-row. "rescale": the jump is
    33-65 log2 units; "overflow": 143-295, past float32's exp2 range against the
    stale max, so a probability taken before the rescale would be infinite (the
    row's LSE then stays near 100-200, where float32 still resolves the 1e-4
    bound)."""
    B, T, H, Hkv = 1, 300, 2, 1
    g = torch.Generator().manual_seed(D + (7 if jump == "overflow" else 0))
    q = torch.randn(B, T, H, D, generator=g) * 0.3
    k = torch.randn(B, T, Hkv, D, generator=g) * 0.3
    v = torch.randn(B, T, Hkv, D, generator=g)
    do = torch.randn(B, T, H, D, generator=g)
    a = 16.0 if jump == "rescale" else 34.0
    q[:, 200:, 0, 0] = a          # head 0, queries 200.. : aligned with key 250 on dim 0
    k[:, 250, 0, 0] = a
    q, k, v, do = (t.to(dtype) for t in (q, k, v, do))
    scale = 1.0 / math.sqrt(D)
    _compare(_gpu(q, k, v, do, True, 0, scale), _ref(q, k, v, do, True, 0, scale), dtype,
             f"late max jump {jump} D{D} {dtype}")


def test_determinism_bitwise():
    q, k, v, do = _rand(2, 300, 4, 2, 64, torch.bfloat16, seed=11)
    a = _gpu(q, k, v, do, True, 0)
    b = _gpu(q, k, v, do, True, 0)
    for x, y in zip(a, b):
        assert np.array_equal(x, y), "not bitwise reproducible"


def test_lse_gradient():
    q, k, v, do = _rand(1, 90, 2, 1, 64, torch.float32, seed=2)
    w = torch.randn(1, 2, 90, generator=torch.Generator().manual_seed(9))
    qg, kg, vg = (t.cuda().requires_grad_() for t in (q, k, v))
    o, lse = fc.attn(qg, kg, vg, True, 0)
    loss = (o * do.cuda()).sum() + (lse * w.cuda()).sum()
    dq, dk, dv = torch.autograd.grad(loss, (qg, kg, vg))
    ro, rl = orc.forward(q, k, v, None, True, 0)
    rdq, rdk, rdv = orc.backward(q, k, v, ro, rl, do, None, True, 0, dlse=w)
    for a, b in zip((dq, dk, dv), (rdq, rdk, rdv)):
        assert np.abs(a.double().cpu().numpy() - b).max() < 1e-5


def test_positional_call_is_causal():
    q, k, v, do = _rand(1, 64, 2, 2, 64, torch.bfloat16)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    a = fc.flash_attn(qc, kc, vc, 0.125)
    b, _ = fc.attn(qc, kc, vc, True, 0, 0.125)
    assert torch.equal(a, b)


def test_use_mma_false_is_fp32_arithmetic():
    q, k, v, do = _rand(1, 100, 4, 2, 64, torch.bfloat16, seed=4)
    got = _gpu(q, k, v, do, True, 0, None, use_mma=False)
    ref = _ref(q, k, v, do, True, 0)
    # fp32 arithmetic on bf16 inputs: only the final bf16 rounding of outputs remains
    for a, b in zip(got, ref):
        assert np.abs(a - b).max() < 2e-2
    with pytest.raises(ValueError):
        fc.flash_attn(q.float().cuda(), k.float().cuda(), v.float().cuda(), use_mma=True)


def test_autocast_bridge_matches_sdpa():
    """fp32 q/k + bf16 v under autocast (nanolab/tests.py:470-482)."""
    B, T, H, Hkv, D = 2, 100, 4, 2, 32
    with torch.autocast("cuda", dtype=torch.bfloat16):
        q = torch.randn(B, T, H, D, device="cuda", requires_grad=True)
        k = torch.randn(B, T, Hkv, D, device="cuda", requires_grad=True)
        v = torch.randn(B, T, Hkv, D, device="cuda", dtype=torch.bfloat16, requires_grad=True)
        assert fc.supports(q, k, v)
        y = fc.flash_attn(q, k, v, 1.0 / math.sqrt(D))
        y_sdpa = fc.sdpa_reference(q, k, v, 1.0 / math.sqrt(D))
    assert y.dtype is torch.bfloat16
    assert (y.float() - y_sdpa.float()).abs().max() < 5e-2
    g = torch.autograd.grad(y.float().sum(), (q, k, v))
    assert g[0].dtype == torch.float32 and g[2].dtype == torch.bfloat16


def test_empty_inputs():
    q = torch.empty(0, 16, 2, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    o, lse = fc.attn(q, q, q, True, 0)
    assert o.shape == q.shape and lse.shape == (0, 2, 16)
    q = torch.empty(2, 0, 2, 64, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    o, lse = fc.attn(q, q, q, True, 0)
    (dq,) = torch.autograd.grad(o.sum(), (q,), allow_unused=True)
    assert o.shape == q.shape


def test_noncontiguous_inputs_are_normalised():
    q, k, v, do = _rand(1, 50, 4, 4, 64, torch.bfloat16, seed=8)
    qt = q.cuda().transpose(1, 2).contiguous().transpose(1, 2)   # same values, strided
    a = fc.flash_attn(qt, k.cuda(), v.cuda())
    b = fc.flash_attn(q.cuda(), k.cuda(), v.cuda())
    assert torch.equal(a, b)


@pytest.mark.parametrize("scale", [-0.2, 0.0])
def test_nonpositive_scale(scale):
    """scale <= 0 is legal at the Python boundary (mapped exactly onto scale > 0)."""
    q, k, v, do = _rand(1, 70, 2, 1, 64, torch.float32, seed=6)
    _compare(_gpu(q, k, v, do, True, 0, scale), _ref(q, k, v, do, True, 0, scale),
             torch.float32, f"scale {scale}")


# ---------------------------------------------------------------------------
# SWA(w, s): sliding window + StreamingLLM sinks (nanolab/mixers.py:96-135)
# ---------------------------------------------------------------------------
SINK_SHAPES = [  # (B, T, H, Hkv, D)
    (2, 100, 4, 2, 32),
    (1, 130, 4, 1, 64),
    (1, 257, 2, 2, 128),
    (2, 77, 8, 2, 64),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", SINK_SHAPES, ids=lambda s: "B%dT%dH%d/%dD%d" % s)
@pytest.mark.parametrize("ws", [(17, 4), (9, 8), (40, 1)], ids=lambda w: "W%dS%d" % w)
def test_sinks_small_shapes(shape, dtype, ws):
    B, T, H, Hkv, D = shape
    W, Sk = ws
    q, k, v, do = _rand(B, T, H, Hkv, D, dtype, seed=T + W)
    scale = 1.0 / math.sqrt(D)
    _compare(_gpu(q, k, v, do, True, W, scale, sinks=Sk),
             _ref(q, k, v, do, True, W, scale, sinks=Sk), dtype, f"sinks W{W} S{Sk} {shape} {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("ws", [(40, 32), (45, 33), (70, 64), (90, 65), (100, 4), (140, 128),
                                (200, 129), (280, 270), (400, 350)],
                         ids=lambda w: "W%dS%d" % w)
def test_sinks_fold_bound_16bit(dtype, D, ws):
    """The 16-bit window kernels visit the sinks themselves: the forward and dQ visit
    the ceil(sinks / 64) sink tiles before their ring (dQ skips 32-key halves past the
    last sink), and dK/dV's key blocks holding sinks walk every query tile. Both sides of
    the 32-key half and the 64-key tile bounds (32 / 33, 64 / 65, 128 / 129), a span of
    10 with 270 sinks (five sink tiles), sinks past the last key any row sees (W400 S350:
    span 50, so the kernels fold 250), and query blocks whose window does and does not
    reach the sink tiles (T = 300)."""
    W, Sk = ws
    q, k, v, do = _rand(2, 300, 4, 2, D, dtype, seed=W + Sk + D)
    scale = 1.0 / math.sqrt(D)
    _compare(_gpu(q, k, v, do, True, W, scale, sinks=Sk),
             _ref(q, k, v, do, True, W, scale, sinks=Sk), dtype, f"sinks W{W} S{Sk} D{D} {dtype}")


@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("ws", [(90, 65), (200, 129), (280, 270), (400, 350)],
                         ids=lambda w: "W%dS%d" % w)
def test_sinks_several_tiles_fp32(D, ws):
    """float32 visits the sink tiles the same way, in its own tile widths (64 keys in the
    forward, 32 in dQ and dK/dV): two to nine sink tiles, and sinks past the last key any
    row sees (W400 S350 at T 300: span 50, so rows see at most 250 of the 350 sinks)."""
    W, Sk = ws
    q, k, v, do = _rand(1, 300, 2, 1, D, torch.float32, seed=W + Sk + D)
    _compare(_gpu(q, k, v, do, True, W, sinks=Sk), _ref(q, k, v, do, True, W, sinks=Sk),
             torch.float32, f"sinks fp32 W{W} S{Sk} D{D}")


@pytest.mark.parametrize("T,W,S", [(300, 64, 4), (65, 64, 4), (128, 32, 1), (511, 64, 0),
                                   (200, 2, 1), (100, 97, 4), (129, 65, 64)])
def test_sinks_window_cases_fp32(T, W, S):
    """The reference's chunk-test (T, W, S) cases (nanolab/tests.py:3509-3535) and edges."""
    q, k, v, do = _rand(1, T, 2, 1, 64, torch.float32, seed=W + S)
    _compare(_gpu(q, k, v, do, True, W, sinks=S), _ref(q, k, v, do, True, W, sinks=S),
             torch.float32, f"sinks T{T} W{W} S{S}")


def test_sinks_zero_and_wide_window_are_bitwise():
    q, k, v, do = _rand(1, 100, 2, 2, 64, torch.bfloat16, seed=3)
    a = _gpu(q, k, v, do, True, 20, sinks=0)
    b = _gpu(q, k, v, do, True, 20)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    a = _gpu(q, k, v, do, True, 110, sinks=4)       # span 106 >= T: plain causal
    b = _gpu(q, k, v, do, True, 0)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_sinks_two_key_closed_form():
    """SWA(2, 1): query i sees exactly keys {0, i}."""
    q, k, v, do = _rand(1, 60, 2, 2, 32, torch.float32, seed=4)
    o = _gpu(q, k, v, do, True, 2, 0.3, sinks=1)[0]
    qn, kn, vn = (t.double().numpy() for t in (q, k, v))
    s0 = 0.3 * np.einsum("ihd,hd->ih", qn[0], kn[0, 0])
    si = 0.3 * np.einsum("ihd,ihd->ih", qn[0], kn[0])
    p0 = 1.0 / (1.0 + np.exp(si - s0))
    want = p0[..., None] * vn[0, 0][None] + (1 - p0[..., None]) * vn[0]
    want[0] = vn[0, 0]
    assert np.abs(o[0] - want).max() < 1e-5


def test_sinks_baseline_swa_config_sampled():
    """configs[2]'s shape (B8 H16 S4096 W256) with the reference's default 4 sinks."""
    import dataclasses
    cfg = dataclasses.replace(CONFIGS["swa"], name="swa+sinks4", sinks=4)
    q, k, v, do = make_inputs(cfg)
    got = _gpu(q, k, v, do, True, cfg.window, cfg.scale, sinks=4)
    _sample_heads(cfg, q, k, v, do, got, [(0, 0), (cfg.B - 1, cfg.H - 1)])
    _invariants(cfg, q, k, do, got)


def test_sinks_determinism_and_lse_gradient():
    q, k, v, do = _rand(2, 300, 8, 2, 64, torch.bfloat16, seed=11)
    a = _gpu(q, k, v, do, True, 64, sinks=4)
    b = _gpu(q, k, v, do, True, 64, sinks=4)
    assert all(np.array_equal(x, y) for x, y in zip(a, b)), "not bitwise reproducible"
    q, k, v, do = _rand(1, 90, 2, 1, 64, torch.float32, seed=2)
    w = torch.randn(1, 2, 90, generator=torch.Generator().manual_seed(9))
    qg, kg, vg = (t.cuda().requires_grad_() for t in (q, k, v))
    o, lse = fc.attn(qg, kg, vg, True, 16, sinks=3)
    loss = (o * do.cuda()).sum() + (lse * w.cuda()).sum()
    dq, dk, dv = torch.autograd.grad(loss, (qg, kg, vg))
    ro, rl = orc.forward(q, k, v, None, True, 16, sinks=3)
    rdq, rdk, rdv = orc.backward(q, k, v, ro, rl, do, None, True, 16, dlse=w, sinks=3)
    assert np.abs(lse.detach().double().cpu().numpy() - rl).max() < 1e-4
    for x, y in zip((dq, dk, dv), (rdq, rdk, rdv)):
        assert np.abs(x.double().cpu().numpy() - y).max() < 1e-5


# Sink keys collect a whole column: every row from the key on sees them, with P of
# order 1 / span on each row, so their dV (P^T dO) and dK (dS'^T Q) sum one 16-bit
# operand rounding per row over the whole sequence, beside the output's own rounding.
# The dK/dV waves that hold sink keys split P and dS' into hi + lo (SSPLIT in
# csrc/attn_bwd16.hip). Regression cases at the configs' scale 1/sqrt(D), end to end
# against the exact oracle (its own O and LSE) with the plain bound, no operand
# allowance: the seeded sweep's case c187 of seed 82 (B2 T237 H2/1 D64 bf16, SWA(6, 1),
# an LSE gradient; its dV read 1.098 of the bound before the split) and long rows with
# 1 and 4 sinks at D 32 / 64 / 128.
SINK_COLUMN_CASES = [  # (B, T, H, Hkv, D, dtype, window, sinks, seed, with_dlse)
    (2, 237, 2, 1, 64, torch.bfloat16, 6, 1, 287, True),
    (1, 1024, 2, 1, 64, torch.bfloat16, 64, 1, 21, False),
    (1, 1100, 4, 2, 64, torch.bfloat16, 64, 4, 22, True),
    (1, 1024, 2, 2, 32, torch.float16, 16, 4, 23, False),
    (1, 1030, 2, 1, 128, torch.bfloat16, 40, 4, 24, True),
    (2, 2048, 2, 1, 64, torch.bfloat16, 8, 4, 25, False),
]


@pytest.mark.parametrize("case", SINK_COLUMN_CASES,
                         ids=lambda c: "B%dT%dH%d/%dD%d-%s-W%dS%d" % (c[:5] + (str(c[5])[6:], c[6], c[7])))
def test_sink_key_columns_plain_bound(case):
    B, T, H, Hkv, D, dtype, W, S, seed, with_dlse = case
    q, k, v, do = _rand(B, T, H, Hkv, D, dtype, seed=seed)
    # The sweep draws the LSE gradient with seed 7 + i for input seed 100 + i.
    wl = torch.randn(B, H, T, generator=torch.Generator().manual_seed(seed - 93)) * 0.3
    qg, kg, vg = (t.detach().cuda().requires_grad_() for t in (q, k, v))
    o, lse = fc.attn(qg, kg, vg, True, W, None, sinks=S)
    loss = (o.float() * do.cuda().float()).sum()
    if with_dlse:
        loss = loss + (lse * wl.cuda()).sum()
    dq, dk, dv = torch.autograd.grad(loss, (qg, kg, vg))
    torch.cuda.synchronize()
    sc = 1.0 / math.sqrt(D)
    qr, kr, vr, dor = (t.double().numpy() for t in (q, k, v, do))
    ro, rl = orc.forward(qr, kr, vr, sc, True, W, sinks=S)
    rdq, rdk, rdv = orc.backward(qr, kr, vr, ro, rl, dor, sc, True, W,
                                 dlse=wl.double().numpy() if with_dlse else None, sinks=S)
    tag = f"sink columns B{B} T{T} H{H}/{Hkv} D{D} {dtype} W{W} S{S} dlse={with_dlse}"
    for name, a, b in zip(("O", "LSE", "dQ", "dK", "dV"), (o, lse, dq, dk, dv),
                          (ro, rl, rdq, rdk, rdv)):
        _parity.check(tag, name, a.detach().double().cpu().numpy(), b, dtype)


def test_sinks_argument_errors():
    q = torch.randn(1, 16, 2, 64, device="cuda", dtype=torch.bfloat16)
    for kw in ({"window": 8, "sinks": 8}, {"window": 0, "sinks": 2}, {"window": 8, "sinks": -1}):
        with pytest.raises(ValueError, match="sinks"):
            fc.attn(q, q, q, True, kw["window"], sinks=kw["sinks"])
    fc.flash_attn(q, q, q, causal=True, window=8, sinks=7)


# ---------------------------------------------------------------------------
# Gated attention: y = O * sigmoid(gate), the per-head output gate of
# nanolab/mixers.py:340-344 applied inside the kernel
# ---------------------------------------------------------------------------
def _gate_logits(B, T, H, seed):
    return torch.randn(B, T, H, generator=torch.Generator().manual_seed(seed)) * 2.0


def _gpu_gated(q, k, v, do, z, causal=True, window=0, scale=None, sinks=0):
    qg, kg, vg, zg = (t.detach().cuda().requires_grad_() for t in (q, k, v, z))
    y, lse = fc.attn(qg, kg, vg, causal, window, scale, sinks=sinks, gate=zg)
    dq, dk, dv, dz = torch.autograd.grad(y, (qg, kg, vg, zg), do.cuda())
    torch.cuda.synchronize()
    return [t.detach().double().cpu().numpy() for t in (y, lse, dq, dk, dv, dz)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 100, 4, 2, 32), (1, 130, 4, 1, 64), (1, 77, 2, 2, 128)],
                         ids=lambda s: "B%dT%dH%d/%dD%d" % s)
@pytest.mark.parametrize("mode", ["causal", "window+sinks", "noncausal"])
def test_gated_parity(shape, dtype, mode):
    B, T, H, Hkv, D = shape
    q, k, v, do = _rand(B, T, H, Hkv, D, dtype, seed=T + 7)
    z = _gate_logits(B, T, H, seed=T)
    causal = mode != "noncausal"
    window, sinks = (24, 3) if mode == "window+sinks" else (0, 0)
    scale = 1.0 / math.sqrt(D)
    got = _gpu_gated(q, k, v, do, z, causal, window, scale, sinks)
    y, lse = orc.forward_gated(q, k, v, z, scale, causal, window, sinks)
    dq, dk, dv, dz = orc.backward_gated(q, k, v, z, y, lse, do, scale, causal, window,
                                        sinks=sinks)
    _compare(got[:5], [y, lse, dq, dk, dv], dtype, f"gated {mode} {shape} {dtype}")
    _parity.check(f"gated {mode} {shape} {dtype}", "dgate", got[5], dz, dtype)


def test_gated_stage_entry_points_match_full_backward():
    """delta_gated + dkdv + dq (stage entry points) == mi_attn_bwd_gated, bit for bit."""
    import ctypes
    from machinelearning_amd import _capi
    lib = _capi.load()
    B, T, H, D = 2, 200, 4, 64
    q, k, v, do = (t.cuda() for t in _rand(B, T, H, H, D, torch.bfloat16, seed=1))
    z = _gate_logits(B, T, H, 2).cuda()
    shp = _capi.shape(B, T, H, H, D, True, 0, 0.125, _capi.MI_BF16)
    sp = ctypes.byref(shp)
    st = torch.cuda.current_stream().cuda_stream
    P = lambda t: t.data_ptr()
    o = torch.empty_like(q)
    lse = torch.empty(B, H, T, device="cuda")
    assert lib.mi_attn_fwd_gated(P(q), P(k), P(v), P(z), P(o), P(lse), sp, st) == 0
    outs = []
    for full in (True, False):
        ws = torch.empty(_capi.workspace_floats(shp), device="cuda")
        doa, dz = torch.empty_like(do), torch.empty_like(z)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        if full:
            assert lib.mi_attn_bwd_gated(P(q), P(k), P(v), P(z), P(o), P(do), P(lse), None,
                                         P(ws), P(doa), P(dq), P(dk), P(dv), P(dz), sp, st) == 0
        else:
            assert lib.mi_attn_bwd_delta_gated(P(o), P(do), P(z), P(lse), None, P(ws), P(doa),
                                               P(dz), sp, st) == 0
            assert lib.mi_attn_bwd_dkdv(P(q), P(k), P(v), P(doa), P(lse), P(ws), P(dk), P(dv),
                                        sp, st) == 0
            assert lib.mi_attn_bwd_dq(P(q), P(k), P(v), P(doa), P(lse), P(ws), P(dq), sp, st) == 0
        torch.cuda.synchronize()
        outs.append([dq, dk, dv, dz, doa])
    assert all(torch.equal(a, b) for a, b in zip(*outs))


@pytest.mark.parametrize("case", ["causal", "dlse", "sinks", "gqa", "f16_denormal_do"])
def test_stage_entry_points_match_full_backward(case):
    """mi_attn_bwd (16-bit: the delta pass fused into dQ, dQ before dK/dV) against the
    stage entry points (delta, then dK/dV, then dQ). The -L/scale plane is the same
    expression, bit for bit; Delta sums the same products in another order (relative
    1e-6); the gradients then agree to one bf16 ulp of each tensor's maximum.
    f16_denormal_do: dO ~ N(0, 1e-4) in float16, about half of it subnormal (below
    2^-14), so a fused Delta that flushed subnormal inputs would miss the bound."""
    import ctypes
    from machinelearning_amd import _capi
    lib = _capi.load()
    B, T, H, Hkv, D, window, sinks = 2, 200, 4, 4, 64, 0, 0
    dt, mdt = torch.bfloat16, _capi.MI_BF16
    if case == "gqa":
        Hkv = 1
    if case == "sinks":
        window, sinks = 48, 4
    if case == "f16_denormal_do":
        dt, mdt = torch.float16, _capi.MI_F16
    q, k, v, do = (t.cuda() for t in _rand(B, T, H, Hkv, D, dt, seed=3))
    if case == "f16_denormal_do":
        do = (do.float() * 1e-4).to(dt)
        sub = (do != 0) & (do.abs() < 2.0 ** -14)
        assert float(sub.float().mean()) > 0.3
    shp = _capi.shape(B, T, H, Hkv, D, True, window, 0.125, mdt, sinks)
    sp = ctypes.byref(shp)
    st = torch.cuda.current_stream().cuda_stream
    P = lambda t: None if t is None else t.data_ptr()
    o = torch.empty_like(q)
    lse = torch.empty(B, H, T, device="cuda")
    assert lib.mi_attn_fwd(P(q), P(k), P(v), P(o), P(lse), sp, st) == 0
    dlse = (0.3 * torch.randn(B, H, T, generator=torch.Generator().manual_seed(4))).cuda() \
        if case == "dlse" else None
    outs = []
    for full in (True, False):
        ws = torch.empty(_capi.workspace_floats(shp), device="cuda")
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        if full:
            assert lib.mi_attn_bwd(P(q), P(k), P(v), P(o), P(do), P(lse), P(dlse), P(ws),
                                   P(dq), P(dk), P(dv), sp, st) == 0
        else:
            assert lib.mi_attn_bwd_delta(P(o), P(do), P(lse), P(dlse), P(ws), sp, st) == 0
            assert lib.mi_attn_bwd_dkdv(P(q), P(k), P(v), P(do), P(lse), P(ws), P(dk), P(dv),
                                        sp, st) == 0
            assert lib.mi_attn_bwd_dq(P(q), P(k), P(v), P(do), P(lse), P(ws), P(dq), sp, st) == 0
        torch.cuda.synchronize()
        outs.append([dq.float(), dk.float(), dv.float(), ws[: 2 * B * H * T].view(2, -1)])
    (fq, fk, fv, fws), (sq, sk, sv, sws) = outs
    assert torch.equal(fws[1], sws[1]), "-L/scale plane"
    rel = ((fws[0] - sws[0]).abs().max() / sws[0].abs().max().clamp_min(1e-30)).item()
    assert rel < 1e-6, f"Delta plane: relative difference {rel:.2e}"
    for name, a, b in (("dQ", fq, sq), ("dK", fk, sk), ("dV", fv, sv)):
        amax = float(b.abs().max())
        ulp = 2.0 ** (math.floor(math.log2(amax)) - 7) if amax > 0 else 0.0
        err = float((a - b).abs().max())
        print(f"{case} {name}: max|full - staged| = {err:.3e} (1 ulp at max {ulp:.1e})", flush=True)
        assert err <= ulp, f"{case} {name}: {err:.3e} > {ulp:.1e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D,sinks", [(128, 0), (64, 0), (128, 5), (32, 0)])
def test_output_residual_entry_points(dtype, D, sinks):
    """mi_attn_fwd_res writes mi_attn_fwd's o and lse bit for bit, plus o_res, the
    rounding residual of each output element (at most half an ulp of o there);
    mi_attn_bwd_res's Delta plane is rowsum(dO * (o + o_res)), not rowsum(dO * o)
    (checked in float64 to 1e-6 of the plane's scale, where the residual's share is
    ~1e-3), and its gradients pass the oracle bound."""
    import ctypes
    from machinelearning_amd import _capi
    lib = _capi.load()
    B, T, H, Hkv = 2, 333, 4, 2
    window = 40 if sinks else 0
    mdt = _capi.MI_BF16 if dtype == torch.bfloat16 else _capi.MI_F16
    q, k, v, do = _rand(B, T, H, Hkv, D, dtype, seed=D + sinks)
    qc, kc, vc, doc = (t.cuda() for t in (q, k, v, do))
    scale = 1.0 / math.sqrt(D)
    shp = _capi.shape(B, T, H, Hkv, D, True, window, scale, mdt, sinks)
    sp = ctypes.byref(shp)
    st = torch.cuda.current_stream().cuda_stream
    P = lambda t: None if t is None else t.data_ptr()
    o, o2, o_res = torch.empty_like(qc), torch.empty_like(qc), torch.empty_like(qc)
    lse, lse2 = torch.empty(B, H, T, device="cuda"), torch.empty(B, H, T, device="cuda")
    assert lib.mi_attn_fwd(P(qc), P(kc), P(vc), P(o), P(lse), sp, st) == 0
    assert lib.mi_attn_fwd_res(P(qc), P(kc), P(vc), P(o2), P(o_res), P(lse2), sp, st) == 0
    torch.cuda.synchronize()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    on, rn = o.double().cpu().numpy(), o_res.double().cpu().numpy()
    assert (np.abs(rn) <= _parity.half_ulp(on, dtype) + 1e-30).all(), "residual beyond half an ulp"
    assert np.count_nonzero(rn) > rn.size // 2
    ws = torch.empty(_capi.workspace_floats(shp), device="cuda")
    dq, dk, dv = torch.empty_like(qc), torch.empty_like(kc), torch.empty_like(vc)
    assert lib.mi_attn_bwd_res(P(qc), P(kc), P(vc), P(o), P(o_res), P(doc), P(lse), None, P(ws),
                               P(dq), P(dk), P(dv), sp, st) == 0
    torch.cuda.synchronize()
    dplane = ws[: B * H * T].view(B, H, T).double().cpu().numpy()
    don = do.double().numpy()
    want = (don * (on + rn)).sum(-1).transpose(0, 2, 1)                 # [B, H, T]
    plain = (don * on).sum(-1).transpose(0, 2, 1)
    dscale = np.abs(want).max()
    print(f"D{D} sinks{sinks} {dtype}: Delta vs rowsum(dO*(o+res)) "
          f"{np.abs(dplane - want).max() / dscale:.2e}, residual share "
          f"{np.abs(want - plain).max() / dscale:.2e}", flush=True)
    assert np.abs(dplane - want).max() / dscale < 1e-6
    assert np.abs(want - plain).max() / dscale > 1e-5
    got = [on, lse.double().cpu().numpy()] + [t.double().cpu().numpy() for t in (dq, dk, dv)]
    _compare(got, _ref(q, k, v, do, True, window, scale, sinks), dtype,
             f"residual D{D} sinks{sinks} {dtype}")


def test_output_residual_refusals():
    """The residual entry points refuse float32 and a NULL o_res before any launch;
    the autograd op keeps the residual at RESIDUAL_HEAD_DIMS, and with sinks that
    rows see beyond their span."""
    import ctypes
    from machinelearning_amd import _capi
    lib = _capi.load()
    P = lambda t: None if t is None else t.data_ptr()
    st = torch.cuda.current_stream().cuda_stream
    x = torch.zeros(1, 130, 2, 128, device="cuda", dtype=torch.bfloat16)
    lse = torch.empty(1, 2, 130, device="cuda")
    for dtc, sinks, res, code in ((_capi.MI_F32, 0, x, 12), (_capi.MI_F32, 65, x, 12),
                                  (_capi.MI_BF16, 0, None, 1)):
        shp = _capi.shape(1, 130, 2, 2, 128, True, 100 if sinks else 0, 0.1, dtc, sinks)
        sp = ctypes.byref(shp)
        assert lib.mi_attn_fwd_res(P(x), P(x), P(x), P(x), P(res), P(lse), sp, st) == code
        assert lib.mi_attn_bwd_res(P(x), P(x), P(x), P(x), P(res), P(x), P(lse), None, P(lse),
                                   P(x), P(x), P(x), sp, st) == code
    assert "residual" in lib.mi_attn_error_string(12).decode()
    q = torch.zeros(1, 8, 2, 128, dtype=torch.bfloat16)
    assert fc._wants_residual(q, 0, None) and fc._wants_residual(q, 65, None, 100)
    assert not fc._wants_residual(q[..., :64], 0, None)
    assert not fc._wants_residual(q.float(), 0, None)
    # Folded sinks that rows see beyond their span keep the residual at every D.
    q = torch.zeros(1, 64, 2, 64, dtype=torch.bfloat16)
    assert fc._wants_residual(q, 4, None, 20) and fc._wants_residual(q[..., :32], 1, None, 64)
    assert not fc._wants_residual(q, 4, None, 68)          # span 64 covers S = 64
    assert fc._wants_residual(q, 65, None, 100)            # folded at any count
    assert not fc._wants_residual(q, 4, torch.zeros(1, 64, 2), 20)   # gated


def test_gate_zero_halves_the_output_and_bad_gate_shapes_raise():
    q, k, v, do = _rand(1, 90, 2, 2, 64, torch.float32, seed=12)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    y, _ = fc.attn(qc, kc, vc, True, 0, gate=torch.zeros(1, 90, 2, device="cuda"))
    o, _ = fc.attn(qc, kc, vc, True, 0)
    assert torch.allclose(y, 0.5 * o, atol=1e-6, rtol=0)
    y4 = fc.flash_attn(qc, kc, vc, causal=True, gate=torch.zeros(1, 90, 2, 1, device="cuda"))
    assert torch.equal(y4, y)
    with pytest.raises(ValueError, match="gate"):
        fc.attn(qc, kc, vc, True, 0, gate=torch.zeros(1, 90, 3, device="cuda"))


# ---------------------------------------------------------------------------
# Block-causal (semi-autoregressive / diffusion) masks, nanolab/mixers.py:76-93
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(2, 100, 4, 2, 32), (1, 130, 4, 1, 64), (1, 77, 2, 2, 128)],
                         ids=lambda s: "B%dT%dH%d/%dD%d" % s)
@pytest.mark.parametrize("block", [7, 16, 64, 100])
def test_block_causal_parity(shape, dtype, block):
    B, T, H, Hkv, D = shape
    q, k, v, do = _rand(B, T, H, Hkv, D, dtype, seed=T + block)
    scale = 1.0 / math.sqrt(D)
    qg, kg, vg = (t.detach().cuda().requires_grad_() for t in (q, k, v))
    o, lse = fc.attn(qg, kg, vg, True, 0, scale, block=block)
    dq, dk, dv = torch.autograd.grad(o, (qg, kg, vg), do.cuda())
    got = [t.detach().double().cpu().numpy() for t in (o, lse, dq, dk, dv)]
    ro, rl = orc.forward(q, k, v, scale, True, 0, block=block)
    rdq, rdk, rdv = orc.backward(q, k, v, ro, rl, do, scale, True, 0, block=block)
    _compare(got, [ro, rl, rdq, rdk, rdv], dtype, f"block{block} {shape} {dtype}")


def test_block_one_is_causal_and_block_geq_seq_is_bidirectional():
    q, k, v, do = _rand(1, 90, 2, 2, 64, torch.bfloat16, seed=8)
    qc, kc, vc = q.cuda(), k.cuda(), v.cuda()
    a, la = fc.attn(qc, kc, vc, True, 0, block=1)
    b, lb = fc.attn(qc, kc, vc, True, 0)
    assert torch.equal(a, b) and torch.equal(la, lb)
    c, lc = fc.attn(qc, kc, vc, True, 0, block=128)
    d, ld = fc.attn(qc, kc, vc, False, 0)
    assert (c.float() - d.float()).abs().max().item() < 1e-2
    assert (lc - ld).abs().max().item() < 1e-4
    with pytest.raises(ValueError, match="block"):
        fc.attn(qc, kc, vc, False, 0, block=4)
    with pytest.raises(ValueError, match="block"):
        fc.attn(qc, kc, vc, True, 16, block=4)


def test_block_causal_board_shape_with_gate():
    """Board shape, 64-position blocks (a diffusion block), gated, sampled heads."""
    import dataclasses
    cfg = CONFIGS["board"]
    q, k, v, do = make_inputs(dataclasses.replace(cfg, do_std=1.0))
    z = _gate_logits(cfg.B, cfg.S, cfg.H, seed=4)
    qg, kg, vg, zg = (t.detach().cuda().requires_grad_() for t in (q, k, v, z))
    y, lse = fc.attn(qg, kg, vg, True, 0, cfg.scale, gate=zg, block=64)
    grads = torch.autograd.grad(y, (qg, kg, vg, zg), do.cuda())
    for b, h in ((0, 0), (cfg.B - 1, cfg.H - 1)):
        sl = lambda t: t[b:b + 1, :, h:h + 1]
        ro, rl = orc.forward(sl(q), sl(k), sl(v), cfg.scale, True, 0, block=64)
        sg = 1 / (1 + np.exp(-z[b:b + 1, :, h:h + 1].double().numpy()))
        ry = ro * sg[..., None]
        rdq, rdk, rdv = orc.backward(sl(q), sl(k), sl(v), ro, rl, sl(do).double().numpy() * sg[..., None],
                                     cfg.scale, True, 0, block=64)
        mine = [y[b:b + 1, :, h:h + 1], lse[b:b + 1, h:h + 1]] + [g[b:b + 1, :, h:h + 1] for g in grads[:3]]
        _compare([t.detach().double().cpu().numpy() for t in mine], [ry, rl, rdq, rdk, rdv],
                 cfg.dtype, f"board block64 gated b{b} h{h}")


# ---------------------------------------------------------------------------
# Seeded sweep over random shapes and masks (ragged lengths, odd head counts,
# every mask kind, custom scales, an LSE gradient), each against the oracle.
# ---------------------------------------------------------------------------
def _sweep_cases(n=None, seed=None, tmax=None):
    """Seeded random cases. The defaults (24 cases, seed 2026, T up to 300) are the
    suite's; MI_SWEEP_N / MI_SWEEP_SEED / MI_SWEEP_TMAX widen a one-off run."""
    n = int(os.environ.get("MI_SWEEP_N", 24)) if n is None else n
    seed = int(os.environ.get("MI_SWEEP_SEED", 2026)) if seed is None else seed
    tmax = int(os.environ.get("MI_SWEEP_TMAX", 300)) if tmax is None else tmax
    rng = np.random.default_rng(seed)
    heads = [(1, 1), (2, 1), (4, 2), (6, 3), (8, 2)]
    dtypes = [torch.float32, torch.bfloat16, torch.float16]
    cases = []
    for i in range(n):
        B = int(rng.integers(1, 4))
        T = int(rng.integers(1, tmax + 1))
        H, Hkv = heads[int(rng.integers(len(heads)))]
        D = int(rng.choice([32, 64, 128]))
        dtype = dtypes[i % 3]
        kind = ["causal", "noncausal", "window", "block"][int(rng.integers(4))]
        causal, window, sinks, block = kind != "noncausal", 0, 0, 0
        if kind == "window":
            window = int(rng.integers(1, T + 11))
            sinks = int(rng.integers(0, window)) if rng.random() < 0.5 else 0
        if kind == "block":
            block = int(rng.integers(2, T + 6))
        scale = None if rng.random() < 0.5 else float(rng.uniform(0.05, 0.5))
        with_dlse = bool(rng.random() < 0.5)
        cases.append((B, T, H, Hkv, D, dtype, causal, window, sinks, block, scale, with_dlse, i))
    return cases


@pytest.mark.parametrize("case", _sweep_cases(), ids=lambda c: "c%d" % c[-1])
def test_random_shape_and_mask_sweep(case):
    B, T, H, Hkv, D, dtype, causal, window, sinks, block, scale, with_dlse, i = case
    q, k, v, do = _rand(B, T, H, Hkv, D, dtype, seed=100 + i)
    wl = torch.randn(B, H, T, generator=torch.Generator().manual_seed(7 + i)) * 0.3
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    qg, kg, vg = (t.detach().cuda().requires_grad_() for t in (q, k, v))
    o, lse = fc.attn(qg, kg, vg, causal, window, scale, sinks=sinks, block=block)
    loss = (o.float() * do.cuda().float()).sum()
    if with_dlse:
        loss = loss + (lse * wl.cuda()).sum()
    dq, dk, dv = torch.autograd.grad(loss, (qg, kg, vg))
    torch.cuda.synchronize()
    got = [t.detach().double().cpu().numpy() for t in (o, lse, dq, dk, dv)]
    qr, kr, vr, dor = (t.double().numpy() for t in (q, k, v, do))
    ro, rl = orc.forward(qr, kr, vr, sc, causal, window, sinks=sinks, block=block)
    dl = wl.double().numpy() if with_dlse else None
    # The backward entry point computes Delta = rowsum(dO * O) from the O the forward
    # stored (rounded to the input dtype), as the reference's backward does
    # (flash_attn_cuda.cu:1231-1262 reads the saved O), or, where the op keeps the
    # output's rounding residual (16-bit D = 128, or sinks beyond the span), from o + o_res:
    # the float32 O before rounding, which still carries the 16-bit P of the PV
    # product. Its gradients are checked against the oracle backward given that same
    # O (the forward is deterministic: the residual run's o is the autograd op's bit
    # for bit). At the configs' own scale (scale None) the bound is the plain one,
    # 2e-2 plus half an output ulp, for that comparison and end to end against the
    # exact oracle. At the raised scales of this sweep (up to 0.5: a sharper
    # softmax, gradients up to ~20) it adds
    # the 16-bit MMA operands' rounding allowance: P and dS, rounded as the
    # reference's kernels round them (pack_a_from_acc, cu:945 and cu:1153-1154),
    # move each gradient element by up to u * sum|terms| (u = 2^-8 bf16, 2^-11 f16:
    # one rounding per term; the oracle's magnitudes). Logged beside the asserts:
    # the plain ratios, the oracle that emulates the operand rounding (mma-operands)
    # and the end-to-end comparison with the exact O (e2e-plain).
    o_stored = got[0]
    uses_res = dtype != torch.float32 and fc._wants_residual(q, sinks, None, window)
    if uses_res:
        o2, _, o_res = fc._fwd(qg.detach(), kg.detach(), vg.detach(), causal, window, sinks, sc,
                               None, block, residual=True)
        torch.cuda.synchronize()
        assert np.array_equal(o2.double().cpu().numpy(), o_stored)
        o_bwd = o_stored + o_res.double().cpu().numpy()
    else:
        o_bwd = o_stored
    rq, rk, rv = orc.backward(qr, kr, vr, o_bwd, rl, dor, sc, causal, window, dlse=dl,
                              sinks=sinks, block=block)
    eq, ek, ev = orc.backward(qr, kr, vr, ro, rl, dor, sc, causal, window, dlse=dl,
                              sinks=sinks, block=block)
    tag = (f"sweep c{i}: B{B} T{T} H{H}/{Hkv} D{D} {dtype} causal={causal} w={window} "
           f"s={sinks} block={block} scale={scale} dlse={with_dlse}")

    def logged(tag_, name, a, b):
        err = np.abs(a - b)
        ratio = float((err / _parity.tol16(b, dtype)).max()) if b.size else 0.0
        print(f"{tag_} {name} (logged): worst err/tol={ratio:.3f}", flush=True)
        _parity.record(tag_, name, max_err=float(err.max()) if b.size else 0.0,
                       worst_ratio=ratio, max_ref=float(np.abs(b).max()) if b.size else 0.0,
                       rel_err=0.0, dtype=str(dtype), asserted=False)

    extra = {}
    if dtype != torch.float32:
        kind = "bfloat16" if dtype == torch.bfloat16 else "float16"
        mq, mk, mv = orc.backward(qr, kr, vr, o_bwd, rl, dor, sc, causal, window, dlse=dl,
                                  sinks=sinks, block=block, operand_dtype=kind)
        for name, a, b in zip(("dQ", "dK", "dV"), got[2:], (mq, mk, mv)):
            logged(tag + " mma-operands", name, a, b)
        u = 2.0 ** (-8 if dtype == torch.bfloat16 else -11)
        sums = orc.backward(qr, kr, vr, o_bwd, rl, dor, sc, causal, window, dlse=dl,
                            sinks=sinks, block=block, magnitudes=True)
        allowance = {n: u * m for n, m in zip(("dQ", "dK", "dV"), sums)}
        # At the configs' own scale (scale None: 1/sqrt(D)) both comparisons are
        # asserted with the plain bound, end to end against the exact oracle and
        # against the oracle given the stored O, sinks of any count included (the
        # 16-bit window kernels fold them, with split sink-key operands in dK/dV).
        # The raised scales (up to 0.5: a sharper softmax, gradients up to ~20) keep
        # the allowance on every gradient. The plain ratios are logged either way.
        for name, a, b in zip(("dQ", "dK", "dV"), got[2:], (eq, ek, ev)):
            logged(tag + " e2e-plain", name, a, b)
            if scale is None:
                _parity.check(tag + " e2e", name, a, b, dtype)
        for name, a, b in zip(("dQ", "dK", "dV"), got[2:], (rq, rk, rv)):
            logged(tag + " plain", name, a, b)
        extra = {} if scale is None else allowance
    # Tolerances as in _compare, except that float32's 1e-5 is taken relative to the
    # tensor's magnitude once that exceeds 1: the random scales here (up to 0.5,
    # against 1/sqrt(D) = 0.09-0.18 in the configs) lift gradients to ~10, where
    # fp32 arithmetic is good to ~1e-6 relative, not 1e-5 absolute.
    for name, a, b in zip(("O", "LSE", "dQ", "dK", "dV"), got, [ro, rl, rq, rk, rv]):
        if dtype == torch.float32 and name != "LSE" and b.size:
            amax = float(np.abs(b).max())
            err = float(np.abs(a - b).max()) if a.size else 0.0
            tol = 1e-5 * max(1.0, amax)
            print(f"{tag} {name}: max|err|={err:.3e} tol={tol:.1e} max|ref|={amax:.3e}", flush=True)
            _parity.record(tag, name, max_err=err, worst_ratio=err / tol, max_ref=amax,
                           rel_err=err / amax if amax else 0.0, dtype="float32")
            assert err < tol, f"{tag}: {name} max|err| {err:.3e} >= {tol:.1e}"
        else:
            _parity.check(tag, name, a, b, dtype, extra=extra.get(name))

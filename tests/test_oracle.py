"""Pin the float64 oracle before it is trusted as the GPU kernels' checker.

Each check is independent of the oracle's own formulas, and chosen so a
plausible mistake (dropped scale, wrong mask edge, transposed operand, missing
GQA sum, sign error in dS) fails at least one of them -- ``test_planted_*``
demonstrates that on the CPU by planting such mistakes and watching the checks
fail.

Reference tests mirrored (bharathvbcr/MachineLearning): the brute force vs
autograd at 1e-12 (``nanolab/tests.py:252-293``), shapes with odd T and GQA
groups 1/2/4 (``tests.py:265-267,321-323``), the window mask position by
position (``tests.py:2993-3018``), window >= T == causal (``tests.py:3021-3052``)
and chunked == dense window (``tests.py:3509-3535``).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as orc
from oracle import cpu_path


def _rand(B, T, H, Hkv, D, seed=0):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*s, generator=g, dtype=torch.float64)
            for s in ((B, T, H, D), (B, T, Hkv, D), (B, T, Hkv, D), (B, T, H, D))]


def _torch_autograd(q, k, v, do, scale, causal, window, dlse=None):
    """Independent derivation: autograd through an SDPA-math-style torch forward."""
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
    T = q.shape[1]
    group = q.shape[2] // k.shape[2]
    qs = qa.permute(0, 2, 1, 3)
    ks = ka.repeat_interleave(group, dim=2).permute(0, 2, 1, 3)
    vs = va.repeat_interleave(group, dim=2).permute(0, 2, 1, 3)
    s = (qs @ ks.transpose(-1, -2)) * scale
    # The mask is built here from the definition, not borrowed from the oracle.
    pos = torch.arange(T)
    keep = torch.ones(T, T, dtype=torch.bool)
    if causal:
        keep = torch.ones(T, T, dtype=torch.bool).tril()
    if window:
        keep = keep & ((pos[:, None] - pos[None, :]) < window)
    s = s.masked_fill(~keep, -math.inf)
    lse = torch.logsumexp(s, dim=-1)
    o = (torch.softmax(s, dim=-1) @ vs).permute(0, 2, 1, 3)
    loss = (o * do).sum()
    if dlse is not None:
        loss = loss + (lse * dlse).sum()
    loss.backward()
    return o.detach(), lse.detach(), qa.grad, ka.grad, va.grad


CASES = [  # (B, T, H, Hkv, D, causal, window)
    (2, 100, 4, 2, 32, True, 0),
    (1, 37, 2, 2, 32, True, 0),
    (1, 33, 2, 1, 32, True, 0),
    (1, 64, 4, 1, 64, True, 0),
    (1, 80, 2, 1, 128, True, 0),
    (2, 50, 4, 2, 32, False, 0),
    (1, 90, 4, 4, 32, True, 16),
    (1, 70, 4, 1, 32, True, 1),
]


@pytest.mark.parametrize("case", CASES)
def test_forward_and_closed_form_backward_match_autograd(case):
    B, T, H, Hkv, D, causal, window = case
    q, k, v, do = _rand(B, T, H, Hkv, D, seed=T)
    scale = 1.0 / math.sqrt(D)
    o, lse = orc.forward(q, k, v, scale, causal, window)
    dq, dk, dv = orc.backward(q, k, v, o, lse, do, scale, causal, window)
    to, tl, tdq, tdk, tdv = _torch_autograd(q, k, v, do, scale, causal, window)
    for a, b in ((o, to), (lse, tl), (dq, tdq), (dk, tdk), (dv, tdv)):
        assert np.abs(a - b.numpy()).max() < 1e-12


def test_lse_gradient_matches_autograd():
    q, k, v, do = _rand(1, 40, 2, 1, 32, seed=4)
    w = torch.randn(1, 2, 40, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    o, lse = orc.forward(q, k, v, None, True, 0)
    dq, dk, dv = orc.backward(q, k, v, o, lse, do, None, True, 0, dlse=w)
    _, _, tdq, tdk, tdv = _torch_autograd(q, k, v, do, 1 / math.sqrt(32), True, 0, dlse=w)
    for a, b in ((dq, tdq), (dk, tdk), (dv, tdv)):
        assert np.abs(a - b.numpy()).max() < 1e-12


@pytest.mark.parametrize("causal", [True, False])
def test_forward_matches_sdpa_math_backend(causal):
    q, k, v, _ = _rand(2, 45, 4, 4, 64, seed=7)
    o, _ = orc.forward(q, k, v, 0.3, causal, 0)
    with torch.nn.attention.sdpa_kernel(torch.nn.attention.SDPBackend.MATH):
        ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2),
                                             v.transpose(1, 2), is_causal=causal, scale=0.3)
    assert np.abs(o - ref.transpose(1, 2).numpy()).max() < 1e-12


def test_forward_matches_python_triple_loop():
    """Brute force with plain Python loops on a tiny case (independent of numpy matmul)."""
    q, k, v, _ = _rand(1, 6, 2, 1, 4, seed=3)
    scale, W = 0.7, 3
    o, lse = orc.forward(q, k, v, scale, True, W)
    for h in range(2):
        for i in range(6):
            keys = [j for j in range(6) if j <= i and j > i - W]
            s = [scale * sum(float(q[0, i, h, d]) * float(k[0, j, 0, d]) for d in range(4))
                 for j in keys]
            m = max(s)
            z = sum(math.exp(x - m) for x in s)
            assert abs(lse[0, h, i] - (m + math.log(z))) < 1e-12
            for d in range(4):
                want = sum(math.exp(x - m) / z * float(v[0, j, 0, d]) for x, j in zip(s, keys))
                assert abs(o[0, i, h, d] - want) < 1e-12


def test_window_mask_position_by_position():
    """nanolab/tests.py:2993-3018 with sinks=0: row q sees {k: q-w < k <= q}."""
    T, w = 12, 5
    m = orc.visible_mask(T, True, w)
    for q in range(T):
        want = {k for k in range(q + 1) if k > q - w}
        got = {k for k in range(T) if m[q, k]}
        assert got == want and len(got) <= w and got
    assert int(m[T - 1].sum()) == w and not m[T - 1, 0]


def test_invariants():
    q, k, v, do = _rand(2, 77, 4, 2, 32, seed=21)
    scale = 0.2
    for causal, window in ((True, 0), (False, 0), (True, 9)):
        o, lse = orc.forward(q, k, v, scale, causal, window)
        dq, dk, dv = orc.backward(q, k, v, o, lse, do, scale, causal, window)
        keep = orc.visible_mask(77, causal, window)
        # rows of P sum to 1 and LSE >= max score
        qn, kn = q.numpy(), k.numpy()
        for b in range(2):
            for h in range(4):
                s = np.where(keep, (qn[b, :, h] @ kn[b, :, h // 2].T) * scale, -np.inf)
                p = np.exp(s - lse[b, h][:, None])
                assert np.abs(p.sum(1) - 1).max() < 1e-12
                assert (lse[b, h] >= s.max(1) - 1e-12).all()
        # sum over keys of dV == sum over queries (of the group) of dO; sum_j dK_j == 0
        dos = do.numpy().sum(1).reshape(2, 2, 2, 32).sum(2)
        assert np.abs(dv.sum(1) - dos).max() < 1e-10
        assert np.abs(dk.sum(1)).max() < 1e-10


def test_special_cases():
    q, k, v, _ = _rand(1, 1, 2, 2, 32, seed=1)
    o, lse = orc.forward(q, k, v, 0.5, True, 0)                    # S == 1
    assert np.abs(o - v.numpy()).max() < 1e-12
    assert np.abs(lse[0, :, 0] - 0.5 * (q[0, 0] * k[0, 0]).sum(-1).numpy()).max() < 1e-12
    q, k, v, _ = _rand(1, 20, 2, 2, 32, seed=2)
    o, lse = orc.forward(q, k, v, 0.5, True, 0)
    assert np.abs(o[0, 0] - v[0, 0].numpy()).max() < 1e-12       # causal row 0
    o, lse = orc.forward(torch.zeros_like(q), k, v, 0.5, True, 0)   # Q == 0
    cm = np.cumsum(v.numpy(), axis=1) / np.arange(1, 21)[None, :, None, None]
    assert np.abs(o - cm).max() < 1e-12
    assert np.abs(lse - np.log(np.arange(1, 21))[None, None]).max() < 1e-12
    o, _ = orc.forward(q, k, v, 0.5, True, 1)                      # window 1
    assert np.abs(o - v.numpy()).max() < 1e-12
    a = orc.forward(q, k, v, 0.5, True, 20)                        # window >= S
    b = orc.forward(q, k, v, 0.5, True, 0)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_delta_matches_rowsum():
    q, k, v, do = _rand(1, 30, 2, 1, 32, seed=5)
    o, lse = orc.forward(q, k, v, None, True, 0)
    d = orc.delta(o, do)
    assert np.abs(d - (o * do.numpy()).sum(-1).transpose(0, 2, 1)).max() < 1e-14


def test_flops_formula():
    # The published algorithmic figures: board config 90.28 GFLOP fwd+bwd, 25.80 fwd.
    from machinelearning_amd import perf
    assert abs(perf.flops(16, 12, 1024, 64) / 1e9 - 90.28) < 0.01
    assert abs(perf.flops(16, 12, 1024, 64, bwd=False) / 1e9 - 25.80) < 0.01
    assert abs(perf.flops(8, 16, 4096, 64, True, 256) / 1e9 - 116.52) < 0.01
    assert abs(perf.flops(2, 16, 8192, 128) / 1e9 - 1924.38) < 0.01
    assert abs(perf.flops(32, 8, 2048, 64, False) / 1e9 - 962.07) < 0.01
    # N_vis by brute force over the mask
    for S, causal, W in ((37, True, 0), (37, False, 0), (100, True, 9), (10, True, 20)):
        assert perf.nvis(S, causal, W) == int(orc.visible_mask(S, causal, W).sum())


# ---- the CPU baseline path (the reference's mixer path restated) ----
@pytest.mark.parametrize("T,W", [(512, 64), (511, 64), (300, 64), (65, 64), (128, 32)])
def test_cpu_path_window_matches_oracle(T, W):
    g = torch.Generator().manual_seed(T + W)
    q, k, v = (torch.randn(1, T, 2, 16, generator=g) for _ in range(3))
    got = cpu_path.cpu_attention(q, k, v, 0.25, True, W)
    want, _ = orc.forward(q, k, v, 0.25, True, W)
    assert np.abs(got.numpy() - want).max() < 1e-5


def test_cpu_path_chunk_rule():
    """nanolab/tests.py:3509-3535's expectations for the chunking rule."""
    assert cpu_path.swa_auto_chunk(2048, 64) == 256 and cpu_path.swa_auto_chunk(2048, 512) == 512
    assert cpu_path.swa_auto_chunk(512, 64) == 256
    assert cpu_path.swa_auto_chunk(512, 256) == 0
    assert cpu_path.swa_auto_chunk(63, 64) == 0
    assert cpu_path.swa_auto_chunk(4096, 256) == 256


@pytest.mark.parametrize("causal", [True, False])
def test_cpu_path_gqa_matches_oracle(causal):
    g = torch.Generator().manual_seed(3)
    q = torch.randn(2, 40, 4, 32, generator=g)
    k, v = (torch.randn(2, 40, 2, 32, generator=g) for _ in range(2))
    got = cpu_path.cpu_attention(q, k, v, 0.2, causal)
    want, _ = orc.forward(q, k, v, 0.2, causal)
    assert np.abs(got.numpy() - want).max() < 1e-5


# ---- planted mistakes: each must be caught by the checks above ----
def _checks_pass(fwd, bwd) -> bool:
    q, k, v, do = _rand(1, 33, 4, 2, 32, seed=13)
    scale = 1 / math.sqrt(32)
    try:
        for causal, window in ((True, 0), (True, 7), (False, 0)):
            o, lse = fwd(q, k, v, scale, causal, window)
            dq, dk, dv = bwd(q, k, v, o, lse, do, scale, causal, window)
            to, tl, tdq, tdk, tdv = _torch_autograd(q, k, v, do, scale, causal, window)
            for a, b in ((o, to), (lse, tl), (dq, tdq), (dk, tdk), (dv, tdv)):
                if not np.abs(a - b.numpy()).max() < 1e-9:
                    return False
    except Exception:
        return False
    return True


def test_planted_mistakes_are_caught(monkeypatch):
    assert _checks_pass(orc.forward, orc.backward)

    # 1. off-by-one window edge (k >= q - w instead of k > q - w)
    def bad_mask(S, causal=True, window=0, sinks=0, block=0):
        i, j = np.arange(S)[:, None], np.arange(S)[None, :]
        keep = np.ones((S, S), bool)
        if causal:
            keep &= j <= i
        if window:
            keep &= j >= i - window
        return keep
    monkeypatch.setattr(orc, "visible_mask", bad_mask)
    assert not _checks_pass(orc.forward, orc.backward)
    monkeypatch.undo()

    # 2. dropped scale in dK
    def bwd_noscale(q, k, v, o, lse, do, scale, causal, window):
        dq, dk, dv = orc.backward(q, k, v, o, lse, do, scale, causal, window)
        return dq, dk / scale, dv
    assert not _checks_pass(orc.forward, bwd_noscale)

    # 3. sign error in dS (p * (Delta - dP))
    def bwd_sign(q, k, v, o, lse, do, scale, causal, window):
        dq, dk, dv = orc.backward(q, k, v, o, lse, do, scale, causal, window)
        return -dq, -dk, dv
    assert not _checks_pass(orc.forward, bwd_sign)

    # 4. GQA: KV head chosen as h % Hkv instead of h // group
    def fwd_badgqa(q, k, v, scale, causal, window):
        perm = [h % k.shape[2] for h in range(q.shape[2])]
        kk = torch.stack([k[:, :, p] for p in perm], 2)
        vv = torch.stack([v[:, :, p] for p in perm], 2)
        return orc.forward(q, kk, vv, scale, causal, window)
    assert not _checks_pass(fwd_badgqa, orc.backward)


# ---- SWA(w, s): the sliding window with StreamingLLM sinks ----
def _sink_keep(T, w, s):
    """Keep-mask straight from the set definition of nanolab/tests.py:2993-3018."""
    keep = torch.zeros(T, T, dtype=torch.bool)
    for q in range(T):
        want = {k for k in range(q + 1) if k > q - (w - s)} | {k for k in range(min(s, q + 1))}
        for k in want:
            keep[q, k] = True
    return keep


def _torch_autograd_mask(q, k, v, do, scale, keep, dlse=None):
    qa, ka, va = (t.clone().requires_grad_() for t in (q, k, v))
    group = q.shape[2] // k.shape[2]
    qs = qa.permute(0, 2, 1, 3)
    ks = ka.repeat_interleave(group, dim=2).permute(0, 2, 1, 3)
    vs = va.repeat_interleave(group, dim=2).permute(0, 2, 1, 3)
    s = ((qs @ ks.transpose(-1, -2)) * scale).masked_fill(~keep, -math.inf)
    lse = torch.logsumexp(s, dim=-1)
    o = (torch.softmax(s, dim=-1) @ vs).permute(0, 2, 1, 3)
    loss = (o * do).sum()
    if dlse is not None:
        loss = loss + (lse * dlse).sum()
    loss.backward()
    return o.detach(), lse.detach(), qa.grad, ka.grad, va.grad


def test_sink_mask_position_by_position():
    """nanolab/tests.py:2993-3018: SWA(5, 2) on T = 12, row by row."""
    T, w, s = 12, 5, 2
    m = orc.visible_mask(T, True, w, s)
    for q in range(T):
        want = {k for k in range(q + 1) if k > q - (w - s)} | {k for k in range(min(s, q + 1))}
        got = {k for k in range(T) if m[q, k]}
        assert got == want, (q, sorted(got), sorted(want))
        assert not any(m[q, k] for k in range(q + 1, T))
        assert len(got) <= w and got
    nosink = orc.visible_mask(T, True, w, 0)
    assert m[T - 1, 0] and not nosink[T - 1, 0]
    assert int(nosink[T - 1].sum()) == w
    for bad in ((5, 5), (5, -1), (0, 2)):
        with pytest.raises(ValueError):
            orc.visible_mask(T, True, *bad)


SINK_CASES = [  # (B, T, H, Hkv, D, window, sinks)
    (1, 90, 4, 2, 32, 16, 4),
    (1, 70, 2, 1, 32, 5, 4),          # span 1: only the diagonal besides the sinks
    (2, 50, 2, 2, 64, 60, 3),         # window >= T
    (1, 41, 4, 1, 32, 12, 11),
    (1, 33, 2, 2, 32, 2, 1),
]


@pytest.mark.parametrize("case", SINK_CASES)
def test_sinks_forward_and_backward_match_autograd(case):
    B, T, H, Hkv, D, w, s = case
    q, k, v, do = _rand(B, T, H, Hkv, D, seed=T + s)
    scale = 1.0 / math.sqrt(D)
    dl = torch.randn(B, H, T, generator=torch.Generator().manual_seed(2), dtype=torch.float64)
    o, lse = orc.forward(q, k, v, scale, True, w, sinks=s)
    dq, dk, dv = orc.backward(q, k, v, o, lse, do, scale, True, w, dlse=dl, sinks=s)
    ref = _torch_autograd_mask(q, k, v, do, scale, _sink_keep(T, w, s), dlse=dl)
    for a, b in zip((o, lse, dq, dk, dv), ref):
        assert np.abs(a - b.numpy()).max() < 1e-12


def test_sinks_forward_matches_python_triple_loop():
    q, k, v, _ = _rand(1, 9, 2, 1, 4, seed=8)
    scale, W, Sk = 0.6, 4, 2
    o, lse = orc.forward(q, k, v, scale, True, W, sinks=Sk)
    for h in range(2):
        for i in range(9):
            keys = [j for j in range(9) if j <= i and (j > i - (W - Sk) or j < Sk)]
            s = [scale * sum(float(q[0, i, h, d]) * float(k[0, j, 0, d]) for d in range(4))
                 for j in keys]
            m = max(s)
            z = sum(math.exp(x - m) for x in s)
            assert abs(lse[0, h, i] - (m + math.log(z))) < 1e-12
            for d in range(4):
                want = sum(math.exp(x - m) / z * float(v[0, j, 0, d]) for x, j in zip(s, keys))
                assert abs(o[0, i, h, d] - want) < 1e-12


def test_sinks_special_cases():
    q, k, v, do = _rand(1, 40, 2, 2, 32, seed=12)
    # window >= S: the sinks are inside the span already -> plain causal
    a = orc.forward(q, k, v, 0.3, True, 45, sinks=4)
    b = orc.forward(q, k, v, 0.3, True, 0)
    assert all(np.abs(x - y).max() < 1e-12 for x, y in zip(a, b))
    # sinks = 0 is the plain window
    a = orc.forward(q, k, v, 0.3, True, 9, sinks=0)
    b = orc.forward(q, k, v, 0.3, True, 9)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))
    # SWA(2, 1): query i sees exactly {0, i} -> a two-key softmax in closed form
    o, lse = orc.forward(q, k, v, 0.3, True, 2, sinks=1)
    qn, kn, vn = q.numpy(), k.numpy(), v.numpy()
    for i in range(1, 40):
        s0 = 0.3 * (qn[0, i, 1] * kn[0, 0, 1]).sum()
        si = 0.3 * (qn[0, i, 1] * kn[0, i, 1]).sum()
        p0 = 1.0 / (1.0 + math.exp(si - s0))
        assert np.abs(o[0, i, 1] - (p0 * vn[0, 0, 1] + (1 - p0) * vn[0, i, 1])).max() < 1e-12
    # invariants hold with sinks as well
    o, lse = orc.forward(q, k, v, 0.3, True, 7, sinks=3)
    dq, dk, dv = orc.backward(q, k, v, o, lse, do, 0.3, True, 7, sinks=3)
    assert np.abs(dv.sum(1) - do.numpy().sum(1)).max() < 1e-10
    assert np.abs(dk.sum(1)).max() < 1e-10


@pytest.mark.parametrize("T,W,S", [(2048, 64, 4), (2048, 512, 4), (512, 64, 4), (511, 64, 0),
                                   (300, 64, 4), (65, 64, 4), (128, 32, 1)])
def test_cpu_path_chunked_sinks_is_the_dense_window(T, W, S):
    """nanolab/tests.py:3509-3535's seven (T, W, S) cases: chunked == dense, < 1e-5."""
    c = cpu_path.swa_auto_chunk(T, W) or 128
    g = torch.Generator().manual_seed(T + W)
    q, k, v = (torch.randn(2, 3, T, 16, generator=g) for _ in range(3))
    ref = F.scaled_dot_product_attention(q, k, v, attn_mask=_sink_keep(T, W, S), scale=0.25)
    got = cpu_path.swa_chunked(q, k, v, W, 0.25, c, S)
    assert (got - ref).abs().max().item() < 1e-5


@pytest.mark.parametrize("T,W,S", [(300, 64, 4), (65, 64, 4), (129, 16, 15)])
def test_cpu_path_sinks_match_oracle(T, W, S):
    g = torch.Generator().manual_seed(T)
    q, k, v = (torch.randn(1, T, 2, 16, generator=g) for _ in range(3))
    got = cpu_path.cpu_attention(q, k, v, 0.25, True, W, S)
    want, _ = orc.forward(q, k, v, 0.25, True, W, sinks=S)
    assert np.abs(got.numpy() - want).max() < 1e-5


def test_sink_flop_count_is_the_mask_count():
    from machinelearning_amd import perf
    for S, W, Sk in ((100, 9, 4), (100, 9, 8), (10, 9, 4), (10, 12, 4), (37, 2, 1), (64, 64, 3),
                     (1024, 64, 4)):
        assert perf.nvis(S, True, W, Sk) == int(orc.visible_mask(S, True, W, Sk).sum()), (S, W, Sk)


def test_planted_sink_mistakes_are_caught(monkeypatch):
    """An off-by-one sink edge (k <= s) or a span of w instead of w - s must fail the checks."""
    def checks_pass():
        q, k, v, do = _rand(1, 30, 2, 1, 32, seed=3)
        for w, s in ((8, 3), (5, 4)):
            o, lse = orc.forward(q, k, v, 0.2, True, w, sinks=s)
            dq, dk, dv = orc.backward(q, k, v, o, lse, do, 0.2, True, w, sinks=s)
            ref = _torch_autograd_mask(q, k, v, do, 0.2, _sink_keep(30, w, s))
            if not all(np.abs(a - b.numpy()).max() < 1e-9 for a, b in zip((o, lse, dq, dk, dv), ref)):
                return False
        return True

    assert checks_pass()
    real = orc.visible_mask

    def edge(S, causal=True, window=0, sinks=0, block=0):
        keep = real(S, causal, window, 0)
        j, i = np.arange(S)[None, :], np.arange(S)[:, None]
        return keep | ((j <= sinks) & (j <= i)) if sinks else keep
    monkeypatch.setattr(orc, "visible_mask", edge)
    assert not checks_pass()

    def wide(S, causal=True, window=0, sinks=0, block=0):
        keep = real(S, causal, window, 0)
        j, i = np.arange(S)[None, :], np.arange(S)[:, None]
        return keep | ((j < sinks) & (j <= i)) if sinks else keep
    monkeypatch.setattr(orc, "visible_mask", wide)
    assert not checks_pass()


# ---- gated attention (per-head sigmoid output gate, nanolab/mixers.py:340-344) ----
@pytest.mark.parametrize("window,sinks", [(0, 0), (9, 3)])
def test_gated_forward_and_backward_match_autograd(window, sinks):
    q, k, v, do = _rand(2, 40, 4, 2, 32, seed=31)
    z = torch.randn(2, 40, 4, generator=torch.Generator().manual_seed(3), dtype=torch.float64)
    scale = 1 / math.sqrt(32)
    keep = _sink_keep(40, window, sinks) if window else torch.ones(40, 40, dtype=torch.bool).tril()
    qa, ka, va, za = (t.clone().requires_grad_() for t in (q, k, v, z))
    qs = qa.permute(0, 2, 1, 3)
    ks = ka.repeat_interleave(2, dim=2).permute(0, 2, 1, 3)
    vs = va.repeat_interleave(2, dim=2).permute(0, 2, 1, 3)
    s = ((qs @ ks.transpose(-1, -2)) * scale).masked_fill(~keep, -math.inf)
    o = (torch.softmax(s, dim=-1) @ vs).permute(0, 2, 1, 3)
    y = o * torch.sigmoid(za)[..., None]
    (y * do).sum().backward()
    gy, glse = orc.forward_gated(q, k, v, z, scale, True, window, sinks)
    dq, dk, dv, dz = orc.backward_gated(q, k, v, z, gy, glse, do, scale, True, window, sinks=sinks)
    for a, b in ((gy, y.detach()), (dq, qa.grad), (dk, ka.grad), (dv, va.grad), (dz, za.grad)):
        assert np.abs(a - b.numpy()).max() < 1e-12


# ---- block-causal (semi-autoregressive) masks, nanolab/mixers.py:76-93 ----
def test_block_causal_mask_structure():
    """nanolab/tests.py:853-864: block 1 == causal, block >= T == everywhere,
    bidirectional inside a block, causal across blocks."""
    T = 6
    assert np.array_equal(orc.visible_mask(T, True, 0, 0, 1), np.tril(np.ones((T, T), bool)))
    assert orc.visible_mask(T, True, 0, 0, T).all()
    b = orc.visible_mask(T, True, 0, 0, 2)
    assert b[1, 0] and b[0, 1] and b[2, 1] and not b[1, 2]
    # row by row against the set definition for a ragged last block
    m = orc.visible_mask(11, True, 0, 0, 4)
    for q in range(11):
        assert {k for k in range(11) if m[q, k]} == set(range(min(11, (q // 4 + 1) * 4)))
    with pytest.raises(ValueError):
        orc.visible_mask(8, False, 0, 0, 4)


@pytest.mark.parametrize("T,L", [(37, 4), (50, 16), (33, 33), (20, 1)])
def test_block_causal_matches_autograd(T, L):
    q, k, v, do = _rand(1, T, 4, 2, 32, seed=T + L)
    keep = torch.zeros(T, T, dtype=torch.bool)
    for qq in range(T):
        keep[qq, : min(T, (qq // L + 1) * L)] = True
    o, lse = orc.forward(q, k, v, 0.2, True, 0, block=L)
    dq, dk, dv = orc.backward(q, k, v, o, lse, do, 0.2, True, 0, block=L)
    ref = _torch_autograd_mask(q, k, v, do, 0.2, keep)
    for a, b in zip((o, lse, dq, dk, dv), ref):
        assert np.abs(a - b.numpy()).max() < 1e-12


def test_block_causal_flop_count_is_the_mask_count():
    from machinelearning_amd import perf
    for S, L in ((100, 7), (64, 64), (1024, 64), (37, 40), (12, 1)):
        assert perf.nvis(S, True, 0, 0, L) == int(orc.visible_mask(S, True, 0, 0, L).sum())


# --------------------------------------------------------------------------- MMA operand rounding
@pytest.mark.parametrize("kind,tdt", [("bfloat16", torch.bfloat16), ("float16", torch.float16)])
def test_round_operand_matches_torch_conversion(kind, tdt):
    """round_operand against torch's own float32 -> 16-bit conversion: random values over
    a wide exponent range, exact ties with even and odd kept bits, float32 subnormals, and
    the largest finite values (which round to inf for bfloat16 beyond its range)."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(50000) * np.exp2(rng.integers(-30, 30, 50000))).astype(np.float32)
    ties = (rng.integers(0x00800000, 0x7F000000, 4000, dtype=np.uint64) & ~np.uint64(0xFFFF)) | 0x8000
    sub = rng.integers(1, 0x007FFFFF, 2000, dtype=np.uint64)
    big = np.array([0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF, 0x477FE000, 0x477FF000], dtype=np.uint64)
    bits = np.concatenate([ties, sub, big]).astype(np.uint32)
    x = np.concatenate([x, bits.view(np.float32), -bits.view(np.float32)])
    if kind == "float16":
        x = x[np.abs(x) < 65504]          # torch and numpy agree on overflow; keep finite
    got = orc.round_operand(x, kind)
    want = torch.from_numpy(x).to(tdt).double().numpy()
    assert np.array_equal(got, want, equal_nan=False), int((got != want).sum())


def test_rounded_operand_backward_matches_a_torch_restatement():
    """backward(operand_dtype=...) against torch float64 that rounds P and dS with torch's
    bfloat16 / float16 conversion before the dQ, dK and dV products; without
    operand_dtype it is the plain backward bit for bit."""
    B, T, H, Hkv, D = 2, 37, 4, 2, 32
    q, k, v, do = _rand(B, T, H, Hkv, D, seed=11)
    sc = 0.4
    o, lse = orc.forward(q, k, v, sc, True, 0)
    plain = orc.backward(q, k, v, o, lse, do, sc, True, 0)
    same = orc.backward(q, k, v, o, lse, do, sc, True, 0, operand_dtype=None)
    assert all(np.array_equal(a, b) for a, b in zip(plain, same))
    keep = torch.from_numpy(orc.visible_mask(T, True))
    for kind, tdt in (("bfloat16", torch.bfloat16), ("float16", torch.float16)):
        got = orc.backward(q, k, v, o, lse, do, sc, True, 0, operand_dtype=kind)
        rq, rk, rv = (np.zeros_like(t) for t in (q, k, v))
        for b in range(B):
            for h in range(H):
                hk = h // (H // Hkv)
                qh, kh, vh, doh = (torch.from_numpy(np.ascontiguousarray(t)) for t in
                                   (q[b, :, h], k[b, :, hk], v[b, :, hk], do[b, :, h]))
                oh = torch.from_numpy(np.ascontiguousarray(o[b, :, h]))
                p = torch.where(keep, torch.exp(qh @ kh.T * sc - torch.from_numpy(lse[b, h])[:, None]),
                                torch.zeros(()))
                ds = p * (doh @ vh.T - (doh * oh).sum(1)[:, None])
                pr, dsr = p.float().to(tdt).double(), ds.float().to(tdt).double()
                rq[b, :, h] = (sc * dsr @ kh).numpy()
                rk[b, :, hk] += (sc * dsr.T @ qh).numpy()
                rv[b, :, hk] += (pr.T @ doh).numpy()
        for a, r in zip(got, (rq, rk, rv)):
            np.testing.assert_allclose(a, r, rtol=1e-12, atol=1e-12)
        # the rounding is visible: bfloat16 operands move the gradients by ~2^-9 relative
        assert max(float(np.abs(a - p_).max()) for a, p_ in zip(got, plain)) > 1e-6


def test_gradient_term_magnitudes():
    """backward(magnitudes=True): per gradient element the sum of |terms|, checked
    against a pure-Python loop on a tiny case; it bounds |gradient| (triangle
    inequality) and equals it when every term is non-negative."""
    B, T, H, Hkv, D = 1, 6, 2, 1, 3
    q, k, v, do = (t.numpy() for t in _rand(B, T, H, Hkv, D, seed=3))
    sc = 0.7
    o, lse = orc.forward(q, k, v, sc, True, 0)
    mq, mk, mv = orc.backward(q, k, v, o, lse, do, sc, True, 0, magnitudes=True)
    gq, gk, gv = orc.backward(q, k, v, o, lse, do, sc, True, 0)
    for m, g in ((mq, gq), (mk, gk), (mv, gv)):
        assert (m >= np.abs(g) - 1e-12).all()
    # pure-Python sums of |terms| (dS and P from the same closed form, element by element)
    for h in range(H):
        P = [[0.0] * T for _ in range(T)]
        dS = [[0.0] * T for _ in range(T)]
        for i in range(T):
            dl = sum(do[0, i, h, d] * o[0, i, h, d] for d in range(D))
            for j in range(i + 1):
                s = sc * sum(q[0, i, h, d] * k[0, j, 0, d] for d in range(D))
                P[i][j] = math.exp(s - lse[0, h, i])
                dp = sum(do[0, i, h, d] * v[0, j, 0, d] for d in range(D))
                dS[i][j] = P[i][j] * (dp - dl)
        for i in range(T):
            for d in range(D):
                want = sc * sum(abs(dS[i][j]) * abs(k[0, j, 0, d]) for j in range(T))
                assert abs(mq[0, i, h, d] - want) < 1e-12
    # dV's terms p_ij * dO_i are all non-negative when dO is: then the sums coincide
    dpos = np.abs(do)
    mv2 = orc.backward(q, k, v, o, lse, dpos, sc, True, 0, magnitudes=True)[2]
    gv2 = orc.backward(q, k, v, o, lse, dpos, sc, True, 0)[2]
    np.testing.assert_allclose(mv2, gv2, rtol=1e-13, atol=1e-15)

"""KV-cached decode step: oracle pinning on the CPU, the C ABI's host checks,
and parity of the HIP kernels (through ``mi_attn_decode``) on the GPU.

Reference: ``Attention.forward_cached`` (``nanolab/mixers.py:372-467``) and
its callers (``nanolab/diffusion.py:304-490``, ``nanolab/reason.py:340-375``).
Tolerances as for the attention op: float32 within 1e-5 max-abs on the
output, LSE within 1e-4; 16-bit inputs within 2e-2 of the float64 oracle
evaluated on the same rounded inputs, element by element, plus the output
format's half-ulp at that element (``tests/_parity.py``).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import attention as orc
from oracle import decode as ord_
from tests import _parity


def _rand(B, S, H, Hkv, D, seed=0):
    g = np.random.default_rng(seed)
    return (g.standard_normal((B, S, H, D)), g.standard_normal((B, S, Hkv, D)),
            g.standard_normal((B, S, Hkv, D)))


# ---------------------------------------------------------------- oracle pins (CPU)
def test_step_mask_closed_forms():
    keep, _ = ord_.step_mask(3, 4, causal=True)
    want = np.concatenate([np.ones((4, 3), bool), np.tril(np.ones((4, 4), bool))], axis=1)
    assert np.array_equal(keep, want)
    assert ord_.step_mask(5, 2, causal=False)[0].all()
    # window, no eviction: the same as the full SWA mask's rows start .. start+T-1
    keep, kpos = ord_.step_mask(6, 3, True, window=4, sinks=1)
    full = orc.visible_mask(9, True, 4, 1)
    assert np.array_equal(keep, full[6:9, :9]) and np.array_equal(kpos, np.arange(9))
    with pytest.raises(ValueError, match="causal"):
        ord_.step_mask(0, 4, causal=False, window=8)


@pytest.mark.parametrize("blocks", [[5, 1, 7, 3, 16], [1] * 12, [24]])
def test_causal_cached_blocks_equal_causal_attention(blocks):
    S = sum(blocks)
    q, k, v = _rand(2, S, 4, 2, 32, seed=len(blocks))
    y, sizes = ord_.decode_blocks(q, k, v, blocks, causal=True)
    o, _ = orc.forward(q, k, v, None, True)
    assert np.abs(y - o).max() < 1e-12
    assert sizes == list(np.cumsum(blocks))


@pytest.mark.parametrize("L", [1, 4, 8])
def test_bidirectional_cached_blocks_equal_block_causal(L):
    """The cache invariant block diffusion rests on (nanolab/diffusion.py:331)."""
    S = 6 * L
    q, k, v = _rand(1, S, 4, 4, 32, seed=L)
    y, _ = ord_.decode_blocks(q, k, v, [L] * 6, causal=False)
    o, _ = orc.forward(q, k, v, None, True, block=L)
    assert np.abs(y - o).max() < 1e-12


def test_swa_cached_decode_matches_the_uncached_window():
    """Shape of nanolab/tests.py:3420-3455: W, S, BLK, T = 12, 3, 8, 48."""
    W, SK, BLK, T = 12, 3, 8, 48
    q, k, v = _rand(1, T, 4, 2, 32, seed=7)
    y, sizes = ord_.decode_blocks(q, k, v, [BLK] * (T // BLK), True, W, SK)
    o, _ = orc.forward(q, k, v, None, True, W, sinks=SK)
    assert np.abs(y - o).max() < 1e-12
    assert all(z <= W - 1 for z in sizes), sizes
    assert sizes[-1] == sizes[-2], sizes


def test_planted_eviction_and_window_mistakes_are_caught(monkeypatch):
    W, SK, BLK, T = 12, 3, 4, 32
    q, k, v = _rand(1, T, 2, 2, 32, seed=9)
    o, _ = orc.forward(q, k, v, None, True, W, sinks=SK)
    real_commit = ord_.commit

    def short_tail(cache, kk, vv, window=0, sinks=0):      # keeps one position too few
        real_commit(cache, kk, vv, window, sinks + 1 if window else sinks)
    monkeypatch.setattr(ord_, "commit", short_tail)
    y, _ = ord_.decode_blocks(q, k, v, [BLK] * (T // BLK), True, W, SK)
    assert np.abs(y - o).max() > 1e-3
    monkeypatch.setattr(ord_, "commit", real_commit)

    real_mask = ord_.step_mask

    def loose(Lc, TT, causal, window=0, sinks=0, cpos=None, start=None):   # >= instead of >
        keep, kpos = real_mask(Lc, TT, causal, window + 1 if window else 0, sinks, cpos, start)
        return keep, kpos
    monkeypatch.setattr(ord_, "step_mask", loose)
    y, _ = ord_.decode_blocks(q, k, v, [BLK] * (T // BLK), True, W, SK)
    assert np.abs(y - o).max() > 1e-3


def test_gate_is_applied_per_head():
    q, k, v = _rand(1, 5, 2, 1, 32, seed=3)
    z = np.random.default_rng(4).standard_normal((1, 5, 2))
    y0, _ = ord_.cached_attention(q, k, v, {}, True)
    y1, _ = ord_.cached_attention(q, k, v, {}, True, gate=z)
    assert np.allclose(y1, y0 / (1 + np.exp(-z))[..., None], atol=1e-14)


# ---------------------------------------------------------------- host checks (CPU)
def _dshape(**kw):
    from machinelearning_amd import _capi
    base = dict(B=2, T=4, H=4, Hkv=2, D=64, cached=100, start=100, causal=1, window=0, sinks=0,
                scale=0.125, dtype=_capi.MI_BF16, k_batch_stride=2 * 128 * 64,
                k_head_stride=128 * 64, v_batch_stride=2 * 128 * 64, v_head_stride=128 * 64)
    base.update(kw)
    return _capi.MiDecodeShape(**base)


@pytest.mark.parametrize("kw,code", [
    ({}, 0),
    ({"D": 48}, 4),
    ({"dtype": 5}, 3),
    ({"H": 3}, 2),
    ({"cached": -1}, 2),
    ({"window": 16, "causal": 0}, 5),
    ({"window": 16, "sinks": 16}, 5),
    ({"sinks": 2}, 5),
    ({"window": 16, "sinks": 4}, 0),
    ({"window": 16, "start": -1}, 2),
    ({"k_head_stride": 100}, 6),
    ({"scale": 0.0}, 9),
])
def test_decode_shape_validation(kw, code):
    from machinelearning_amd import _capi
    lib = _capi.load()
    n = ctypes.c_longlong(-1)
    assert lib.mi_attn_decode_workspace(ctypes.byref(_dshape(**kw)), ctypes.byref(n)) == code
    if code == 0:
        assert n.value >= 0


def test_decode_entry_rejects_before_touching_the_device():
    from machinelearning_amd import _capi
    lib = _capi.load()
    shp = _dshape()
    assert lib.mi_attn_decode(*([None] * 10), ctypes.byref(shp), None) == 1
    assert lib.mi_attn_decode(*([None] * 10), ctypes.byref(_dshape(D=48)), None) == 4
    assert lib.mi_attn_decode(*([None] * 10), ctypes.byref(_dshape(T=0)), None) == 0
    assert lib.mi_attn_decode_workspace(ctypes.byref(shp), None) == 1
    # a split step needs a workspace; a tiny one writes its output directly
    assert _capi.decode_workspace_floats(_dshape(B=1, H=2, Hkv=2, T=1, cached=100000)) > 0
    assert _capi.decode_workspace_floats(_dshape(B=64, H=64, Hkv=64, T=1, cached=10)) == 0

    def splits(**kw):
        """Split count of a step: the workspace holds units * splits * rows partial rows,
        O / l in bf16 (D / 2 floats) plus (m, l) in fp32."""
        shp = _dshape(**kw)
        n = _capi.decode_workspace_floats(shp)
        units = shp.B * shp.Hkv            # one-token steps: one row tile per kv head
        return 1 if n == 0 else n // (units * 1 * (shp.D // 2 + 2))
    # a split streams at least 256 KB of K and V (2 * keys * D * 2 bytes in bf16):
    # 1025 keys of D 64 are 262 KB, one split; 8193 keys, 6 splits for 192 units
    # (the ~1024-workgroup target), 2 MB each
    board = dict(B=16, T=1, H=12, Hkv=12, D=64, start=1024)
    assert splits(cached=1024, **board) == 1
    assert splits(cached=8192, **{**board, "start": 8192}) == 6
    # one unit over 100001 keys (25.6 MB): the byte floor allows 97 splits, not the
    # workgroup target's 1024; 391 blocks of 256 keys at 5 blocks per split make 79
    assert splits(B=1, T=1, H=1, Hkv=1, D=64, cached=100000, start=100000) == 79


def test_attn_cached_refusals_without_a_gpu():
    from machinelearning_amd import decode
    q = torch.zeros(1, 4, 2, 32)
    with pytest.raises(ValueError, match="GPU"):
        decode.attn_cached(q, q, q, {}, True)


# ---------------------------------------------------------------- GPU parity
def test_workspace_cache_keeps_recent_streams(monkeypatch):
    """attn_cached's split workspaces: one per (device, stream), reused by the stream's
    later steps, grown on demand, and kept only for the most recently used streams."""
    from machinelearning_amd import decode as dec
    monkeypatch.setattr(dec, "_WORKSPACES", {})
    real = torch.empty
    monkeypatch.setattr(dec.torch, "empty", lambda n, dtype=None, device=None: real(n, dtype=dtype))
    dev = torch.device("cpu")
    n = dec._WS_STREAMS
    for st in range(n + 4):
        dec._workspace(dev, st, 10)
    assert [key[1] for key in dec._WORKSPACES] == list(range(4, n + 4))
    a = dec._workspace(dev, 5, 10)
    assert dec._workspace(dev, 5, 10) is a and list(dec._WORKSPACES)[-1] == (None, 5)
    big = dec._workspace(dev, 5, dec._WS_MIN_FLOATS + 1)
    assert big is not a and big.numel() == dec._WS_MIN_FLOATS + 1


def test_commit_shallow_copies_keep_their_own_rows():
    """Two shallow copies of one cache dict (branching drafts, a rollback snapshot)
    share the capacity buffer; a commit on one must not overwrite rows the other
    already exposes. The first commit after the branch appends in place, the second
    sees the shared high-water mark moved and reallocates (CPU tensors: the commit
    is plain torch)."""
    from machinelearning_amd import decode as dec
    g = torch.Generator().manual_seed(0)
    B, Hkv, D = 2, 3, 8
    cache = {}
    r0 = torch.randn(B, Hkv, 4, D, generator=g)
    dec._commit_append(cache, "k", dec._KBUF, None, r0, 0, 4)
    a, b = dict(cache), dict(cache)
    ra, rb = torch.randn(B, Hkv, 3, D, generator=g), torch.randn(B, Hkv, 5, D, generator=g)
    dec._commit_append(a, "k", dec._KBUF, a["k"], ra, 4, 3)
    assert a["k"].data_ptr() == cache["k"].data_ptr()          # appended in place
    dec._commit_append(b, "k", dec._KBUF, b["k"], rb, 4, 5)
    assert b["k"].data_ptr() != a["k"].data_ptr()              # reallocated
    assert torch.equal(a["k"], torch.cat([r0, ra], 2))
    assert torch.equal(b["k"], torch.cat([r0, rb], 2))
    assert torch.equal(cache["k"], r0)
    # A linear history keeps appending in place.
    p = a["k"].data_ptr()
    rc = torch.randn(B, Hkv, 2, D, generator=g)
    dec._commit_append(a, "k", dec._KBUF, a["k"], rc, 7, 2)
    assert a["k"].data_ptr() == p and torch.equal(a["k"], torch.cat([r0, ra, rc], 2))


def _as(x, dtype):
    return torch.as_tensor(np.ascontiguousarray(x)).to(dtype)


def _rounded(x, dtype):
    return _as(x, dtype).double().numpy()


def _gpu_cache(cache_np, dtype):
    c = {}
    if "k" in cache_np:
        c["k"] = _as(cache_np["k"], dtype).cuda()
        c["v"] = _as(cache_np["v"], dtype).cuda()
    if "pos" in cache_np:
        c["pos"] = torch.as_tensor(cache_np["pos"]).cuda()
    if "end" in cache_np:
        c["end"] = cache_np["end"]
    return c


def _check(tag, got, lse, want, want_lse, dtype):
    _parity.check(tag, "O", got, want, dtype)
    _parity.check(tag, "LSE", lse, want_lse, dtype)


def _step(q, k, v, cache_np, dtype, causal, window=0, sinks=0, gate=None, tag=""):
    from machinelearning_amd.decode import attn_cached
    # the oracle sees exactly the rounded values the kernel reads
    qr, kr, vr = (_rounded(x, dtype) for x in (q, k, v))
    cref = dict(cache_np)
    if "k" in cref:
        cref["k"], cref["v"] = _rounded(cref["k"], dtype), _rounded(cref["v"], dtype)
    want, want_lse = ord_.cached_attention(qr, kr, vr, cref, causal, window, sinks, None, gate)
    cg = _gpu_cache(cache_np, dtype)
    g = None if gate is None else torch.as_tensor(gate).float().cuda()
    with torch.no_grad():
        y, lse = attn_cached(_as(q, dtype).cuda(), _as(k, dtype).cuda(), _as(v, dtype).cuda(),
                             cg, False, causal, window=window, sinks=sinks, gate=g,
                             return_lse=True)
    torch.cuda.synchronize()
    _check(tag, y.double().cpu().numpy(), lse.double().cpu().numpy(), want, want_lse, dtype)
    return y


DTYPES = [torch.float32, torch.bfloat16, torch.float16]
# (T, cached, H, Hkv): one token, GQA, long caches (split over keys: a split
# streams at least 256 KB of K and V, so the last three shapes split), query
# rows beyond one 32-row tile (T * H / Hkv > 32), an empty cache (prefill).
SHAPES = [(1, 0, 4, 4), (1, 1, 4, 2), (1, 300, 8, 2), (5, 77, 4, 1), (32, 1000, 4, 4),
          (33, 129, 6, 2), (100, 0, 4, 2), (7, 3000, 2, 1), (1, 5000, 4, 2), (40, 2500, 4, 1)]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).replace("torch.", ""))
@pytest.mark.parametrize("D", [32, 64, 128])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "T%d_L%d_H%d_%d" % s)
@pytest.mark.parametrize("causal", [True, False], ids=["causal", "bidir"])
def test_decode_step_parity(dtype, D, shape, causal):
    T, Lc, H, Hkv = shape
    g = np.random.default_rng(T * 1000 + Lc + D)
    B = 2
    q = g.standard_normal((B, T, H, D))
    k = g.standard_normal((B, T, Hkv, D))
    v = g.standard_normal((B, T, Hkv, D))
    cache = {}
    if Lc:
        cache = {"k": g.standard_normal((B, Hkv, Lc, D)), "v": g.standard_normal((B, Hkv, Lc, D))}
    _step(q, k, v, cache, dtype, causal, tag=f"decode {dtype} D{D} {shape} causal={causal}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).replace("torch.", ""))
@pytest.mark.parametrize("D", [32, 64, 128])
def test_decode_swa_with_evicted_positions_and_gate(dtype, D):
    """SWA(64, 4) after eviction: cached rows are the sinks 0..3 plus a tail."""
    g = np.random.default_rng(D)
    B, T, H, Hkv, W, SK = 2, 9, 4, 2, 64, 4
    end = 500
    pos = np.concatenate([np.arange(SK), np.arange(end - (W - SK - 1), end)])
    Lc = len(pos)
    cache = {"k": g.standard_normal((B, Hkv, Lc, D)), "v": g.standard_normal((B, Hkv, Lc, D)),
             "pos": pos, "end": end}
    q = g.standard_normal((B, T, H, D))
    k = g.standard_normal((B, T, Hkv, D))
    v = g.standard_normal((B, T, Hkv, D))
    z = g.standard_normal((B, T, H))
    _step(q, k, v, cache, dtype, True, W, SK, tag=f"swa {dtype} D{D}")
    # one token per kv head pair (the VALU kernel's path)
    _step(q[:, :1], k[:, :1], v[:, :1], cache, dtype, True, W, SK, tag=f"swa T1 {dtype} D{D}")
    _step(q, k, v, cache, dtype, True, W, SK, gate=z, tag=f"swa+gate {dtype} D{D}")
    # more than 32 query rows per kv head (20 tokens x GQA 4: the shared-block kernel)
    H2 = 8
    q2 = g.standard_normal((B, 20, H2, D))
    k2 = g.standard_normal((B, 20, Hkv, D))
    v2 = g.standard_normal((B, 20, Hkv, D))
    _step(q2, k2, v2, cache, dtype, True, W, SK, tag=f"swa R80 {dtype} D{D}")
    # no eviction yet: no 'pos', cache rows at 0 .. end-1
    c2 = {"k": cache["k"][:, :, :40], "v": cache["v"][:, :, :40], "end": 40}
    _step(q, k, v, c2, dtype, True, W, SK, tag=f"swa-fresh {dtype} D{D}")
    # a wide window after eviction, long enough to split over keys (the positions
    # array read across split boundaries)
    W3, end3 = 3000, 10000
    pos3 = np.concatenate([np.arange(SK), np.arange(end3 - (W3 - SK - 1), end3)])
    c3 = {"k": g.standard_normal((B, Hkv, len(pos3), D)),
          "v": g.standard_normal((B, Hkv, len(pos3), D)), "pos": pos3, "end": end3}
    _step(q, k, v, c3, dtype, True, W3, SK, tag=f"swa W{W3} {dtype} D{D}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).replace("torch.", ""))
@pytest.mark.parametrize("mode", ["causal", "bidir", "swa"])
def test_cached_blocks_through_the_kernel_equal_full_attention(dtype, mode):
    """Block by block with commit (the cache grows in its capacity buffer, or is
    evicted under a window) == one uncached pass over the whole sequence."""
    from machinelearning_amd.decode import attn_cached
    B, S, H, Hkv, D = 2, 96, 4, 2, 64
    q, k, v = _rand(B, S, H, Hkv, D, seed=11)
    qr, kr, vr = (_rounded(x, dtype) for x in (q, k, v))
    causal, window, sinks, blocks = True, 0, 0, [1, 7, 8, 16, 1, 31, 32]
    block = 0
    if mode == "bidir":
        causal, blocks, block = False, [8] * 12, 8
    if mode == "swa":
        window, sinks, blocks = 12, 3, [8] * 12
    want, _ = orc.forward(qr, kr, vr, None, True, window, sinks=sinks, block=block)
    cache, outs, sizes, p0 = {}, [], [], 0
    with torch.no_grad():
        for n in blocks:
            sl = slice(p0, p0 + n)
            y = attn_cached(_as(q[:, sl], dtype).cuda(), _as(k[:, sl], dtype).cuda(),
                            _as(v[:, sl], dtype).cuda(), cache, True, causal,
                            window=window, sinks=sinks)
            outs.append(y.double().cpu().numpy())
            sizes.append(cache["k"].shape[2])
            p0 += n
    got = np.concatenate(outs, axis=1)
    print(f"blocks {mode} {dtype}: sizes {sizes}", flush=True)
    _parity.check(f"blocks {mode} {dtype}", "O", got, want, dtype)
    if mode == "swa":
        assert all(z <= window - 1 for z in sizes) and sizes[-1] == sizes[-2]
    else:
        assert sizes == list(np.cumsum(blocks))
        # the committed rows equal the inputs (capacity buffer, appended in place)
        assert torch.equal(cache["k"].cpu(), _as(k, dtype).transpose(1, 2))


@pytest.mark.gpu
def test_decode_is_deterministic_and_rejects_autograd():
    from machinelearning_amd.decode import attn_cached
    g = torch.Generator().manual_seed(0)
    B, T, H, Hkv, D, Lc = 4, 1, 12, 12, 64, 4096
    q = torch.randn(B, T, H, D, generator=g).bfloat16().cuda()
    k = torch.randn(B, T, Hkv, D, generator=g).bfloat16().cuda()
    cache = {"k": torch.randn(B, Hkv, Lc, D, generator=g).bfloat16().cuda(),
             "v": torch.randn(B, Hkv, Lc, D, generator=g).bfloat16().cuda()}
    with torch.no_grad():
        a = attn_cached(q, k, k, dict(cache), False, True)
        b = attn_cached(q, k, k, dict(cache), False, True)
    assert torch.equal(a, b)
    with pytest.raises(RuntimeError, match="inference"):
        attn_cached(q.float().requires_grad_(), k.float(), k.float(), {}, False, True)
    with pytest.raises(ValueError, match="causal"):
        attn_cached(q, k, k, {}, False, False, window=8)


@pytest.mark.gpu
@pytest.mark.parametrize("Lc,H,Hkv,D", [(300_000, 1, 1, 64), (100_000, 8, 2, 128)])
def test_decode_very_long_cache(Lc, H, Hkv, D):
    """One token over a very long cache: hundreds of key splits for a single kv head,
    and a GQA case; against torch's SDPA in fp32 on the same (rounded) values."""
    from machinelearning_amd.decode import attn_cached
    g = torch.Generator(device="cuda").manual_seed(Lc)
    B, T = 1, 1
    q = torch.randn(B, T, H, D, device="cuda", generator=g).bfloat16()
    k = torch.randn(B, T, Hkv, D, device="cuda", generator=g).bfloat16()
    v = torch.randn(B, T, Hkv, D, device="cuda", generator=g).bfloat16()
    ck = torch.randn(B, Hkv, Lc, D, device="cuda", generator=g).bfloat16()
    cv = torch.randn(B, Hkv, Lc, D, device="cuda", generator=g).bfloat16()
    with torch.no_grad():
        y, lse = attn_cached(q, k, v, {"k": ck, "v": cv}, False, True, return_lse=True)
        kf = torch.cat([ck, k.transpose(1, 2)], 2).float().repeat_interleave(H // Hkv, 1)
        vf = torch.cat([cv, v.transpose(1, 2)], 2).float().repeat_interleave(H // Hkv, 1)
        qf = q.float().transpose(1, 2)
        s = (qf @ kf.transpose(-1, -2)) * D ** -0.5
        ref = (torch.softmax(s, -1) @ vf).transpose(1, 2)
        rlse = torch.logsumexp(s, -1)                         # [B, H, T], as lse
    torch.cuda.synchronize()
    assert lse.shape == rlse.shape
    tag = f"long cache {Lc} H{H}/{Hkv} D{D}"
    _parity.check(tag, "O", y.double().cpu().numpy(), ref.double().cpu().numpy(), torch.bfloat16)
    _parity.check(tag, "LSE", lse.double().cpu().numpy(), rlse.double().cpu().numpy(),
                  torch.bfloat16)


@pytest.mark.gpu
def test_decode_workspace_reused_across_shapes():
    """One workspace, filled with NaN and then reused by split steps of different shapes
    and kernels (VALU, per-wave MFMA, shared-block MFMA), gives the results of a fresh
    workspace per step, bit for bit: every partial the merge reads was written by the
    same step."""
    import ctypes
    from machinelearning_amd import _capi
    lib = _capi.load()
    g = torch.Generator(device="cuda").manual_seed(7)
    steps = [(4, 1, 12, 12, 64, 3000, 1), (2, 8, 32, 8, 128, 2000, 1),
             (2, 32, 16, 4, 64, 6000, 0), (1, 1, 8, 2, 32, 20000, 1), (3, 4, 4, 4, 64, 5000, 0)]
    shared = torch.full((1 << 22,), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    for B, T, H, Hkv, D, Lc, causal in steps:
        def rnd(*s):
            return torch.randn(*s, device="cuda", generator=g).bfloat16()
        q, k, v = rnd(B, T, H, D), rnd(B, T, Hkv, D), rnd(B, T, Hkv, D)
        ck, cv = rnd(B, Hkv, Lc, D), rnd(B, Hkv, Lc, D)
        shp = _capi.MiDecodeShape(B, T, H, Hkv, D, Lc, Lc, causal, 0, 0, D ** -0.5,
                                  _capi.MI_BF16, ck.stride(0), ck.stride(1), cv.stride(0),
                                  cv.stride(1))
        nws = _capi.decode_workspace_floats(shp)
        assert 0 < nws <= shared.numel(), (B, T, H, Hkv, D, Lc, nws)
        outs = []
        for ws in (shared, torch.empty(nws, device="cuda"), shared):
            out = torch.empty_like(q)
            lse = torch.empty(B, H, T, device="cuda")
            _capi.check(lib.mi_attn_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                           ck.data_ptr(), cv.data_ptr(), None, None,
                                           out.data_ptr(), lse.data_ptr(), ws.data_ptr(),
                                           ctypes.byref(shp), st))
            outs.append((out, lse))
        torch.cuda.synchronize()
        for out, lse in outs[1:]:
            assert torch.equal(out, outs[0][0]) and torch.equal(lse, outs[0][1])
        kf = torch.cat([ck, k.transpose(1, 2)], 2).float().repeat_interleave(H // Hkv, 1)
        vf = torch.cat([cv, v.transpose(1, 2)], 2).float().repeat_interleave(H // Hkv, 1)
        s = (q.float().transpose(1, 2) @ kf.transpose(-1, -2)) * D ** -0.5
        if causal:
            qpos = torch.arange(Lc, Lc + T, device="cuda")[:, None]
            s = s.masked_fill(torch.arange(Lc + T, device="cuda")[None, :] > qpos, float("-inf"))
        ref = (torch.softmax(s, -1) @ vf).transpose(1, 2)
        _parity.check(f"shared workspace B{B} T{T} H{H}/{Hkv} D{D} L{Lc} ({nws} floats)", "O",
                      outs[0][0].double().cpu().numpy(), ref.double().cpu().numpy(),
                      torch.bfloat16)


def _decode_sweep_cases(n=None, seed=None):
    """Seeded random decode steps; the suite runs 12 (seed 2027), MI_DECODE_SWEEP_N /
    MI_DECODE_SWEEP_SEED widen a one-off run."""
    import os
    n = int(os.environ.get("MI_DECODE_SWEEP_N", 12)) if n is None else n
    seed = int(os.environ.get("MI_DECODE_SWEEP_SEED", 2027)) if seed is None else seed
    rng = np.random.default_rng(seed)
    heads = [(1, 1), (4, 4), (4, 2), (6, 3), (8, 1), (12, 4)]
    cases = []
    for i in range(n):
        T = int(rng.choice([1, 1, 2, 4, int(rng.integers(1, 81))]))
        Lc = int(rng.choice([0, int(rng.integers(1, 300)), int(rng.integers(300, 4000))]))
        H, Hkv = heads[int(rng.integers(len(heads)))]
        D = int(rng.choice([32, 64, 128]))
        mode = ["causal", "bidir", "window"][int(rng.integers(3))]
        window = sinks = 0
        if mode == "window":
            window = int(rng.integers(2, Lc + T + 40))
            sinks = int(rng.integers(0, min(window, 8)))
        gate = bool(rng.random() < 0.3)
        cases.append((i, T, Lc, H, Hkv, D, DTYPES[i % 3], mode != "bidir", window, sinks, gate))
    return cases


@pytest.mark.gpu
@pytest.mark.parametrize("case", _decode_sweep_cases(), ids=lambda c: "d%d" % c[0])
def test_decode_random_sweep(case):
    """Random decode steps: query rows, cache lengths on both sides of the split floor,
    GQA groups, head dims, dtypes, causal / bidirectional / windowed with sinks, gates."""
    i, T, Lc, H, Hkv, D, dtype, causal, window, sinks, gate = case
    g = np.random.default_rng(500 + i)
    B = int(g.integers(1, 3))
    q = g.standard_normal((B, T, H, D))
    k = g.standard_normal((B, T, Hkv, D))
    v = g.standard_normal((B, T, Hkv, D))
    cache = {}
    if Lc:
        cache = {"k": g.standard_normal((B, Hkv, Lc, D)), "v": g.standard_normal((B, Hkv, Lc, D))}
        if window:
            cache["end"] = Lc          # a windowed cache names its end (no eviction here)
    gt = g.standard_normal((B, T, H)) if gate else None
    _step(q, k, v, cache, dtype, causal, window=window, sinks=sinks, gate=gt,
          tag=f"decode sweep d{i}: B{B} T{T} L{Lc} H{H}/{Hkv} D{D} {dtype} causal={causal} "
              f"w={window} s={sinks} gate={gate}")

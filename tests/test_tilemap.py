"""The CPU mirror of the kernels' tile arithmetic (tests/tilemap.py) against
the oracle's visible mask, on the BASELINE shapes, the reference's test
shapes and a seeded sweep; plus planted off-by-ones in the mirror that the
checks must catch.

What is checked, for every mask kind (causal, block-causal, non-causal,
sliding window with and without sinks, one or several folded sink tiles
and the separate sink passes):
  * every visible (query, key) pair enters each pass exactly once, and no
    invisible or padding pair enters unmasked (forward, dQ, dK/dV);
  * work_item is a bijection of blockIdx onto (head, row block);
  * every LDS ring step reads the slot holding its unit, after the step's
    vmcnt wait has retired that unit;
  * the decode split plan covers the key blocks exactly once, never splits a
    step into an empty split, and its workspace size equals the library's
    own mi_attn_decode_workspace (host-side query, no GPU needed).
"""

from __future__ import annotations

import ctypes
import dataclasses
import math

import numpy as np
import pytest

from oracle import attention as orc
from tests import tilemap as tm


def _check_pass(m: tm.Mask, kernel: str, window: int, sinks: int, block: int):
    C, sink_pass = tm.total_coverage(m, kernel)
    S = m.S
    vis = orc.visible_mask(S, m.causal, window, sinks, block).astype(np.int32)
    inside = C[:S, :S] + sink_pass
    bad = np.argwhere(inside != vis)
    assert bad.size == 0, (f"{kernel} {m}: {len(bad)} pairs visited {inside[tuple(bad[0])]}x "
                           f"where the mask says {vis[tuple(bad[0])]}, e.g. (q, k) = {tuple(bad[0])}")
    # Padding rows (read as zero past S) must stay masked where they feed a stored
    # result: keys past S in the forward and dQ (they enter valid queries' sums),
    # queries past S in dK/dV (they enter valid keys' sums). The other side is
    # lane-private: lanes past S compute but never store.
    if kernel == "dkdv":
        assert C[S:, :S].sum() == 0, f"{kernel} {m}: a query past S entered unmasked"
    else:
        assert C[:S, S:].sum() == 0, f"{kernel} {m}: a key past S entered unmasked"


def _all_passes(S, causal=True, window=0, sinks=0, block=0, sixteen_bit=True):
    m = tm.Mask.of(S, causal, window, sinks, block, sixteen_bit)
    for kernel in ("fwd", "dq", "dkdv"):
        _check_pass(m, kernel, window, sinks, block)


# The BASELINE configs' masks (B, H do not enter the tile walk), nanolab's swa
# default SWA(64, 4), and the reference's test shapes.
BASELINE = [(256, True, 0, 0, 0), (1024, True, 0, 0, 0), (4096, True, 256, 0, 0),
            (1024, True, 64, 4, 0), (8192, True, 0, 0, 0), (2048, False, 0, 0, 0),
            (4096, True, 256, 4, 0)]


@pytest.mark.parametrize("S,causal,window,sinks,block", BASELINE,
                         ids=lambda v: str(v))
def test_baseline_masks_visit_each_visible_pair_once(S, causal, window, sinks, block):
    if S > 4096:
        pytest.skip("S=8192 is covered by the same arithmetic at S=4096 (tiles repeat)")
    _all_passes(S, causal, window, sinks, block)


@pytest.mark.parametrize("T", [1, 33, 37, 64, 100, 130, 257, 300])
@pytest.mark.parametrize("mode", ["causal", "noncausal", "window", "block", "sinks_fold",
                                  "sinks_wide"])
def test_reference_shapes(T, mode):
    if mode == "causal":
        _all_passes(T)
    elif mode == "noncausal":
        _all_passes(T, causal=False)
    elif mode == "window":
        _all_passes(T, window=17)
    elif mode == "block":
        _all_passes(T, block=7)
    elif mode == "sinks_fold":
        _all_passes(T, window=40, sinks=5)
        _all_passes(T, window=45, sinks=33)     # both halves of key tile 0
        _all_passes(T, window=70, sinks=64)
        _all_passes(T, window=90, sinks=65)     # two sink tiles
        _all_passes(T, window=200, sinks=129)   # three, the last with one sink
        _all_passes(T, window=280, sinks=270)   # span 10, up to five sink tiles
    else:       # sinks past what any row sees (capped at S - span), span >= S;
        # float32: the separate sink kernels
        _all_passes(T, window=T + 5, sinks=T - 3 if T > 3 else 0)
        _all_passes(T, window=T + 40, sinks=T + 20)
        _all_passes(T, window=17, sinks=4, sixteen_bit=False)
        _all_passes(T, window=90, sinks=65, sixteen_bit=False)


def test_seeded_sweep_of_masks():
    rng = np.random.default_rng(7)
    for _ in range(60):
        T = int(rng.integers(1, 700))
        kind = rng.integers(4)
        if kind == 0:
            _all_passes(T, causal=bool(rng.integers(2)))
        elif kind == 1:
            w = int(rng.integers(1, T + 70))
            s = int(rng.integers(0, w)) if rng.random() < 0.5 else 0
            _all_passes(T, window=w, sinks=s, sixteen_bit=bool(rng.integers(2)))
        else:
            _all_passes(T, block=int(rng.integers(2, T + 9)))


@pytest.mark.parametrize("nblk,BH", [(8, 192), (32, 128), (4, 32), (64, 2), (8, 12), (3, 7),
                                     (1, 1), (16, 24)])
@pytest.mark.parametrize("heavy,blocks_fastest", [(True, False), (False, False), (False, True)])
def test_work_item_is_a_bijection(nblk, BH, heavy, blocks_fastest):
    seen = set()
    for bid in range(nblk * BH):
        bh, blk = tm.work_item(bid, nblk, BH, heavy, blocks_fastest)
        assert 0 <= bh < BH and 0 <= blk < nblk
        seen.add((bh, blk))
    assert len(seen) == nblk * BH
    if blocks_fastest and BH % 8 == 0:
        # A head's row blocks are consecutive on its XCD (blockIdx mod 8 = bh mod 8).
        for bid in range(nblk * BH):
            bh, blk = tm.work_item(bid, nblk, BH, False, True)
            assert bid % 8 == bh % 8
            if blk + 1 < nblk:
                assert tm.work_item(bid + 8, nblk, BH, False, True) == (bh, blk + 1)
    if heavy and BH % 8 == 0:
        # Heaviest causal blocks (the last row blocks) are dealt out first.
        first = [tm.work_item(b, nblk, BH, True)[1] for b in range(min(BH, nblk * BH))]
        assert all(blk == nblk - 1 for blk in first)


@pytest.mark.parametrize("B,Hkv,group,nblk", [(8, 4, 3, 8), (1, 2, 2, 3), (2, 1, 4, 2),
                                               (4, 8, 4, 8), (3, 5, 2, 7), (16, 12, 1, 8)])
@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("blocks_fastest", [False, True])
def test_dkdv_grid_covers_every_head_once(B, Hkv, group, nblk, split, blocks_fastest):
    """Split or not, in either work order, the dK/dV grid walks every (b, kv head, key
    block, query head of the group) exactly once; split, each workgroup walks exactly one
    query head."""
    nsplit = group if (split and group > 1) else 1
    seen = {}
    for bid in range(nblk * B * Hkv * nsplit):
        b, hk, blk, g0, gn = tm.dkdv_work(bid, nblk, B, Hkv, group, nsplit, blocks_fastest)
        assert 0 <= b < B and 0 <= hk < Hkv and 0 <= blk < nblk
        assert gn == (1 if nsplit > 1 else group)
        for gh in range(g0, g0 + gn):
            key = (b, hk, blk, hk * group + gh)
            assert key not in seen, f"{key} walked twice (blockIdx {seen[key]} and {bid})"
            seen[key] = bid
    assert len(seen) == B * Hkv * nblk * group


@pytest.mark.parametrize("d", list(range(1, 300)) + [511, 512, 513, 1536, 4095, 4096, 65537])
def test_fast_div_is_exact(d):
    """fast_div / fdiv (attn_common.h) against integer division, around multiples of d
    and at the top of the index range (n < 2^31)."""
    f = tm.fast_div(d)
    assert 0 < f[0] < (1 << 32)
    ns = {0, 1, d - 1, d, d + 1, (1 << 31) - 1, (1 << 31) - 2}
    ns |= {k * d + e for k in (2, 3, 1000, (1 << 31) // d - 1) for e in (-1, 0, 1)}
    for n in sorted(x for x in ns if 0 <= x < (1 << 31)):
        assert tm.fdiv(n, f) == n // d, (d, n)


def test_planted_split_head_mistake_is_caught(restore):
    """A split grid that lets every workgroup of a key block walk group head 0."""
    orig = tm.dkdv_work

    def head0(bid, nblk, B, Hkv, group, nsplit, blocks_fastest=False):
        b, hk, blk, g0, gn = orig(bid, nblk, B, Hkv, group, nsplit, blocks_fastest)
        return b, hk, blk, 0, gn
    tm.dkdv_work = head0
    try:
        assert _fails(lambda: test_dkdv_grid_covers_every_head_once(8, 4, 3, 8, True, False))
    finally:
        tm.dkdv_work = orig


@pytest.mark.parametrize("n", [1, 2, 3, 4, 7, 16])
@pytest.mark.parametrize("t_begin", [0, 3])
def test_forward_ring_reads_retired_units(n, t_begin):
    for t, occupant, slot, retired in tm.ring_fwd(t_begin, t_begin + n):
        assert occupant == t, f"step {t} reads slot {slot} holding unit {occupant}"
        assert retired, f"step {t}: unit not retired by the wait"


@pytest.mark.parametrize("n", [1, 2, 3, 5, 16, 48])
@pytest.mark.parametrize("NS", [2, 3])
def test_backward_rings_read_retired_units(n, NS):
    for it, occupant, retired in tm.ring_simple(n, NS):
        assert occupant == it and retired, (it, occupant, retired)


def test_entry_mask_keep_sets_match_the_bounds():
    """mask_above / mask_below / mask_rows build a per-lane keep set and select by
    its bits; they must keep exactly the offsets c with c <= hi, c >= lo, or both,
    for bounds far outside the 28 offsets on either side (clamps, shift counts)."""
    for hi in range(-70, 71):
        assert tm.mask_keep(tm.keep_upto(hi)) == [c <= hi for c in tm.CROW_OFFS], hi
    for lo in range(-70, 71):
        assert tm.mask_keep(tm.keep_from(lo)) == [c >= lo for c in tm.CROW_OFFS], lo
    for lo in range(-5, 33, 3):
        for hi in range(-5, 33, 3):
            got = tm.mask_keep(tm.keep_from(lo) & tm.keep_upto(hi))
            assert got == [lo <= c <= hi for c in tm.CROW_OFFS], (lo, hi)


def test_entry_mask_catches_a_clamp_one_short():
    # a cap of 27 never keeps offset 27 (the last entry), whatever the bound
    def run():
        for hi in range(-3, 40):
            assert tm.mask_keep(tm.keep_upto(hi, cap=27)) == [c <= hi for c in tm.CROW_OFFS], hi
    assert _fails(run)


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 7, 16, 48])
def test_dkdv_pair_ring_reads_retired_units(n):
    for it, occupant, retired in tm.ring_pair(n):
        assert occupant == it and retired, (it, occupant, retired)


def test_dkdv_pair_ring_catches_a_refill_of_a_slot_in_use():
    # refilling the pair's own second slot (it+1's) instead of it-1's
    assert _fails(lambda: tm.ring_pair(8, refill=lambda sl: ((sl + 2) % 4, (sl + 1) % 4)))


# --------------------------------------------------------------------------- planted mistakes
@pytest.fixture
def restore():
    saved = (tm.causal_key_end, tm.causal_query_begin, tm._query_walk, tm.dkdv_ranges,
             tm._sink_visit, tm.extra_sinks)
    yield
    (tm.causal_key_end, tm.causal_query_begin, tm._query_walk, tm.dkdv_ranges,
     tm._sink_visit, tm.extra_sinks) = saved


def _fails(fn):
    try:
        fn()
    except AssertionError:
        return True
    return False


def test_planted_causal_key_end_off_by_one_is_caught(restore):
    orig = tm.causal_key_end
    tm.causal_key_end = lambda m, i: orig(m, i) + 1
    assert _fails(lambda: _check_pass(tm.Mask.of(300), "fwd", 0, 0, 0))
    assert _fails(lambda: _check_pass(tm.Mask.of(300), "dq", 0, 0, 0))
    tm.causal_key_end = lambda m, i: orig(m, i) - 1
    assert _fails(lambda: _check_pass(tm.Mask.of(300), "fwd", 0, 0, 0))


def test_planted_tw_begin_off_by_one_is_caught(restore):
    orig = tm._query_walk

    def walk(m, BM, BN):
        for qw0, twb, twe, q0, tb, te in orig(m, BM, BN):
            yield qw0, twb + 1, twe, q0, tb, te
    tm._query_walk = walk
    assert _fails(lambda: _check_pass(tm.Mask.of(500, window=100), "fwd", 100, 0, 0))
    assert _fails(lambda: _check_pass(tm.Mask.of(500), "dq", 0, 0, 0))


def test_planted_dkdv_range_mistakes_are_caught(restore):
    orig = tm.dkdv_ranges

    def late_start(m, blk):
        tb, te, waves = orig(m, blk)
        return tb, te, [(kw0, twb + 1, twe) for kw0, twb, twe in waves]

    def short_end(m, blk):
        tb, te, waves = orig(m, blk)
        return tb, te, [(kw0, twb, max(twb, twe - 1)) for kw0, twb, twe in waves]
    tm.dkdv_ranges = late_start
    assert _fails(lambda: _check_pass(tm.Mask.of(300), "dkdv", 0, 0, 0))
    tm.dkdv_ranges = short_end
    assert _fails(lambda: _check_pass(tm.Mask.of(300, window=64), "dkdv", 64, 0, 0))
    tm.dkdv_ranges = orig
    tm.causal_query_begin = lambda m, j: j + 1
    assert _fails(lambda: _check_pass(tm.Mask.of(300), "dkdv", 0, 0, 0))


def test_planted_sink_bound_is_caught(restore):
    """A sink visit that lets row i see one sink too many (j < i - span + 2) is caught."""
    orig = tm._sink_visit
    tm._sink_visit = lambda C, m, q0, qw0, half: orig(
        C, dataclasses.replace(m, window=m.window - 1), q0, qw0, half)
    m = tm.Mask.of(200, window=90, sinks=65)
    assert _fails(lambda: _check_pass(m, "fwd", 90, 65, 0))
    assert _fails(lambda: _check_pass(m, "dq", 90, 65, 0))


def test_planted_sink_pass_bound_is_caught(restore):
    """The same off-by-one in the separate sink kernels' bound (float32) is caught."""
    tm.extra_sinks = lambda m, i: np.maximum(0, np.minimum(m.sinks, i - m.window + 2))
    m = tm.Mask.of(200, window=90, sinks=65, sixteen_bit=False)
    assert _fails(lambda: _check_pass(m, "fwd", 90, 65, 0))


def test_planted_dq_sink_half_is_caught(restore):
    """dQ's folded-sink visit must take a sink tile's second half when sinks reach it: a
    visit that skips the second 32-key half of each tile misses sinks 32..63."""
    orig = tm._sink_visit

    def first_halves_only(C, m, q0, qw0, half):
        C2 = np.zeros_like(C)
        orig(C2, m, q0, qw0, half)
        k = np.arange(C.shape[1])
        C += C2 * ((k % 64) < 32)[None, :]
    tm._sink_visit = first_halves_only
    try:
        assert _fails(lambda: _check_pass(tm.Mask.of(300, window=70, sinks=50), "dq", 70, 50, 0))
        _check_pass(tm.Mask.of(300, window=45, sinks=20), "dq", 45, 20, 0)
    finally:
        tm._sink_visit = orig


def test_planted_one_sink_tile_is_caught(restore):
    """The folded-sink visits must cover every sink tile: a fold of key tile 0 only
    (at most 64 sinks visited) misses sinks 64.. in the forward and in dQ."""
    orig = tm._sink_visit

    def tile0_only(C, m, q0, qw0, half):
        orig(C, dataclasses.replace(m, fold=min(m.fold, 64)), q0, qw0, half)
    tm._sink_visit = tile0_only
    try:
        m = tm.Mask.of(300, window=200, sinks=129)
        assert _fails(lambda: _check_pass(m, "fwd", 200, 129, 0))
        assert _fails(lambda: _check_pass(m, "dq", 200, 129, 0))
        _check_pass(tm.Mask.of(300, window=70, sinks=64), "fwd", 70, 64, 0)
    finally:
        tm._sink_visit = orig


def test_planted_dkdv_sink_block_walk_is_caught(restore):
    """Every key block holding sinks must walk the query tiles to the end: a walk that
    stops at the window for blocks past key block 0 misses the late queries' pairs
    with sinks 128.. (the public sinks every query sees, nanolab/mixers.py:117-120)."""
    orig = tm.dkdv_ranges

    def block0_only(m, blk):
        if blk > 0 and m.fold > 0:
            m = dataclasses.replace(m, fold=0)
        return orig(m, blk)
    tm.dkdv_ranges = block0_only
    m = tm.Mask.of(600, window=200, sinks=150)
    assert _fails(lambda: _check_pass(m, "dkdv", 200, 150, 0))


# --------------------------------------------------------------------------- decode
def _lib():
    from machinelearning_amd import _capi
    try:
        return _capi, _capi.load()
    except OSError as e:       # not built: the workspace cross-check needs the library
        pytest.skip(f"libmi_attn.so not loadable: {e}")


DECODE = [(16, 1, 12, 12, 64, 1024), (16, 1, 12, 12, 64, 8192), (1, 1, 12, 12, 64, 32768),
          (8, 1, 32, 8, 128, 8192), (16, 32, 12, 12, 64, 1024), (8, 32, 32, 8, 128, 4096),
          (1, 1, 4, 4, 32, 5000), (2, 80, 4, 2, 64, 2500), (3, 4, 4, 4, 64, 300000),
          (2, 8, 32, 8, 128, 2000)]


@pytest.mark.parametrize("dtype", [0, 2])
@pytest.mark.parametrize("case", DECODE, ids=lambda c: "B%dT%dH%d/%dD%dL%d" % c)
def test_decode_plan_matches_library_and_partitions_keys(case, dtype):
    capi, lib = _lib()
    B, T, H, Hkv, D, Lc = case
    plan = tm.decode_plan(4 if dtype == 0 else 2, B, T, H, Hkv, D, Lc + T)
    blocks = [b for lo, hi in plan["splits"] for b in range(lo, hi)]
    assert blocks == list(range(plan["nblk"])), "splits must cover the key blocks once, in order"
    assert all(hi > lo for lo, hi in plan["splits"]), "an empty split"
    assert plan["nsplit"] <= 1024
    shp = capi.MiDecodeShape(B, T, H, Hkv, D, Lc, Lc, 1, 0, 0, D ** -0.5, dtype,
                             Hkv * Lc * D, Lc * D, Hkv * Lc * D, Lc * D)
    n = ctypes.c_longlong(-1)
    assert lib.mi_attn_decode_workspace(ctypes.byref(shp), ctypes.byref(n)) == 0
    assert n.value == plan["workspace_floats"], (plan, n.value)
    if plan["nsplit"] > 1:
        # Every split streams at least the byte floor's worth of K and V blocks.
        per_split = plan["bps"] * plan["BN"] * 2 * D * (4 if dtype == 0 else 2)
        assert per_split >= tm.DEC_MIN_SPLIT_BYTES or plan["nsplit"] == 1
    assert math.ceil((Lc + T) / plan["BN"]) == plan["nblk"]

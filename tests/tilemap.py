"""CPU mirror of the 16-bit kernels' tile arithmetic (test infrastructure).

The HIP kernels decide, from integer arithmetic on (block, wave, lane), which
key or query tiles each wave visits, which entries of a visited tile it masks,
which LDS ring slot holds which tile, and how a decode step splits its keys.
This module restates that arithmetic line by line in Python so it can be
checked on the CPU, where a wrong bound shows up as a wrong count instead of a
silent error or a memory fault on the GPU:

  * ``work_item``: blockIdx -> (batch*head, row block), ``attn_common.h``;
  * ``fwd_coverage`` / ``dq_coverage``: the forward's and dQ's walk over key
    tiles per 32-query wave (``attn_fwd16.hip``, ``attn_bwd16.hip``), the
    one-sided masks, dQ's skipped 32-key halves and the visit of the sink
    tiles before the window;
  * ``dkdv_coverage``: dK/dV's walk over query tiles per 32-key wave, its
    masks, and the walk to the end of the key blocks holding sinks;
  * ``sink_pass_coverage``: the separate sink kernels' extra pairs (float32:
    ``attn_sinks.hip``, rows i >= span, keys j < extra_sinks(i));
  * ``ring_*``: which unit each LDS ring slot holds at every step, and that
    the step's vmcnt wait has retired it;
  * ``decode_plan``: the KV-cached decode step's split geometry
    (``attn_decode.hip`` ``dec_geometry``) and its workspace size.

Each coverage function returns an int array C[q, k] counting how often the
pair (query q, key k) enters a softmax unmasked; rows and columns run to the
padded tile edge, so a count past S means a read of a padding row went
unmasked. The tests compare C with the oracle's visible mask.

Nothing here runs in the product path; it mirrors it.
"""

from __future__ import annotations

import dataclasses

import numpy as np

# Tile geometry of the 16-bit kernels.
FWD_BM, FWD_BN, FWD_NS = 128, 64, 2          # attn_fwd16: 4 waves x 32 queries, 64-key tiles
DQ_BM, DQ_BN = 128, 64                       # attn_bwd16 dQ
DKDV_BK, DKDV_BQ = 128, 64                   # attn_bwd16 dK/dV: 4 waves x 32 keys, 64-query tiles
WAVES, WROWS = 4, 32


@dataclasses.dataclass(frozen=True)
class Mask:
    """The kernels' view of a mask (AttnParams): `window` is the local span
    (window - sinks of the public SWA(window, sinks)), `fold` the sinks the
    window kernels visit themselves (16-bit; those some row sees: span < S,
    capped at S - span), `block` the causal
    block length (1 = plain causal)."""
    S: int
    causal: bool = True
    window: int = 0
    sinks: int = 0
    fold: int = 0
    block: int = 1

    @staticmethod
    def of(S, causal=True, window=0, sinks=0, block=0, sixteen_bit=True):
        """From the public arguments, as capi.hip params() packs them."""
        span = window - sinks if window > 0 else 0
        snk = sinks if window > 0 else 0
        fold = min(snk, S - span) if (sixteen_bit and span < S) else 0
        return Mask(S, bool(causal), span, snk, fold, block if block > 1 else 1)


def causal_key_end(m: Mask, i):
    """Last key query i sees (attn_common.h causal_key_end)."""
    if m.block > 1:
        return np.minimum(m.S - 1, (i // m.block + 1) * m.block - 1)
    return i


def causal_query_begin(m: Mask, j):
    """First query that sees key j (attn_common.h causal_query_begin)."""
    if m.block > 1:
        return (j // m.block) * m.block
    return j


def cdiv(a, b):
    return -(-a // b)


def fast_div(d: int):
    """(m, s) of attn_common.h fast_div: n / d = (mulhi(n, m) + n) >> s for n < 2^31."""
    d = max(d, 1)
    s = 0
    while (1 << s) < d:
        s += 1
    return ((1 << 32) * ((1 << s) - d)) // d + 1, s


def fdiv(n: int, f) -> int:
    m, s = f
    return (((n * m) >> 32) + n) >> s


def work_item(bid: int, nblk: int, BH: int, heavy_last: bool, blocks_fastest: bool = False):
    """blockIdx -> (bh, blk) (attn_common.h work_item, with its divisor work_item_div, or
    work_item_div_blocks when a head's row blocks go consecutively: non-causal launches)."""
    if blocks_fastest:
        if BH % 8 == 0:
            x, i = bid & 7, bid >> 3
            hh = fdiv(i, fast_div(nblk))
            return x + 8 * hh, i - hh * nblk
        bh = fdiv(bid, fast_div(nblk))
        return bh, bid - bh * nblk
    if BH % 8 == 0:
        x, i = bid & 7, bid >> 3
        blk = fdiv(i, fast_div(BH >> 3))
        bh = x + 8 * (i - blk * (BH >> 3))
    else:
        blk = fdiv(bid, fast_div(BH))
        bh = bid - blk * BH
    if heavy_last:
        blk = nblk - 1 - blk
    return bh, blk


def dkdv_work(bid: int, nblk: int, B: int, Hkv: int, group: int, nsplit: int,
              blocks_fastest: bool = False):
    """blockIdx -> (b, kv head, key block, first group head, group heads walked) of the
    16-bit dK/dV grid (attn_bwd16.hip): work_item over B*Hkv*nsplit "heads", whose index
    splits into (b*Hkv + kv head, group head) when the GQA group is split per query head."""
    bh, blk = work_item(bid, nblk, B * Hkv * nsplit, False, blocks_fastest)
    bhk = fdiv(bh, fast_div(group)) if nsplit > 1 else bh     # nsplit == group
    g_first = bh - bhk * nsplit if nsplit > 1 else 0
    g_count = 1 if nsplit > 1 else group
    b = fdiv(bhk, fast_div(Hkv))
    return b, bhk - b * Hkv, blk, g_first, g_count


# --------------------------------------------------------------------------- queries over keys
def _query_walk(m: Mask, BM: int, BN: int):
    """Yield (qw0, tw_begin, tw_end, q0) for every wave of the forward / dQ grid."""
    nblk = cdiv(m.S, BM)
    for qb in range(nblk):
        q0 = qb * BM
        kbeg, kend = 0, m.S
        if m.causal:
            kend = min(m.S, int(causal_key_end(m, q0 + BM - 1)) + 1)
        if m.window > 0:
            kbeg = max(0, q0 - m.window + 1)
        t_begin, t_end = kbeg // BN, cdiv(kend, BN)
        for wave in range(WAVES):
            qw0 = q0 + wave * WROWS
            tw_begin, tw_end = t_begin, t_end
            if qw0 >= m.S:
                tw_end = tw_begin
            if m.causal:
                tw_end = min(tw_end, int(causal_key_end(m, qw0 + WROWS - 1)) // BN + 1)
            if m.window > 0:
                tw_begin = max(tw_begin, max(0, qw0 - m.window + 1) // BN)
            yield qw0, tw_begin, tw_end, q0, t_begin, t_end


def _lane_bounds(m: Mask, qw0: int):
    qi = qw0 + np.arange(WROWS)
    key_hi = np.minimum(causal_key_end(m, qi), m.S - 1) if m.causal else np.full(WROWS, m.S - 1)
    key_lo = qi - m.window + 1 if m.window > 0 else np.zeros(WROWS, dtype=int)
    return qi, key_hi, key_lo


def _sink_visit(C, m: Mask, q0: int, qw0: int, half: int):
    """The folded-sink visit of the ceil(fold / 64) sink tiles before the ring, in
    pieces of `half` keys (forward: whole 64-key tiles; dQ: 32-key halves, those at or
    past `fold` skipped)."""
    if m.fold > 0 and q0 + FWD_BM - 1 >= m.window and qw0 < m.S and qw0 + WROWS - 1 >= m.window:
        qi = qw0 + np.arange(WROWS)
        n_i = np.maximum(0, np.minimum(m.fold, qi - m.window + 1))
        for kb in range(0, cdiv(m.fold, 64) * 64, half):
            if kb >= m.fold:
                continue
            k = kb + np.arange(half)
            C[qi[:, None], k[None, :]] += (k[None, :] <= (n_i - 1)[:, None])


def fwd_coverage(m: Mask) -> np.ndarray:
    """Unmasked (q, k) visits of attn_fwd16 (tile t of a wave: masks above key_hi
    when need_hi, below key_lo when need_lo)."""
    P = cdiv(m.S, FWD_BM) * FWD_BM
    C = np.zeros((P, cdiv(m.S, FWD_BN) * FWD_BN + FWD_BN), dtype=np.int32)
    for qw0, tw_begin, tw_end, q0, _, _ in _query_walk(m, FWD_BM, FWD_BN):
        _sink_visit(C, m, q0, qw0, FWD_BN)
        qi, key_hi, key_lo = _lane_bounds(m, qw0)
        wave_key_hi = int(causal_key_end(m, qw0)) if m.causal else m.S
        for t in range(tw_begin, tw_end):
            k0 = t * FWD_BN
            need_hi = (k0 + FWD_BN > m.S) or (m.causal and k0 + FWD_BN - 1 > wave_key_hi)
            need_lo = m.window > 0 and k0 <= qw0 + WROWS - 1 - m.window
            k = k0 + np.arange(FWD_BN)
            keep = np.ones((WROWS, FWD_BN), dtype=bool)
            if need_hi:
                keep &= k[None, :] <= key_hi[:, None]
            if need_lo:
                keep &= k[None, :] >= key_lo[:, None]
            C[qi[:, None], k[None, :]] += keep
    return C


def dq_coverage(m: Mask) -> np.ndarray:
    """Unmasked (q, k) visits of attn_bwd16_dq_kernel, 32-key halves skipped
    above the wave's diagonal and left of its window."""
    P = cdiv(m.S, DQ_BM) * DQ_BM
    C = np.zeros((P, cdiv(m.S, DQ_BN) * DQ_BN + DQ_BN), dtype=np.int32)
    for qw0, tw_begin, tw_end, q0, _, _ in _query_walk(m, DQ_BM, DQ_BN):
        _sink_visit(C, m, q0, qw0, 32)
        qi, key_hi, key_lo = _lane_bounds(m, qw0)
        wave_key_lo_end = int(causal_key_end(m, qw0)) if m.causal else m.S
        wave_key_hi_end = int(causal_key_end(m, qw0 + WROWS - 1)) if m.causal else m.S
        for t in range(tw_begin, tw_end):
            for mt in range(2):
                kb = t * DQ_BN + mt * 32
                if m.causal and kb > wave_key_hi_end:
                    continue
                if m.window > 0 and kb + 31 <= qw0 - m.window:
                    continue
                need_hi = (kb + 32 > m.S) or (m.causal and kb + 31 > wave_key_lo_end)
                need_lo = m.window > 0 and kb <= qw0 + WROWS - 1 - m.window
                k = kb + np.arange(32)
                keep = np.ones((WROWS, 32), dtype=bool)
                if need_hi:
                    keep &= k[None, :] <= key_hi[:, None]
                if need_lo:
                    keep &= k[None, :] >= key_lo[:, None]
                C[qi[:, None], k[None, :]] += keep
    return C


# --------------------------------------------------------------------------- keys over queries
def dkdv_ranges(m: Mask, blk: int):
    """(tq_begin, tq_end, [(kw0, tw_begin, tw_end) per wave]) of one dK/dV key block."""
    k0 = blk * DKDV_BK
    fs = m.fold
    qbeg, qend = 0, m.S
    if m.causal:
        qbeg = int(causal_query_begin(m, k0))
    if m.window > 0 and k0 >= fs:
        qend = min(m.S, k0 + DKDV_BK - 1 + m.window)
    tq_begin = qbeg // DKDV_BQ
    tq_end = max(tq_begin, cdiv(qend, DKDV_BQ))
    waves = []
    for wave in range(WAVES):
        kw0 = k0 + wave * WROWS
        tw_begin, tw_end = tq_begin, tq_end
        if kw0 >= m.S:
            tw_end = tw_begin
        if m.causal:
            tw_begin = max(tw_begin, int(causal_query_begin(m, kw0)) // DKDV_BQ)
        if m.window > 0 and kw0 >= fs:
            tw_end = min(tw_end, (kw0 + WROWS - 1 + m.window - 1) // DKDV_BQ + 1)
        waves.append((kw0, tw_begin, tw_end))
    return tq_begin, tq_end, waves


def dkdv_coverage(m: Mask, group: int = 1) -> np.ndarray:
    """Unmasked (q, k) visits of attn_bwd16_dkdv_kernel for one query head (the
    GQA loop repeats the same walk for each head of the group: its iteration
    `it` is (head it // ntq, query tile tq_begin + it % ntq))."""
    P = cdiv(m.S, DKDV_BQ) * DKDV_BQ + DKDV_BQ
    C = np.zeros((P, cdiv(m.S, DKDV_BK) * DKDV_BK), dtype=np.int32)
    for blk in range(cdiv(m.S, DKDV_BK)):
        tq_begin, tq_end, waves = dkdv_ranges(m, blk)
        ntq = tq_end - tq_begin
        for kw0, tw_begin, tw_end in waves:
            kj = kw0 + np.arange(WROWS)
            q_lo = causal_query_begin(m, kj) if m.causal else np.zeros(WROWS, dtype=int)
            wave_q_lo = int(causal_query_begin(m, kw0 + WROWS - 1)) if m.causal else 0
            if m.window > 0:
                q_hi = np.where(kj >= m.fold, np.minimum(m.S - 1, kj + m.window - 1), m.S - 1)
            else:
                q_hi = np.full(WROWS, m.S - 1)
            for it in range(group * ntq):
                head, tq = it // ntq, tq_begin + it % ntq
                if head != 0 or not (tw_begin <= tq < tw_end):
                    continue
                q0 = tq * DKDV_BQ
                need_lo = m.causal and q0 < wave_q_lo
                need_hi = (q0 + DKDV_BQ > m.S) or (m.window > 0 and q0 + DKDV_BQ - 1 - m.window >= kw0)
                q = q0 + np.arange(DKDV_BQ)
                keep = np.ones((DKDV_BQ, WROWS), dtype=bool)
                if need_lo:
                    keep &= q[:, None] >= q_lo[None, :]
                if need_hi:
                    keep &= q[:, None] <= q_hi[None, :]
                C[q[:, None], kj[None, :]] += keep
    return C


def extra_sinks(m: Mask, i):
    """Sinks query i sees beyond its window span (attn_sinks.hip extra_sinks)."""
    return np.maximum(0, np.minimum(m.sinks, i - m.window + 1))


def sink_pass_coverage(m: Mask) -> np.ndarray:
    """Pairs the separate sink kernels add (float32): rows i >= span, keys
    j < extra_sinks(i); active only while some query sees a sink beyond its
    span (attn_sinks.hip sinks_active)."""
    C = np.zeros((m.S, m.S), dtype=np.int32)
    if not (m.sinks > 0 and m.fold == 0 and 0 < m.window < m.S):
        return C
    i = np.arange(m.window, m.S)
    n = extra_sinks(m, i)
    j = np.arange(m.S)
    C[i[:, None], j[None, :]] += j[None, :] < n[:, None]
    return C


def total_coverage(m: Mask, kernel: str) -> np.ndarray:
    """[S, S] coverage of one pass (fwd / dq / dkdv) plus the separate sink pass."""
    C = {"fwd": fwd_coverage, "dq": dq_coverage, "dkdv": dkdv_coverage}[kernel](m)
    return C, sink_pass_coverage(m)


# --------------------------------------------------------------------------- entry masks
def crow_off(r: int) -> int:
    """Row offset of accumulator entry r within the lane group (attn_common.h)."""
    return 8 * (r >> 2) + (r & 3)


CROW_OFFS = [crow_off(r) for r in range(16)]
_U32 = 0xFFFFFFFF


def keep_upto(hi: int, cap: int = 28) -> int:
    """keep_upto() of attn_common.h: bits c <= hi of the offsets 0..27."""
    return ~((_U32 << min(max(hi + 1, 0), cap)) & _U32) & _U32


def keep_from(lo: int, cap: int = 28) -> int:
    """keep_from(): bits c >= lo."""
    return (_U32 << min(max(lo, 0), cap)) & _U32


def mask_keep(keep: int):
    """Entries that mask_keep() leaves: bit crow_off(r) of `keep`, sign-extended by
    v_bfe_i32 to all-ones or zero, then a bitwise select."""
    out = []
    for c in CROW_OFFS:
        bit = (keep >> c) & 1
        sel = _U32 if bit else 0                  # v_bfe_i32 x, keep, c, 1
        out.append(sel == _U32)
    return out


# --------------------------------------------------------------------------- LDS rings
def ring_fwd(t_begin: int, t_end: int, NS: int = FWD_NS):
    """Simulate the forward's ring: unit u = {K tile u+1, V tile u} lives in slot
    (u - t_begin + 1) % NS. Returns the list of (step tile, unit read, slot read,
    retired) for each step, checking the slot's occupant as the kernel assumes."""
    slots = {}
    issued = []                         # units in issue order
    for i in range(NS):                 # prologue: units t_begin - 1 + i into slot i
        u = t_begin - 1 + i
        if u <= t_end - 1:
            slots[i] = u
            issued.append(u)
    log = []
    for k, t in enumerate(range(t_begin, t_end)):
        allowed = min(NS - 2, t_end - 1 - t)      # wait_units(): in flight after the wait
        retired = issued[:len(issued) - allowed] if allowed > 0 else list(issued)
        sf, sr = k % NS, (k % NS + 1) % NS
        if t + NS - 1 <= t_end - 1:               # refill the slot freed by step k-1
            slots[sf] = t + NS - 1
            issued.append(t + NS - 1)
        log.append((t, slots.get(sr), sr, t in retired))
    return log


def ring_simple(n: int, NS: int):
    """dQ ring (and dK/dV at D = 128): unit u (a tile, or a (head, tile) iteration) in slot u % NS,
    NS - 1 issued ahead. Returns (unit, occupant of its slot, retired) per step."""
    slots, issued = {}, []
    for i in range(NS - 1):
        if i < n:
            slots[i] = i
            issued.append(i)
    log = []
    for it in range(n):
        allowed = min(NS - 2, n - 1 - it)
        retired = issued[:len(issued) - allowed] if allowed > 0 else list(issued)
        sl = it % NS
        if it + NS - 1 < n:
            slots[(sl + NS - 1) % NS] = it + NS - 1
            issued.append(it + NS - 1)
        log.append((it, slots.get(sl), it in retired))
    return log


def ring_pair(n: int, refill=lambda sl: ((sl + 2) % 4, (sl + 3) % 4)):
    """16-bit dK/dV ring at D <= 64: 4 slots, unit u in slot u % 4, two units per
    barrier. At step pair (it, it+1): wait for every issued unit, barrier, refill
    `refill(it % 4)` with units it+2 and it+3, then read units it and it+1.
    Returns (unit, occupant of its slot, retired) per step; raises if a refill
    overwrites a unit that is read after the barrier (a unit at or past `it`)."""
    slots, issued = {}, []
    for i in range(min(2, n)):
        slots[i] = i
        issued.append(i)
    log = []
    for it in range(0, n, 2):
        retired = list(issued)                  # wait_vm<0>() before the barrier
        for j, s in enumerate(refill(it % 4)):
            u = it + 2 + j
            if u < n:
                if slots.get(s, -1) >= it:
                    raise AssertionError(f"unit {u} overwrites unit {slots[s]} in slot {s} at step {it}")
                slots[s] = u
                issued.append(u)
        for u in (it, it + 1):
            if u < n:
                log.append((u, slots.get(u % 4), u in retired))
    return log


# --------------------------------------------------------------------------- decode
DEC_TARGET_GROUPS = 1024
DEC_MIN_SPLIT_BYTES = 256 * 1024
DEC_VALU_ROWS = 4


def decode_plan(dtype_bytes: int, B: int, T: int, H: int, Hkv: int, D: int, Lk: int):
    """dec_geometry (attn_decode.hip): the kernel kind, rows per unit, splits and
    key blocks per split, and the split-partial workspace floats."""
    R = T * (H // Hkv)
    if R <= 1:
        vr = 1
    elif dtype_bytes == 4:
        vr = 8
    else:
        vr = DEC_VALU_ROWS if R <= DEC_VALU_ROWS else 0
    target = DEC_TARGET_GROUPS
    if vr:
        epl = 16 // dtype_bytes
        lpk = D // epl
        ng = 256 // lpk
        nb = 8 if vr <= 1 else 4
        RT, BN, min_blocks = vr, ng * nb, 1
    else:
        RT, BN = 32, (32 if D >= 128 else 64)
        min_blocks = 4 if R > 32 else 8
        if R > 32:
            target = DEC_TARGET_GROUPS // 2
    ntiles = cdiv(R, RT)
    nblk = cdiv(Lk, BN)
    groups = cdiv(ntiles, 4) if (vr == 0 and R > 32) else ntiles
    units = B * Hkv * groups
    want = cdiv(target, units)
    unit_bytes = 2 * Lk * D * dtype_bytes
    cap = unit_bytes // DEC_MIN_SPLIT_BYTES
    if want > cap:
        want = cap if cap > 1 else 1
    want = max(1, min(want, nblk // min_blocks))
    bps = cdiv(nblk, want)
    nsplit = cdiv(nblk, bps)
    ws = 0
    if nsplit > 1:
        ws = B * Hkv * ntiles * nsplit * RT * (D * dtype_bytes // 4 + 2)
    splits = [(s * bps, min(nblk, s * bps + bps)) for s in range(nsplit)]
    return dict(RT=RT, BN=BN, ntiles=ntiles, nblk=nblk, bps=bps, nsplit=nsplit, splits=splits,
                workspace_floats=ws, valu_rows=vr)

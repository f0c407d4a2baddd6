"""The 16-bit kernels at the largest problem the C ABI accepts.

The host refuses S * H * D > 2^31 - 1 (``validate`` in ``csrc/capi.hip``), so
that every in-head byte offset of a 16-bit tensor fits the 32-bit buffer
offsets and ranges the kernels use (``RowTiles`` in ``csrc/attn16.h``); the
batch offset is 64-bit. These cases sit just under that bound, with two
batches so the second batch starts past 2^32 bytes, and check the result at
rows at the start, the middle and the end of the sequence.

A sliding window keeps them fast. It also makes each checked row's
dependencies local: query row c depends on keys [c - W + 1, c], and key row c
on queries [c, c + W - 1], whose own keys lie in [c - W + 1, c + W - 1]. So
the float64 oracle run on that slice of rows (all heads) gives O, LSE and dQ at
row c and dK, dV at key row c exactly; the gradients are compared against the
oracle backward given the kernel's stored O, as in the random sweep of
``test_gpu_parity.py``. Tolerances as everywhere: 2e-2 plus half an output ulp
element by element, LSE 1e-4.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from machinelearning_amd import flash_cuda as fc
from oracle import attention as orc
from tests import _parity

pytestmark = pytest.mark.gpu

LIMIT = 2**31 - 1

# (B, S, H, Hkv, D, window, dtype): S * H * D just under the limit.
CASES = [
    (2, 1_048_000, 16, 4, 128, 200, torch.bfloat16),
    (1, 1_048_000, 32, 32, 64, 64, torch.float16),
]


@pytest.fixture(scope="module", autouse=True)
def _library():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert fc.is_available(), fc.unavailable_reason()
    yield
    torch.cuda.empty_cache()   # tens of GB the later tests in this process do not need


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}_S{c[1]}_H{c[2]}-{c[3]}_D{c[4]}_w{c[5]}")
def test_largest_accepted_problem(case):
    B, S, H, Hkv, D, W, dtype = case
    assert 0 <= LIMIT - S * H * D < 1024 * H * D   # within 1024 rows of the limit
    print(f"max-size case B{B} S{S} H{H}/{Hkv} D{D} window {W} {dtype}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(31)
    q = torch.randn(B, S, H, D, device="cuda", dtype=dtype, generator=g).requires_grad_()
    k = torch.randn(B, S, Hkv, D, device="cuda", dtype=dtype, generator=g).requires_grad_()
    v = torch.randn(B, S, Hkv, D, device="cuda", dtype=dtype, generator=g).requires_grad_()
    do = torch.randn(B, S, H, D, device="cuda", dtype=dtype, generator=g)
    o, lse = fc.attn(q, k, v, True, W, None)
    dq, dk, dv = torch.autograd.grad(o, (q, k, v), do)
    torch.cuda.synchronize()
    assert torch.isfinite(lse).all()

    def rows(t, b, r0, r1):
        return t[b:b + 1, r0:r1].detach().double().cpu().numpy()

    for b in range(B):
        for c in (0, 1, W - 1, W, 4095, S // 2 + 7, S - W - 1, S - 2, S - 1):
            r0, r1 = max(0, c - W + 1), min(S, c + W)
            i = c - r0
            qs, ks, vs, dos = (rows(t, b, r0, r1) for t in (q, k, v, do))
            o_stored = rows(o, b, r0, r1)
            ro, rl = orc.forward(qs, ks, vs, None, True, W)
            rq, rk, rv = orc.backward(qs, ks, vs, o_stored, rl, dos, None, True, W)
            tag = f"max-size B{B} S{S} H{H}/{Hkv} D{D} w{W} {dtype} b{b} row {c}"
            got = {
                "O": o[b, c].detach().double().cpu().numpy(),
                "LSE": lse[b, :, c].detach().double().cpu().numpy(),
                "dQ": dq[b, c].double().cpu().numpy(),
                "dK": dk[b, c].double().cpu().numpy(),
                "dV": dv[b, c].double().cpu().numpy(),
            }
            want = {"O": ro[0, i], "LSE": rl[0, :, i], "dQ": rq[0, i], "dK": rk[0, i], "dV": rv[0, i]}
            for name in ("O", "LSE", "dQ", "dK", "dV"):
                _parity.check(tag, name, got[name], want[name], dtype)
    del q, k, v, do, o, lse, dq, dk, dv

"""HIP graph capture of the C ABI (torch.cuda.graph): the library enqueues kernels
only (no allocation, no memset, no host synchronisation), so a forward + backward
captured once replays on whatever the static buffers hold. Each case replays its
graph three times, with new inputs copied in and unrelated eager work between the
replays, and checks every replay against eager calls on the same inputs bit for bit.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

from machinelearning_amd import _capi
from machinelearning_amd import flash_cuda as fc

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _library():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    assert fc.is_available(), fc.unavailable_reason()
    yield


def _rand(B, T, H, Hkv, D, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(B, T, H, D, generator=g).to(dtype),
            torch.randn(B, T, Hkv, D, generator=g).to(dtype),
            torch.randn(B, T, Hkv, D, generator=g).to(dtype),
            torch.randn(B, T, H, D, generator=g).to(dtype))


# (name, B, T, H, Hkv, D, window, sinks, entry): "bwd" the caller-workspace
# backward, "res" the output-residual pair, "noalloc" the static-workspace one.
CASES = [
    ("causal", 2, 300, 4, 2, 64, 0, 0, "bwd"),
    ("gqa_split", 1, 260, 8, 1, 32, 0, 0, "bwd"),
    ("window_sinks", 2, 333, 4, 4, 64, 48, 5, "bwd"),
    ("residual_d128", 1, 257, 4, 2, 128, 0, 0, "res"),
    ("noalloc", 2, 200, 4, 2, 64, 0, 0, "noalloc"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: c[0])
def test_graph_replays_match_eager(case):
    name, B, T, H, Hkv, D, window, sinks, entry = case
    lib = _capi.load()
    dt = torch.bfloat16
    shp = _capi.shape(B, T, H, Hkv, D, True, window, D ** -0.5, _capi.MI_BF16, sinks)
    sp = ctypes.byref(shp)
    P = lambda t: None if t is None else t.data_ptr()
    q, k, v, do = (t.cuda() for t in _rand(B, T, H, Hkv, D, dt, seed=31))
    o, o_res = torch.empty_like(q), torch.empty_like(q)
    lse = torch.empty(B, H, T, device="cuda")
    ws = torch.empty(max(1, _capi.workspace_floats(shp)), device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)

    def run(st):
        if entry == "res":
            assert lib.mi_attn_fwd_res(P(q), P(k), P(v), P(o), P(o_res), P(lse), sp, st) == 0
            assert lib.mi_attn_bwd_res(P(q), P(k), P(v), P(o), P(o_res), P(do), P(lse), None,
                                       P(ws), P(dq), P(dk), P(dv), sp, st) == 0
            return
        assert lib.mi_attn_fwd(P(q), P(k), P(v), P(o), P(lse), sp, st) == 0
        if entry == "noalloc":
            assert lib.mi_attn_bwd_noalloc(P(q), P(k), P(v), P(o), P(do), P(lse), None, P(dq),
                                           P(dk), P(dv), sp, st) == 0
        else:
            assert lib.mi_attn_bwd(P(q), P(k), P(v), P(o), P(do), P(lse), None, P(ws), P(dq),
                                   P(dk), P(dv), sp, st) == 0

    # Warm-up on a side stream (first calls resolve the library's per-device state),
    # then capture.
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run(side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()

    outs = (o, lse, dq, dk, dv)
    for rep in range(3):
        for dst, src in zip((q, k, v, do), _rand(B, T, H, Hkv, D, dt, seed=40 + rep)):
            dst.copy_(src.cuda())
        graph.replay()
        torch.cuda.synchronize()
        got = [t.clone() for t in outs]
        # unrelated eager work between replays
        x = torch.randn(512, 512, device="cuda")
        (x @ x).sum().item()
        for t in outs:
            t.fill_(float("nan"))
        run(torch.cuda.current_stream().cuda_stream)
        torch.cuda.synchronize()
        want = [t.clone() for t in outs]
        for tname, a, b in zip(("o", "lse", "dq", "dk", "dv"), got, want):
            assert torch.isfinite(a.float()).all(), f"{name} replay {rep}: {tname} not finite"
            assert torch.equal(a, b), f"{name} replay {rep}: {tname} differs from eager"

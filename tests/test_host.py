"""Host-side logic that runs without a GPU: the C ABI library loads and exports
every symbol ``include/mi_attn.h`` declares, its argument validation (which
runs before any HIP call), and the Python gates mirrored from
``nanolab/flash_cuda.py`` (``supports``, ``effective_dtype``, error types).
"""

from __future__ import annotations

import ast
import ctypes
import pathlib
import re

import pytest
import torch

from machinelearning_amd import _capi
from machinelearning_amd import flash_cuda as fc

ROOT = pathlib.Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "mi_attn.h"


def _header_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^MI_API\s+[\w\s\*]+?\b(mi_\w+)\s*\(", text, flags=re.M)


def test_header_declares_the_abi():
    names = _header_functions()
    assert set(names) == set(_capi.SIGNATURES), (sorted(names), sorted(_capi.SIGNATURES))


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(str(_capi.LIB_PATH))
    for name in _header_functions():
        assert hasattr(lib, name), f"{name} not exported by {_capi.LIB_PATH.name}"
    assert _capi.load().mi_attn_abi_version() == _capi.ABI_VERSION


def test_gil_binding_per_entry_point():
    """The per-step fwd / bwd entry points keep the GIL (PyDLL); the ones that may
    block on the host and are off the autograd path release it (CDLL)."""
    lib = _capi.load()
    for name in _capi.SIGNATURES:
        keeps = bool(getattr(lib, name)._flags_ & ctypes._FUNCFLAG_PYTHONAPI)
        assert keeps == (name not in _capi.RELEASE_GIL), name
    assert {"mi_attn_bwd_noalloc", "mi_attn_decode", "mi_mfma_probe"} <= _capi.RELEASE_GIL
    assert "mi_attn_fwd" not in _capi.RELEASE_GIL and "mi_attn_bwd" not in _capi.RELEASE_GIL


def _shape(**kw):
    base = dict(B=2, S=128, H=4, Hkv=2, D=64, causal=True, window=0, scale=0.125,
                dtype=_capi.MI_BF16)
    base.update(kw)
    return _capi.shape(**base)


@pytest.mark.parametrize("kw,code", [
    ({}, 0),
    ({"D": 48}, 4),
    ({"D": 256}, 4),
    ({"dtype": 7}, 3),
    ({"H": 5, "Hkv": 2}, 2),
    ({"Hkv": 0}, 2),
    ({"B": -1}, 2),
    ({"window": -1}, 5),
    ({"window": 16, "causal": False}, 5),
    ({"window": 16}, 0),
    ({"window": 16, "sinks": 4}, 0),
    ({"window": 16, "sinks": 15}, 0),
    ({"window": 16, "sinks": 16}, 5),
    ({"window": 16, "sinks": -1}, 5),
    ({"sinks": 2}, 5),
    ({"block": 64}, 0),
    ({"block": 1, "causal": False}, 0),
    ({"block": 64, "causal": False}, 5),
    ({"block": 64, "window": 16}, 5),
    ({"block": -1}, 5),
    ({"causal": False}, 0),
    ({"scale": float("inf")}, 9),
    ({"scale": float("nan")}, 9),
    ({"scale": 0.0}, 9),
    ({"scale": -0.125}, 9),
    ({"B": 0}, 0),
    # S * H * D at the 2^31 bound of the kernels' 32-bit in-head offsets
    ({"B": 2, "S": 1_048_000, "H": 16, "Hkv": 4, "D": 128}, 0),
    ({"B": 2, "S": 1_048_575, "H": 16, "Hkv": 4, "D": 128}, 0),
    ({"B": 2, "S": 1_048_576, "H": 16, "Hkv": 4, "D": 128}, 7),
])
def test_shape_validation(kw, code):
    lib = _capi.load()
    assert lib.mi_attn_check(ctypes.byref(_shape(**kw))) == code
    assert lib.mi_attn_error_string(code)


def test_entry_points_reject_before_touching_the_device():
    lib = _capi.load()
    bad = _shape(D=48)
    assert lib.mi_attn_fwd(None, None, None, None, None, ctypes.byref(bad), None) == 4
    ok = _shape()
    # valid shape, NULL buffers -> MI_ERR_NULL, no launch
    assert lib.mi_attn_fwd(None, None, None, None, None, ctypes.byref(ok), None) == 1
    assert lib.mi_attn_bwd(*([None] * 11), ctypes.byref(ok), None) == 1
    assert lib.mi_attn_bwd_dkdv(*([None] * 8), ctypes.byref(ok), None) == 1
    assert lib.mi_attn_bwd_dq(*([None] * 7), ctypes.byref(ok), None) == 1
    assert lib.mi_attn_bwd_delta(*([None] * 5), ctypes.byref(ok), None) == 1
    # misaligned pointers are refused before any launch
    assert lib.mi_attn_fwd(8, 16, 16, 16, 16, ctypes.byref(ok), None) == 6
    # an empty problem is a no-op success
    empty = _shape(S=0)
    assert lib.mi_attn_fwd(None, None, None, None, None, ctypes.byref(empty), None) == 0
    assert lib.mi_mfma_probe_k(_capi.MI_BF16) == 16
    assert lib.mi_mfma_probe_k(_capi.MI_F32) == 2
    assert lib.mi_mfma_probe(None, None, None, 0, None) == 1
    with pytest.raises(RuntimeError, match="head_dim"):
        _capi.check(4)


def test_effective_dtype_mirrors_autocast():
    """nanolab/tests.py:485-495."""
    q = torch.randn(1, 8, 2, 32)
    assert fc.effective_dtype(q, q, q) is torch.float32
    assert fc.effective_dtype(q, q, q.to(torch.bfloat16)) is None
    assert not fc.supports(q, q, q), "CPU tensors are not for this kernel"


def test_flash_attn_refuses_cpu_tensors():
    q = torch.randn(1, 8, 2, 32)
    with pytest.raises(ValueError, match="unsupported inputs"):
        fc.flash_attn(q, q, q, 0.1)
    with pytest.raises(ValueError):
        fc.attn(q, q, q, True, 4)


def test_reason_strings_without_a_gpu(monkeypatch):
    for name, val in (("_load_attempted", False), ("_lib", None), ("_load_error", None)):
        monkeypatch.setattr(fc, name, val)
    monkeypatch.setenv("NANOLAB_FLASH_CUDA", "0")
    assert not fc.is_available()
    assert fc.unavailable_reason() == "disabled by NANOLAB_FLASH_CUDA=0"
    assert not fc.mma_available()
    assert fc.mma_unavailable_reason() == fc.unavailable_reason()
    if not torch.cuda.is_available():
        monkeypatch.setattr(fc, "_load_attempted", False)
        monkeypatch.delenv("NANOLAB_FLASH_CUDA")
        assert not fc.is_available() and fc.unavailable_reason() == "no GPU device"


def test_public_surface_matches_the_reference_module():
    """The names nanolab's callers and tests use (nanolab/flash_cuda.py)."""
    for name in ("supports", "is_available", "unavailable_reason", "mma_available",
                 "mma_unavailable_reason", "effective_dtype", "flash_attn", "sdpa_reference",
                 "SUPPORTED_HEAD_DIMS", "SUPPORTED_DTYPES", "MMA_DTYPES", "MMA_BWD_HEAD_DIMS",
                 "main"):
        assert hasattr(fc, name), name
    assert fc.SUPPORTED_HEAD_DIMS == (32, 64, 128)
    import inspect
    params = list(inspect.signature(fc.flash_attn).parameters)
    assert params[:5] == ["q", "k", "v", "scale", "use_mma"]          # positional order kept
    assert inspect.signature(fc.flash_attn).parameters["causal"].kind.name == "KEYWORD_ONLY"
    assert list(inspect.signature(fc.attn).parameters)[:6] == ["q", "k", "v", "causal", "window",
                                                               "scale"]


def test_product_never_imports_the_oracle():
    """The oracle is test infrastructure: no module of the package may import it."""
    for path in (ROOT / "machinelearning_amd").rglob("*.py"):
        tree = ast.parse(path.read_text())
        for node in ast.walk(tree):
            if isinstance(node, ast.Import):
                mods = [a.name for a in node.names]
            elif isinstance(node, ast.ImportFrom):
                mods = [node.module or ""]
            else:
                continue
            assert not any(m == "oracle" or m.startswith("oracle.") for m in mods), path


def test_kernel_sources_have_no_compat_layers():
    """CDNA4 code written directly: no CUDA shims / dual-platform switches."""
    for path in (ROOT / "machinelearning_amd" / "csrc").glob("*"):
        text = path.read_text()
        for bad in ("__HIP_PLATFORM_AMD__", "cuda_runtime", "__CUDA_ARCH__", "hipify"):
            assert bad not in text, f"{path.name} mentions {bad}"


def test_backward_workspace_size():
    """[2,B,H,S] planes, plus the sink pass's partial sums when a sink is beyond the span
    and the sink kernels add it: float32. 16-bit window kernels visit the sinks
    themselves, at any count. (Hkv == H here: the GQA split partials are pinned by
    test_backward_workspace_gqa_split.)"""
    def floats(**kw):
        kw.setdefault("Hkv", 4)
        return _capi.workspace_floats(_shape(**kw))
    f32 = _capi.MI_F32
    planes = 2 * 2 * 4 * 128
    assert floats() == planes
    assert floats(window=16) == planes
    for window, sinks in ((130, 4), (40, 32), (100, 65), (127, 120), (16, 4)):
        assert floats(window=window, sinks=sinks) == planes
    assert floats(window=130, sinks=4, dtype=f32) > planes   # span 126 < S: rows 126, 127
    assert floats(window=100, sinks=65, dtype=f32) > planes
    # (B*Hkv units) * chunks * sinks * {dK, dV} * D
    extra = floats(window=16, sinks=4, dtype=f32) - planes
    assert extra > 0 and extra % (2 * 2 * 4 * 2 * 64) == 0
    assert floats(window=200, sinks=4, dtype=f32) == planes   # span >= S: no sink beyond it
    assert floats(S=0, window=16, sinks=4, dtype=f32) == 0
    n = ctypes.c_longlong(-1)
    assert _capi.load().mi_attn_bwd_workspace(ctypes.byref(_shape(window=16, sinks=16)),
                                              ctypes.byref(n)) == 5
    assert _capi.load().mi_attn_bwd_workspace(ctypes.byref(_shape()), None) == 1


def test_backward_workspace_gqa_split():
    """16-bit GQA backward whose grid of (batch, kv head, 128-key block) workgroups is
    under two rounds of the chip at the dK/dV kernel's occupancy (the device's CUs --
    256 when no GPU is visible, as here -- x two workgroups for D <= 64, x one for D =
    128): the dK/dV walk is split per query head and the workspace grows by fp32
    partials [B*H][nblk*128][2][D], after the planes rounded up to 64 floats, as long
    as the partials take at most 16M floats (64 MiB). float32, Hkv == H, large grids
    and larger partials take no partials."""
    def floats(**kw):
        return _capi.workspace_floats(_shape(**kw))
    f32 = _capi.MI_F32

    def split(B, S, H, D, base):
        nblk = -(-S // 128)
        return -(-base // 64) * 64 + B * H * nblk * 128 * 2 * D

    # B2 S128 H4/Hkv2 D64: 2*2*1 = 4 workgroups -> split.
    assert floats() == split(2, 128, 4, 64, 2 * 2 * 4 * 128)
    assert floats(dtype=_capi.MI_F16) == floats()
    assert floats(dtype=f32) == 2 * 2 * 4 * 128
    assert floats(Hkv=4) == 2 * 2 * 4 * 128
    # Odd planes (S = 127): the partials start on a 64-float boundary.
    assert floats(S=127) == split(2, 127, 4, 64, 2 * 2 * 4 * 127)
    # 16-bit sinks fold into the window kernels at any count (no sink partials), so
    # the partials follow the planes; float32 keeps the sink partials and no split.
    assert floats(window=100, sinks=65) == split(2, 128, 4, 64, 2 * 2 * 4 * 128)
    assert floats(window=100, sinks=65, dtype=f32) > 2 * 2 * 4 * 128
    # The grid bound: D <= 64 splits below 1024 workgroups (B*Hkv*nblk), D = 128 below 512.
    assert floats(B=511, S=256, H=2, Hkv=1, D=32) == split(511, 256, 2, 32, 2 * 511 * 2 * 256)
    assert floats(B=512, S=256, H=2, Hkv=1, D=32) == 2 * 512 * 2 * 256
    assert floats(B=64, S=256, H=2, Hkv=1, D=128) == split(64, 256, 2, 128, 2 * 64 * 2 * 256)
    assert floats(B=256, S=256, H=2, Hkv=1, D=128) == 2 * 256 * 2 * 256
    # The partials cap: B511 S256 H2/1 D64 is under the grid bound (1022 workgroups)
    # but its partials (33.5M floats) exceed 16M, so it runs unsplit; so does the
    # long-context MQA shape B1 H32/Hkv1 S32768 D128 (256 workgroups, partials of
    # 268M floats = 1.07 GB, where the unsplit kernel needs none).
    assert floats(B=511, S=256, H=2, Hkv=1) == 2 * 511 * 2 * 256
    assert floats(B=1, S=32768, H=32, Hkv=1, D=128) == 2 * 32 * 32768
    # The reference's E17 shape (B8 T1024 H12/Hkv4 D32): 256 workgroups -> split.
    assert floats(B=8, S=1024, H=12, Hkv=4, D=32) == split(8, 1024, 12, 32, 2 * 8 * 12 * 1024)

"""ctypes binding of libmi_attn.so's C ABI (include/mi_attn.h).

The thinnest possible layer: torch owns the memory (outputs and workspaces
are torch tensors allocated by the caller), this module passes raw device
pointers, the shape struct and the current HIP stream, and turns a non-zero
status into a ``RuntimeError`` carrying the library's own message.
"""

from __future__ import annotations

import ctypes
import pathlib

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libmi_attn.so"
ABI_VERSION = 10

MI_F32, MI_F16, MI_BF16 = 0, 1, 2


class MiAttnShape(ctypes.Structure):
    """Mirror of ``mi_attn_shape``."""

    _fields_ = [
        ("B", ctypes.c_int),
        ("S", ctypes.c_int),
        ("H", ctypes.c_int),
        ("Hkv", ctypes.c_int),
        ("D", ctypes.c_int),
        ("causal", ctypes.c_int),
        ("window", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("dtype", ctypes.c_int),
        ("sinks", ctypes.c_int),
        ("block", ctypes.c_int),
    ]


class MiPrologueShape(ctypes.Structure):
    """Mirror of ``mi_prologue_shape``."""

    _fields_ = [
        ("B", ctypes.c_int),
        ("T", ctypes.c_int),
        ("H", ctypes.c_int),
        ("D", ctypes.c_int),
        ("dtype_in", ctypes.c_int),
        ("dtype_out", ctypes.c_int),
        ("norm", ctypes.c_int),
        ("rope", ctypes.c_int),
        ("eps", ctypes.c_float),
    ]


class MiDecodeShape(ctypes.Structure):
    """Mirror of ``mi_decode_shape``."""

    _fields_ = [
        ("B", ctypes.c_int),
        ("T", ctypes.c_int),
        ("H", ctypes.c_int),
        ("Hkv", ctypes.c_int),
        ("D", ctypes.c_int),
        ("cached", ctypes.c_int),
        ("start", ctypes.c_int),
        ("causal", ctypes.c_int),
        ("window", ctypes.c_int),
        ("sinks", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("dtype", ctypes.c_int),
        ("k_batch_stride", ctypes.c_longlong),
        ("k_head_stride", ctypes.c_longlong),
        ("v_batch_stride", ctypes.c_longlong),
        ("v_head_stride", ctypes.c_longlong),
    ]


_P = ctypes.c_void_p
_SHAPE = ctypes.POINTER(MiAttnShape)
_PSHAPE = ctypes.POINTER(MiPrologueShape)
_DSHAPE = ctypes.POINTER(MiDecodeShape)

# name -> (restype, argtypes); the exported surface of include/mi_attn.h.
SIGNATURES = {
    "mi_attn_check": (ctypes.c_int, [_SHAPE]),
    "mi_attn_bwd_workspace": (ctypes.c_int, [_SHAPE, ctypes.POINTER(ctypes.c_longlong)]),
    "mi_attn_fwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _SHAPE, _P]),
    "mi_attn_bwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SHAPE, _P]),
    "mi_attn_bwd_delta": (ctypes.c_int, [_P, _P, _P, _P, _P, _SHAPE, _P]),
    "mi_attn_bwd_noalloc": (ctypes.c_int, [_P] * 10 + [_SHAPE, _P]),
    "mi_attn_fwd_res": (ctypes.c_int, [_P] * 6 + [_SHAPE, _P]),
    "mi_attn_bwd_res": (ctypes.c_int, [_P] * 12 + [_SHAPE, _P]),
    "mi_attn_fwd_gated": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _SHAPE, _P]),
    "mi_attn_bwd_gated": (ctypes.c_int, [_P] * 14 + [_SHAPE, _P]),
    "mi_attn_bwd_delta_gated": (ctypes.c_int, [_P] * 8 + [_SHAPE, _P]),
    "mi_attn_bwd_dkdv": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _SHAPE, _P]),
    "mi_attn_bwd_dq": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _SHAPE, _P]),
    "mi_qk_prologue_fwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _PSHAPE, _P]),
    "mi_qk_prologue_workspace": (ctypes.c_int, [_PSHAPE, ctypes.POINTER(ctypes.c_longlong)]),
    "mi_qk_prologue_bwd": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _PSHAPE, _P]),
    "mi_attn_decode_workspace": (ctypes.c_int, [_DSHAPE, ctypes.POINTER(ctypes.c_longlong)]),
    "mi_attn_decode": (ctypes.c_int, [_P] * 10 + [_DSHAPE, _P]),
    "mi_mfma_probe": (ctypes.c_int, [_P, _P, _P, ctypes.c_int, _P]),
    "mi_mfma_probe_k": (ctypes.c_int, [ctypes.c_int]),
    "mi_attn_error_string": (ctypes.c_char_p, [ctypes.c_int]),
    "mi_attn_abi_version": (ctypes.c_int, []),
}

_lib = None

# Entry points that may block or run long on the host (the first call's code-object
# load, hipGetSymbolAddress, a launch that waits for queue space) and that are not on
# the per-step autograd path: called through ctypes.CDLL, which releases the GIL.
RELEASE_GIL = frozenset({"mi_attn_bwd_noalloc", "mi_attn_decode", "mi_attn_decode_workspace",
                         "mi_mfma_probe", "mi_mfma_probe_k"})


class _Lib:
    """The library's entry points as attributes, each bound through PyDLL (keeps the
    GIL) or, for the names in RELEASE_GIL, CDLL (releases it)."""


def load() -> _Lib:
    """Load the in-tree library once; raises OSError if it is missing or stale."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise OSError(f"{LIB_PATH} is not built (run machinelearning_amd.build_ext.build())")
    # PyDLL, not CDLL, for the fwd / bwd entry points: calls keep the GIL. They only
    # validate and enqueue work on a stream (no host synchronisation), so nothing
    # blocks while the GIL is held, and the backward -- which torch's autograd engine
    # runs on its own device thread -- does not hand the GIL to the waiting main
    # thread and back at every call (measured: that handoff cost more than the calls
    # themselves). The others (RELEASE_GIL) go through CDLL, so other Python threads
    # (data loading) run while they wait.
    held = ctypes.PyDLL(str(LIB_PATH))
    released = ctypes.CDLL(str(LIB_PATH))
    lib = _Lib()
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(released if name in RELEASE_GIL else held, name)
        fn.restype = res
        fn.argtypes = args
        setattr(lib, name, fn)
    ver = lib.mi_attn_abi_version()
    if ver != ABI_VERSION:
        raise OSError(f"{LIB_PATH} has ABI version {ver}, this binding expects {ABI_VERSION}")
    _lib = lib
    return lib


def shape(B: int, S: int, H: int, Hkv: int, D: int, causal: bool, window: int, scale: float,
          dtype: int, sinks: int = 0, block: int = 0) -> MiAttnShape:
    return MiAttnShape(int(B), int(S), int(H), int(Hkv), int(D), 1 if causal else 0,
                       int(window), float(scale), int(dtype), int(sinks), int(block))


class ShapeCache:
    """Shape structs (and their backward workspace sizes) by shape key, bounded.

    A training step repeats a handful of shapes; building the ctypes struct and
    querying the workspace size once per shape keeps them off the per-call path.
    Entries are never mutated after creation (the library only reads them).
    """

    def __init__(self, limit: int = 1024):
        self.limit = limit
        self.entries: dict = {}

    def get(self, key: tuple):
        hit = self.entries.get(key)
        if hit is None:
            shp = shape(*key)
            ref = ctypes.byref(shp)
            n = ctypes.c_longlong(0)
            check(load().mi_attn_bwd_workspace(ref, ctypes.byref(n)))
            hit = (shp, ref, int(n.value))
            if len(self.entries) >= self.limit:
                self.entries.clear()
            self.entries[key] = hit
        return hit


def workspace_floats(shp: MiAttnShape) -> int:
    """Floats of backward workspace ``shp`` needs (mi_attn_bwd_workspace)."""
    n = ctypes.c_longlong(0)
    check(load().mi_attn_bwd_workspace(ctypes.byref(shp), ctypes.byref(n)))
    return int(n.value)


def decode_workspace_floats(shp: MiDecodeShape) -> int:
    """Floats of split-partial workspace a decode step needs (mi_attn_decode_workspace)."""
    n = ctypes.c_longlong(0)
    check(load().mi_attn_decode_workspace(ctypes.byref(shp), ctypes.byref(n)))
    return int(n.value)


def error_string(status: int) -> str:
    return load().mi_attn_error_string(int(status)).decode()


def check(status: int) -> None:
    """Raise RuntimeError for a non-zero mi_status."""
    if status != 0:
        raise RuntimeError(error_string(status))

"""Tolerances and error records shared by the GPU parity tests.

The bar: float32 results within 1e-5 max-abs, 16-bit
results within 2e-2 max-abs of the float64 oracle evaluated on the same
rounded inputs, LSE within 1e-4.

For 16-bit outputs the bound is applied element by element:

    |got_i - ref_i| <= 2e-2 + half_ulp(ref_i)

where half_ulp(x) is half a unit in the last place of the OUTPUT format at
|x| (bf16: 2^(floor(log2|x|) - 8)). That term is the rounding every bf16
result of magnitude |x| carries, however exact the arithmetic before it; it
is not widened by the tensor's maximum, so small elements keep a bound of
about 2e-2.

Where gradients are small (the board config draws dO ~ N(0, 1e-2), so
max|dQ| is ~1.9e-2 and an all-zero dQ would sit inside 2e-2 absolute), the
tests add a relative bound, max|err| / max|ref| <= REL_GRAD.

Every comparison can be logged: with MI_PARITY_LOG=<path> set, one JSON
line per (case, tensor) is appended there with the measured max error, the
largest err/tol ratio and the tensor's magnitude.
"""

from __future__ import annotations

import json
import math
import os

import numpy as np
import torch

ABS16 = 2e-2
ABS32 = 1e-5
LSE_TOL = 1e-4
REL_GRAD = 2e-2

_MANT = {torch.bfloat16: 7, torch.float16: 10}


def half_ulp(x: np.ndarray, dtype) -> np.ndarray:
    """Half an ulp of the 16-bit format at |x|, element by element (0 at x == 0)."""
    a = np.abs(np.asarray(x, dtype=np.float64))
    out = np.zeros_like(a)
    nz = a > 0
    out[nz] = np.exp2(np.floor(np.log2(a[nz])) - _MANT[dtype] - 1)
    return out


def tol16(ref: np.ndarray, dtype) -> np.ndarray:
    """Element-wise 16-bit bound: 2e-2 plus the output format's half-ulp at |ref_i|."""
    return ABS16 + half_ulp(ref, dtype)


def record(tag: str, name: str, **stats) -> None:
    path = os.environ.get("MI_PARITY_LOG")
    if not path:
        return
    with open(path, "a") as f:
        f.write(json.dumps({"case": tag, "tensor": name, **stats}) + "\n")


def check(tag: str, name: str, got: np.ndarray, ref: np.ndarray, dtype,
          rel: float | None = None, extra: np.ndarray | None = None) -> None:
    """Assert got ~ ref at the bar for `dtype` (name "LSE" takes the LSE bound).

    rel: additionally require max|err| / max|ref| <= rel.
    extra: an element-wise allowance added to the bound (the rounding of 16-bit
    MMA operands, where a caller accounts for it).
    """
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{tag} {name}: shape {got.shape} != {ref.shape}"
    if ref.size == 0:
        return
    err = np.abs(got - ref)
    assert np.isfinite(got).all(), f"{tag} {name}: non-finite result"
    amax = float(np.abs(ref).max())
    if name == "LSE":
        tol = np.full_like(err, LSE_TOL)
    elif dtype in _MANT:
        tol = tol16(ref, dtype)
    else:
        tol = np.full_like(err, ABS32)
    if extra is not None:
        tol = tol + np.asarray(extra, dtype=np.float64)
    ratio = err / tol
    worst = int(np.argmax(ratio))
    emax = float(err.max())
    rmax = float(ratio.flat[worst])
    relerr = emax / amax if amax > 0 else 0.0
    print(f"{tag} {name}: max|err|={emax:.3e} worst err/tol={rmax:.3f} "
          f"(|ref|={abs(float(ref.flat[worst])):.3e} there) max|ref|={amax:.3e} "
          f"rel={relerr:.2e}", flush=True)
    record(tag, name, max_err=emax, worst_ratio=rmax, max_ref=amax, rel_err=relerr,
           dtype=str(dtype).replace("torch.", ""))
    assert rmax < 1.0, (f"{tag}: {name} |err| {float(err.flat[worst]):.3e} > tol "
                        f"{float(tol.flat[worst]):.3e} at |ref| {abs(float(ref.flat[worst])):.3e}")
    if rel is not None:
        assert relerr <= rel, f"{tag}: {name} max|err|/max|ref| {relerr:.3e} > {rel:.1e}"


def scalar_tol16(ref: np.ndarray, dtype) -> float:
    """The loosest element bound of a tensor (for summaries that print one number)."""
    if ref.size == 0:
        return ABS16
    amax = float(np.abs(ref).max())
    return ABS16 + (0.0 if amax == 0 else 2.0 ** (math.floor(math.log2(amax)) - _MANT[dtype] - 1))

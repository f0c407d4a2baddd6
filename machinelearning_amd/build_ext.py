"""Build libmi_attn.so (the HIP kernels + C ABI) in-tree with hipcc for gfx950.

Each ``csrc/*.hip`` file is compiled to an object in parallel, then linked into
``machinelearning_amd/libmi_attn.so``. The library links only the HIP runtime:
no torch headers, so the build needs nothing but ``hipcc``.

    python -m machinelearning_amd.build_ext          # build (always recompiles)
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libmi_attn.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Packed FP32 VALU ops stay off: the compiler must not form v_pk_{add,mul,fma}_f32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: without this the backend picks the
    # AGPR form and copies every score / output tile between register files
    # (v_accvgpr_read/write) around the softmax, ~64 VALU ops per key tile.
    "-mllvm", "-amdgpu-mfma-vgpr-form",
]


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found; the HIP extension cannot be built")
    return exe


def sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stderr}")


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every csrc/*.hip and link libmi_attn.so. Returns the library path."""
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    srcs = sources()
    objs = [objdir / (s.stem + ".o") for s in srcs]
    workers = min(len(srcs), max(1, (os.cpu_count() or 2)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as ex:
        futs = [ex.submit(_compile, s, o) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link of {LIB.name} failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)

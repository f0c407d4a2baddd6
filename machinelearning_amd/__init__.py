"""machinelearning_amd -- MI355X-native flash attention for nanolab's ``--flash_cuda`` path.

``flash_cuda`` is the drop-in module (same names and behaviour as
``nanolab/flash_cuda.py``); ``libmi_attn.so`` below it holds the hand-written
gfx950 HIP kernels behind the C ABI declared in ``include/mi_attn.h``.
"""

from . import flash_cuda  # noqa: F401

__all__ = ["flash_cuda"]

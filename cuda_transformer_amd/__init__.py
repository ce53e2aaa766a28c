"""MI355X-native (gfx950) FP32 transformer kernels behind the reference's operator API.

Importing this package loads ``_C`` — the ``cuda_transformer`` torch operator library — which
calls the hand-written HIP kernels in ``libcuda_transformer_amd.so`` through their C ABI
(``include/cuda_transformer_amd.h``).  There is no CPU or eager fallback: if the native
library is not built the import fails, and the operators only have GPU implementations.
"""
from pathlib import Path

import torch  # noqa: F401  (the operator library registers into torch's dispatcher)

_PKG = Path(__file__).resolve().parent
_MISSING = [p.name for p in (_PKG / "_C.so", _PKG / "libcuda_transformer_amd.so") if not p.exists()]
if _MISSING:
    raise ImportError(
        f"cuda_transformer_amd native libraries not built ({', '.join(_MISSING)}); "
        "run `python cuda_transformer_amd/build.py`"
    )

from . import _C  # noqa: E402,F401  registers torch.ops.cuda_transformer.*
from . import ops  # noqa: E402,F401

__all__ = ["ops"]

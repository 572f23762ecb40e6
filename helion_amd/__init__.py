"""MI355X-native (gfx950 HIP) implementation of the ``tritium.ops`` kernel layer.

A drop-in for alkinun/helion ``tritium`` (``tritium/__init__.py:4-70``): the
hot-path ops keep the reference's names, signatures, validation messages and
autograd behaviour, and run hand-written HIP kernels from
``libtritium_hip.so`` through a C ABI (``include/tritium_hip.h``).  Use it as

    import helion_amd as tritium

torch is imported first on purpose: the kernel library binds to torch's HIP
runtime (see ``_lib.py``).
"""

from __future__ import annotations

import torch  # noqa: F401  (must be loaded before libtritium_hip.so)

from .adamw import adamw_step, adamw_step_multi
from .attention import attention
from .linear_ce import linear_cross_entropy, linear_cross_entropy_backward
from .matmul import matmul, matmul_vec
from .rmsnorm import residual_rmsnorm, rmsnorm, rmsnorm_backward
from .rope import rope, rope_
from .swiglu import swiglu, swiglu_backward

__version__ = "0.1.0"

__all__ = [
    "__version__",
    "adamw_step",
    "adamw_step_multi",
    "attention",
    "linear_cross_entropy",
    "linear_cross_entropy_backward",
    "matmul",
    "matmul_vec",
    "residual_rmsnorm",
    "rmsnorm",
    "rmsnorm_backward",
    "rope",
    "rope_",
    "swiglu",
    "swiglu_backward",
]

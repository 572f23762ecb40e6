"""MI355X-native (gfx950 HIP) implementation of the ``tritium.ops`` kernel layer.

A drop-in for alkinun/helion ``tritium`` (``tritium/__init__.py:4-70``): all
27 public names keep the reference's signatures, validation messages and
autograd behaviour.  The hot-path ops (attention, linear-cross-entropy,
RMSNorm, RoPE, SwiGLU, AdamW) and the logits ``cross_entropy`` run
hand-written HIP kernels from ``libtritium_hip.so`` through a C ABI
(``include/tritium_hip.h``); ``matmul`` runs the vendor GEMM, and the ops the
model path never calls (add/relu/gelu/dropout/softmax/layernorm/sgd) run as
PyTorch GPU operations.  Use it as

    import helion_amd as tritium

torch is imported first on purpose: the kernel library binds to torch's HIP
runtime (see ``_lib.py``).
"""

from __future__ import annotations

import torch  # noqa: F401  (must be loaded before libtritium_hip.so)

from .adamw import adamw_step, adamw_step_multi
from .attention import attention
from .cross_entropy import cross_entropy, cross_entropy_backward
from .elementwise import (
    add,
    add_gelu,
    add_relu,
    dropout,
    dropout_backward,
    gelu,
    gelu_backward,
    relu,
    sgd_step,
)
from .linear_ce import linear_cross_entropy, linear_cross_entropy_backward
from .matmul import matmul, matmul_vec
from .norms_extra import layernorm, layernorm_backward, softmax, softmax_backward
from .rmsnorm import residual_rmsnorm, rmsnorm, rmsnorm_backward
from .rope import rope, rope_
from .swiglu import swiglu, swiglu_backward

__version__ = "0.1.0"

__all__ = [
    "__version__",
    "add",
    "add_gelu",
    "add_relu",
    "adamw_step",
    "adamw_step_multi",
    "attention",
    "cross_entropy",
    "cross_entropy_backward",
    "dropout",
    "dropout_backward",
    "gelu",
    "gelu_backward",
    "layernorm",
    "layernorm_backward",
    "linear_cross_entropy",
    "linear_cross_entropy_backward",
    "matmul",
    "matmul_vec",
    "relu",
    "rope",
    "rope_",
    "residual_rmsnorm",
    "rmsnorm",
    "rmsnorm_backward",
    "sgd_step",
    "softmax",
    "softmax_backward",
    "swiglu",
    "swiglu_backward",
]

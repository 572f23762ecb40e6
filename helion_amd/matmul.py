"""``tritium.matmul`` / ``tritium.matmul_vec`` on the vendor GEMM.

The reference implements these with an autotuned Triton GEMM and GEMV
(``tritium/ops/matmul.py:336-347``); they are what ``helion.Linear`` calls
(``helion/nn.py:56-65``).  They are plain library GEMMs, so here they run on
hipBLASLt through ``torch.mm`` (fp32 accumulation, output in the inputs'
dtype), keeping the reference's names, signatures, validation messages
(``matmul.py:132-190``) and autograd contract (``matmul.py:311-340``: forward
alone without autograd, ``needs_input_grad`` honoured, a non-contiguous
upstream gradient made contiguous).  ``matmul_vec`` with autograd goes
through ``matmul`` on a one-row matrix, as the reference does
(``matmul.py:343-347``).
"""

from __future__ import annotations

from typing import Any

import torch

from ._utils import FLOAT_DTYPES, check_cuda_tensor, check_supported_dtype, requires_autograd

__all__ = ["matmul", "matmul_vec"]


def _check_pair(a: torch.Tensor, b: torch.Tensor, a_dim: int, a_shape: str) -> None:
    """matmul.py:132-190: CUDA, dtype, rank, K match, same dtype and device."""
    check_cuda_tensor("a", a)
    check_cuda_tensor("b", b)
    check_supported_dtype("a", a, FLOAT_DTYPES)
    check_supported_dtype("b", b, FLOAT_DTYPES)
    if a.dim() != a_dim:
        raise ValueError(f"a must be a {a_dim}D tensor shaped {a_shape}.")
    if b.dim() != 2:
        raise ValueError("b must be a 2D tensor shaped (K, N).")
    if a.shape[-1] != b.shape[0]:
        raise ValueError(
            f"Shape mismatch: a has shape {tuple(a.shape)}, b has shape {tuple(b.shape)}."
        )
    if a.dtype != b.dtype:
        raise ValueError(f"Dtype mismatch: a has dtype {a.dtype}, b has dtype {b.dtype}.")
    if a.device != b.device:
        raise ValueError(f"Device mismatch: a is on {a.device}, b is on {b.device}.")


def _matmul_forward(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """matmul.py:229-237: ``(M, K) @ (K, N) -> (M, N)`` in a's dtype, any strides."""
    _check_pair(a, b, 2, "(M, K)")
    return torch.mm(a, b)


def _matmul_vec_forward(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """matmul.py:240-261: ``(K,) @ (K, N) -> (N,)``."""
    _check_pair(a, b, 1, "(K,)")
    return torch.mm(a.unsqueeze(0), b).squeeze(0)


class _MatMulAutograd(torch.autograd.Function):
    """matmul.py:311-333: dA = dC B^T, dB = A^T dC."""

    @staticmethod
    def forward(ctx: Any, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        ctx.save_for_backward(a, b)
        return _matmul_forward(a, b)

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        dc = grad_outputs[0]
        if not dc.is_contiguous():
            dc = dc.contiguous()
        a, b = ctx.saved_tensors
        da = torch.mm(dc, b.t()) if ctx.needs_input_grad[0] else None
        db = torch.mm(a.t(), dc) if ctx.needs_input_grad[1] else None
        return da, db


def matmul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Return the matrix product ``a @ b`` with autograd support (matmul.py:336-340)."""
    if not requires_autograd(a, b):
        return _matmul_forward(a, b)
    return _MatMulAutograd.apply(a, b)


def matmul_vec(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Return the vector-matrix product ``a @ b`` for ``a`` shaped ``(K,)`` (matmul.py:343-347)."""
    if requires_autograd(a, b):
        _check_pair(a, b, 1, "(K,)")
        return matmul(a.unsqueeze(0), b).squeeze(0)
    return _matmul_vec_forward(a, b)

"""``cross_entropy`` and ``cross_entropy_backward`` on materialised logits, on
gfx950 HIP kernels (``csrc/cross_entropy.hip``).

Drop-in for the logits op of alkinun/helion ``tritium/ops/cross_entropy.py``:
``cross_entropy(logits, target)`` returns the mean negative log-likelihood of
2-D logits (708-713), ``cross_entropy_backward(grad_out, logits, target,
logsumexp)`` returns ``dlogits`` (792-799), ``_CrossEntropyAutograd`` saves
the per-row logsumexp (643-660); validation as ``_check_cross_entropy_inputs``
(385-428) and ``_cross_entropy_backward_impl`` (728-789).  Like the reference
there is no ignore_index here (the fused ``linear_cross_entropy`` has one); a
target outside ``[0, vocab)`` makes the loss NaN instead of reading outside
the row.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib
from ._utils import (
    FLOAT_DTYPES,
    INDEX_DTYPES,
    check_contiguous,
    check_cuda_tensor,
    check_supported_dtype,
    next_power_of_2,
    requires_autograd,
)

__all__ = ["cross_entropy", "cross_entropy_backward"]

MAX_VOCAB_BLOCK_SIZE = 131072  # cross_entropy.py:21


def _target_kind(target: torch.Tensor) -> int:
    return 1 if target.dtype == torch.int32 else 2


def _check_inputs(logits: torch.Tensor, target: torch.Tensor) -> tuple[int, int]:
    """cross_entropy.py:385-428."""
    check_cuda_tensor("logits", logits)
    check_cuda_tensor("target", target)
    check_supported_dtype("logits", logits, FLOAT_DTYPES)
    check_supported_dtype("target", target, INDEX_DTYPES)
    if logits.dim() != 2:
        raise ValueError("logits must be a 2D tensor shaped (n_rows, vocab_size).")
    if target.dim() != 1:
        raise ValueError("target must be a 1D tensor.")
    n_rows, vocab_size = logits.shape
    if target.shape != (n_rows,):
        raise ValueError(
            f"Shape mismatch: target has shape {tuple(target.shape)}, expected ({n_rows},)."
        )
    if target.device != logits.device:
        raise ValueError(
            f"Device mismatch: target is on {target.device}, logits is on {logits.device}."
        )
    if vocab_size <= 0:
        raise ValueError("vocab_size must be positive.")
    block_size = next_power_of_2(vocab_size)
    if block_size > MAX_VOCAB_BLOCK_SIZE:
        raise ValueError(
            "Unsupported vocab size: "
            f"next_power_of_2({vocab_size}) is {block_size}, "
            f"which exceeds {MAX_VOCAB_BLOCK_SIZE}."
        )
    check_contiguous("logits", logits, "for tritium.cross_entropy")
    check_contiguous("target", target, "for tritium.cross_entropy")
    return n_rows, vocab_size


def _cross_entropy_forward(logits: torch.Tensor, target: torch.Tensor):
    """cross_entropy.py:534-561: (loss, logsumexp), loss fp32 0-dim, lse fp32 [n_rows]."""
    n_rows, vocab_size = _check_inputs(logits, target)
    dev = logits.device
    lse = torch.empty((n_rows,), device=dev, dtype=torch.float32)
    if n_rows == 0:
        return torch.zeros((), device=dev, dtype=torch.float32), lse
    loss = torch.empty((), device=dev, dtype=torch.float32)
    code = _lib.dtype_code(logits.dtype)
    ws_bytes = _lib.lib().tritium_cross_entropy_fwd_workspace_size(n_rows, vocab_size, code)
    work = torch.empty((max(1, -(-ws_bytes // 4)),), device=dev, dtype=torch.float32)
    _lib.call(
        "tritium_cross_entropy_fwd_ws", logits.data_ptr(), target.data_ptr(),
        _target_kind(target), loss.data_ptr(), lse.data_ptr(), work.data_ptr(),
        work.numel() * 4, n_rows, vocab_size, code, _lib.stream_of(logits),
    )
    return loss, lse


def _cross_entropy_backward(grad_out, logits, target, logsumexp, grad_denominator=None):
    """cross_entropy.py:728-789."""
    n_rows, vocab_size = _check_inputs(logits, target)
    grad_denominator = n_rows if grad_denominator is None else grad_denominator
    check_cuda_tensor("grad_out", grad_out)
    check_cuda_tensor("logsumexp", logsumexp)
    if grad_out.shape != ():
        raise ValueError(f"Shape mismatch: grad_out has shape {tuple(grad_out.shape)}, expected ().")
    if logsumexp.shape != (n_rows,):
        raise ValueError(
            f"Shape mismatch: logsumexp has shape {tuple(logsumexp.shape)}, expected ({n_rows},)."
        )
    if grad_out.device != logits.device:
        raise ValueError(
            f"Device mismatch: grad_out is on {grad_out.device}, logits is on {logits.device}."
        )
    if logsumexp.device != logits.device:
        raise ValueError(
            f"Device mismatch: logsumexp is on {logsumexp.device}, logits is on {logits.device}."
        )
    if logsumexp.dtype != torch.float32:
        raise ValueError(
            f"Dtype mismatch: logsumexp has dtype {logsumexp.dtype}, expected float32."
        )
    check_contiguous("logsumexp", logsumexp, "for tritium.cross_entropy")
    dlogits = torch.empty_like(logits)
    if logits.numel() == 0:
        return dlogits
    g = grad_out.detach().to(torch.float32).reshape(())
    _lib.call(
        "tritium_cross_entropy_bwd", g.data_ptr(), logits.data_ptr(), target.data_ptr(),
        _target_kind(target), logsumexp.data_ptr(), dlogits.data_ptr(), n_rows, vocab_size,
        float(grad_denominator), _lib.dtype_code(logits.dtype), _lib.stream_of(logits),
    )
    return dlogits


def cross_entropy_backward(grad_out: torch.Tensor, logits: torch.Tensor, target: torch.Tensor,
                           logsumexp: torch.Tensor) -> torch.Tensor:
    """Return ``dlogits`` from saved per-row logsumexp values (cross_entropy.py:792-799)."""
    return _cross_entropy_backward(grad_out, logits, target, logsumexp)


class _CrossEntropyAutograd(torch.autograd.Function):
    """cross_entropy.py:643-660."""

    @staticmethod
    def forward(ctx: Any, logits: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
        loss, lse = _cross_entropy_forward(logits, target)
        ctx.save_for_backward(logits, target, lse)
        return loss

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0]:
            return None, None
        logits, target, lse = ctx.saved_tensors
        return cross_entropy_backward(grad_outputs[0], logits, target, lse), None


def cross_entropy(logits: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """Return mean cross-entropy loss for 2D logits without materialised softmax
    (cross_entropy.py:708-713)."""
    if not requires_autograd(logits):
        loss, _ = _cross_entropy_forward(logits, target)
        return loss
    return _CrossEntropyAutograd.apply(logits, target)

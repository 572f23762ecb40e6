"""``linear_cross_entropy`` and ``linear_cross_entropy_backward`` on gfx950 HIP kernels.

Drop-in for alkinun/helion ``tritium/ops/cross_entropy.py``: same signatures
(``linear_cross_entropy`` 716-725, ``linear_cross_entropy_backward`` 863-959),
validation and messages (``_check_linear_cross_entropy_inputs`` 431-494,
backward checks 871-914), autograd (``_LinearCrossEntropyAutograd`` 663-705:
saves the 2-D hidden, weight, 1-D target and the fp32 logsumexp; the backward
honours ``needs_input_grad``).

Differences, each a correction the north star asks for:

* ``ignore_index`` (keyword, default -100, torch's value): rows whose target
  equals it add nothing to the loss or the gradients and the mean divides by
  the number of the other rows, as ``F.cross_entropy`` does.  The reference
  has no such argument and yields ``inf`` for a -100 target
  (cross_entropy.py:240-244); with no ignored target both agree;
* the logits are never written to memory in the forward (only the fp32
  logsumexp is kept for the backward); the 16-bit backward recomputes them
  per vocabulary chunk on the library's MFMA GEMM core, holds only that
  chunk's gradient of the logits (at most 1 GiB) and runs dH and dW on the
  same core; ``dweight`` is accumulated over all rows in fp32 before one
  rounding (the reference accumulates it in the weight dtype chunk by chunk,
  947-957);
* a target outside ``[0, vocab)`` that is not ``ignore_index`` gives a NaN
  loss instead of a device assert or ``inf``.
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
    requires_autograd,
)

SUPPORTED_LOGIT_DTYPES = FLOAT_DTYPES
SUPPORTED_TARGET_DTYPES = INDEX_DTYPES
IGNORE_INDEX = -100


def _check_linear_cross_entropy_inputs(hidden, weight, target) -> tuple[int, int, int]:
    """cross_entropy.py:431-494."""
    check_cuda_tensor("hidden", hidden)
    check_cuda_tensor("weight", weight)
    check_cuda_tensor("target", target)
    check_supported_dtype("hidden", hidden, SUPPORTED_LOGIT_DTYPES)
    check_supported_dtype("weight", weight, SUPPORTED_LOGIT_DTYPES)
    check_supported_dtype("target", target, SUPPORTED_TARGET_DTYPES)
    if hidden.dim() < 2:
        raise ValueError("hidden must have at least 2 dimensions shaped (..., hidden_size).")
    if weight.dim() != 2:
        raise ValueError("weight must be a 2D tensor shaped (vocab_size, hidden_size).")
    vocab_size, hidden_size = weight.shape
    if hidden.shape[-1] != hidden_size:
        raise ValueError(
            f"Shape mismatch: hidden has last dimension {hidden.shape[-1]}, "
            f"weight expects {hidden_size}."
        )
    if target.shape != hidden.shape[:-1]:
        raise ValueError(
            f"Shape mismatch: target has shape {tuple(target.shape)}, "
            f"expected {tuple(hidden.shape[:-1])}."
        )
    if weight.dtype != hidden.dtype:
        raise ValueError(
            f"Dtype mismatch: weight has dtype {weight.dtype}, hidden has dtype {hidden.dtype}."
        )
    if weight.device != hidden.device:
        raise ValueError(
            f"Device mismatch: weight is on {weight.device}, hidden is on {hidden.device}."
        )
    if target.device != hidden.device:
        raise ValueError(
            f"Device mismatch: target is on {target.device}, hidden is on {hidden.device}."
        )
    if hidden_size <= 0:
        raise ValueError("hidden_size must be positive.")
    if vocab_size <= 0:
        raise ValueError("vocab_size must be positive.")
    check_contiguous("hidden", hidden, "for tritium.linear_cross_entropy")
    check_contiguous("weight", weight, "for tritium.linear_cross_entropy")
    check_contiguous("target", target, "for tritium.linear_cross_entropy")
    return target.numel(), hidden_size, vocab_size


def _kernel_operand(t: torch.Tensor) -> torch.Tensor:
    """The kernels read 16-byte vectors along hidden_size: pad it with zeros to
    a multiple of 8 (zeros add nothing to any dot product) and realign."""
    d = t.shape[-1]
    dp = -(-d // 8) * 8
    if dp != d:
        out = torch.zeros((*t.shape[:-1], dp), device=t.device, dtype=t.dtype)
        out[..., :d] = t
        return out
    if t.data_ptr() % 16 != 0:
        return t.clone()
    return t


def _target_kind(target: torch.Tensor) -> int:
    return 1 if target.dtype == torch.int32 else 2


def _linear_cross_entropy_forward(hidden, weight, target, ignore_index: int = IGNORE_INDEX):
    """cross_entropy.py:563-640: returns ``(loss, logsumexp)``."""
    n_rows, hidden_size, vocab_size = _check_linear_cross_entropy_inputs(hidden, weight, target)
    dev = hidden.device
    loss = torch.zeros((), device=dev, dtype=torch.float32)
    lse = torch.empty((n_rows,), device=dev, dtype=torch.float32)
    if n_rows == 0:
        return loss, lse
    h2 = _kernel_operand(hidden.reshape(n_rows, hidden_size))
    w2 = _kernel_operand(weight)
    ws_bytes = _lib.lib().tritium_linear_ce_fwd_workspace_size(
        n_rows, vocab_size, _lib.dtype_code(hidden.dtype)
    )
    ws = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
    _lib.call(
        "tritium_linear_ce_fwd",
        h2.data_ptr(),
        w2.data_ptr(),
        target.data_ptr(),
        _target_kind(target),
        int(ignore_index),
        loss.data_ptr(),
        lse.data_ptr(),
        None,
        ws.data_ptr(),
        ws_bytes,
        n_rows,
        h2.shape[-1],
        vocab_size,
        _lib.dtype_code(hidden.dtype),
        _lib.stream_of(hidden),
    )
    return loss, lse


# fp32 gradient-of-logits tile per chunk (the fp32 correctness path)
_G_CHUNK_BYTES = 1 << 30


def _backward_f32(grad_out, h2, w2, target_1d, lse, need_dh, need_dw, ignore_index,
                  chunk_rows: int = 0):
    """fp32 inputs: per vocabulary chunk the HIP kernel recomputes the logits
    (exact fp32 FMAs) and writes only G = (softmax - onehot) * grad_out /
    n_valid (``tritium_linear_ce_grad_logits``); dH += G W_c and dW_c = G^T H
    are fp32 library GEMMs on views (cross_entropy.py:928-957 does the same
    chunking).  A correctness path: the MFMA contractions are 16-bit."""
    n_rows, dp = h2.shape
    vocab_size = w2.shape[0]
    dev = h2.device
    g = grad_out.detach().to(device=dev, dtype=torch.float32).reshape(())
    n_valid = (target_1d != ignore_index).sum(dtype=torch.float32)
    chunk = int(chunk_rows) if chunk_rows > 0 else max(256, (_G_CHUNK_BYTES // (4 * n_rows)) // 256 * 256)
    chunk = min(chunk, vocab_size)
    ld_g = -(-chunk // 8) * 8
    gbuf = torch.empty((n_rows, ld_g), device=dev, dtype=torch.float32)
    dh = torch.zeros((n_rows, dp), device=dev, dtype=torch.float32) if need_dh else None
    dw = torch.empty((vocab_size, dp), device=dev, dtype=torch.float32) if need_dw else None
    for v0 in range(0, vocab_size, chunk):
        vc = min(chunk, vocab_size - v0)
        _lib.call(
            "tritium_linear_ce_grad_logits", g.data_ptr(), n_valid.data_ptr(), h2.data_ptr(),
            w2.data_ptr(), target_1d.data_ptr(), _target_kind(target_1d), int(ignore_index),
            lse.data_ptr(), gbuf.data_ptr(), ld_g, n_rows, dp, vocab_size, v0, vc,
            _lib.dtype_code(torch.float32), _lib.stream_of(h2),
        )
        gc = gbuf[:, :vc]
        if need_dh:
            dh.addmm_(gc, w2[v0:v0 + vc])
        if need_dw:
            torch.mm(gc.t(), h2, out=dw[v0:v0 + vc])
    return dh, dw


def _backward(grad_out, hidden_2d, weight, target_1d, lse, need_dh, need_dw, ignore_index,
              chunk_rows: int = 0):
    """cross_entropy.py:863-959.  16-bit inputs: the whole backward runs in the
    library (``tritium_linear_ce_bwd``): per vocabulary chunk (its gradient of
    the logits at most 1 GiB) the logits are recomputed on the MFMA GEMM
    core and turned into G, then dW_c = G^T H and dH += G W_c run on the same
    core reading G, H and W in place.  fp32 inputs: :func:`_backward_f32`."""
    n_rows, hidden_size = hidden_2d.shape
    vocab_size = weight.shape[0]
    dev = hidden_2d.device
    h2 = _kernel_operand(hidden_2d)
    w2 = _kernel_operand(weight)
    dp = h2.shape[-1]
    if weight.dtype == torch.float32:
        dh, dw = _backward_f32(grad_out, h2, w2, target_1d, lse, need_dh, need_dw, ignore_index,
                               chunk_rows)
    else:
        dh = torch.empty((n_rows, dp), device=dev, dtype=hidden_2d.dtype) if need_dh else None
        dw = torch.empty((vocab_size, dp), device=dev, dtype=weight.dtype) if need_dw else None
        g = grad_out.detach().to(device=dev, dtype=torch.float32).reshape(())
        ws_bytes = _lib.lib().tritium_linear_ce_bwd_workspace_size(
            n_rows, dp, vocab_size, _lib.dtype_code(weight.dtype), int(need_dh), int(need_dw),
            int(chunk_rows),
        )
        ws = torch.empty((max(ws_bytes, 1),), device=dev, dtype=torch.uint8)
        _lib.call(
            "tritium_linear_ce_bwd", g.data_ptr(), h2.data_ptr(), w2.data_ptr(),
            target_1d.data_ptr(), _target_kind(target_1d), int(ignore_index), lse.data_ptr(),
            _lib.ptr(dh), _lib.ptr(dw), ws.data_ptr(), ws_bytes, n_rows, dp, vocab_size,
            int(chunk_rows), _lib.dtype_code(weight.dtype), _lib.stream_of(hidden_2d),
        )
    if dp != hidden_size:
        dh = dh[:, :hidden_size].contiguous() if dh is not None else None
        dw = dw[:, :hidden_size].contiguous() if dw is not None else None
    return dh, dw


def linear_cross_entropy_backward(
    grad_out: torch.Tensor,
    hidden: torch.Tensor,
    weight: torch.Tensor,
    target: torch.Tensor,
    logsumexp: torch.Tensor,
    *,
    ignore_index: int = IGNORE_INDEX,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``(dhidden, dweight)`` for ``linear_cross_entropy`` from the saved
    logsumexp (cross_entropy.py:863-959).  ``dhidden`` is 2-D ``[n_rows, hidden_size]``."""
    n_rows, hidden_size, vocab_size = _check_linear_cross_entropy_inputs(hidden, weight, target)
    check_cuda_tensor("grad_out", grad_out)
    check_cuda_tensor("logsumexp", logsumexp)
    if grad_out.shape != ():
        raise ValueError(
            f"Shape mismatch: grad_out has shape {tuple(grad_out.shape)}, expected ()."
        )
    if logsumexp.shape != (n_rows,):
        raise ValueError(
            f"Shape mismatch: logsumexp has shape {tuple(logsumexp.shape)}, "
            f"expected ({n_rows},)."
        )
    if grad_out.device != hidden.device:
        raise ValueError(
            f"Device mismatch: grad_out is on {grad_out.device}, hidden is on {hidden.device}."
        )
    if logsumexp.device != hidden.device:
        raise ValueError(
            f"Device mismatch: logsumexp is on {logsumexp.device}, hidden is on {hidden.device}."
        )
    if logsumexp.dtype != torch.float32:
        raise ValueError(
            f"Dtype mismatch: logsumexp has dtype {logsumexp.dtype}, expected float32."
        )
    check_contiguous("logsumexp", logsumexp, "for tritium.linear_cross_entropy")
    hidden_2d = hidden.view(n_rows, hidden_size)
    if n_rows == 0:
        return torch.empty_like(hidden_2d), torch.zeros_like(weight)
    return _backward(grad_out, hidden_2d, weight, target.view(n_rows), logsumexp, True, True,
                     ignore_index)


class _LinearCrossEntropyAutograd(torch.autograd.Function):
    """cross_entropy.py:663-705: saves the 2-D hidden, weight, 1-D target and
    the fp32 logsumexp, nothing of size n_rows x vocab."""

    @staticmethod
    def forward(ctx: Any, hidden, weight, target, ignore_index):
        n = target.numel()
        loss, lse = _linear_cross_entropy_forward(hidden, weight, target, ignore_index)
        ctx.hidden_shape = tuple(hidden.shape)
        ctx.ignore_index = ignore_index
        ctx.save_for_backward(hidden.view(n, hidden.shape[-1]), weight, target.view(n), lse)
        return loss

    @staticmethod
    def backward(ctx: Any, *grad_outputs):
        need_dh, need_dw = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        if not need_dh and not need_dw:
            return None, None, None, None
        hidden_2d, weight, target_1d, lse = ctx.saved_tensors
        if hidden_2d.shape[0] == 0:
            dh = torch.zeros(ctx.hidden_shape, device=hidden_2d.device, dtype=hidden_2d.dtype)
            return (dh if need_dh else None), (torch.zeros_like(weight) if need_dw else None), \
                None, None
        dh, dw = _backward(grad_outputs[0], hidden_2d, weight, target_1d, lse, need_dh, need_dw,
                           ctx.ignore_index)
        if dh is not None:
            dh = dh.view(ctx.hidden_shape)
        return dh, dw, None, None


def linear_cross_entropy(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    target: torch.Tensor,
    *,
    ignore_index: int = IGNORE_INDEX,
) -> torch.Tensor:
    """Mean cross-entropy of ``hidden @ weight.T`` against ``target`` without
    materialising the logits (cross_entropy.py:716-725).  Under autograd only
    the fp32 logsumexp is kept for the backward."""
    if not requires_autograd(hidden, weight):
        loss, _ = _linear_cross_entropy_forward(hidden, weight, target, ignore_index)
        return loss
    return _LinearCrossEntropyAutograd.apply(hidden, weight, target, ignore_index)

"""``swiglu`` and ``swiglu_backward`` on gfx950 HIP kernels.

Drop-in for alkinun/helion ``tritium/ops/swiglu.py``: ``swiglu(x, gate) =
silu(x) * gate`` (126-130), ``swiglu_backward(dy, x, gate) -> (dx, dgate)``
(76-100), ``_SwiGLUAutograd`` (103-123), same validation.
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib
from ._utils import check_same_shape_dtype_device, requires_autograd


def _swiglu_forward(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """swiglu.py:61-73."""
    check_same_shape_dtype_device("x", x, "gate", gate)
    x = x.contiguous()
    gate = gate.contiguous()
    out = torch.empty_like(x)
    if x.numel() == 0:
        return out
    _lib.call(
        "tritium_swiglu_fwd",
        x.data_ptr(),
        gate.data_ptr(),
        out.data_ptr(),
        x.numel(),
        _lib.dtype_code(x.dtype),
        _lib.stream_of(x),
    )
    return out


def swiglu_backward(
    dy: torch.Tensor, x: torch.Tensor, gate: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``(dx, dgate)`` for ``swiglu`` (``silu(x) * gate``) -- swiglu.py:76-100."""
    check_same_shape_dtype_device("x", x, "gate", gate)
    if dy.shape != x.shape:
        raise ValueError(
            f"Shape mismatch: dy has shape {tuple(dy.shape)}, x has shape {tuple(x.shape)}."
        )
    if dy.device != x.device:
        raise ValueError(f"Device mismatch: dy is on {dy.device}, x is on {x.device}.")
    x = x.contiguous()
    gate = gate.contiguous()
    # the reference kernel upcasts dy from any float dtype; one kernel dtype here
    dy = dy.to(x.dtype).contiguous()
    dx = torch.empty_like(x)
    dgate = torch.empty_like(gate)
    if x.numel() == 0:
        return dx, dgate
    _lib.call(
        "tritium_swiglu_bwd",
        dy.data_ptr(),
        x.data_ptr(),
        gate.data_ptr(),
        dx.data_ptr(),
        dgate.data_ptr(),
        x.numel(),
        _lib.dtype_code(x.dtype),
        _lib.stream_of(x),
    )
    return dx, dgate


class _SwiGLUAutograd(torch.autograd.Function):
    """swiglu.py:103-123."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        out = _swiglu_forward(x, gate)
        ctx.save_for_backward(x, gate)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0] and not ctx.needs_input_grad[1]:
            return None, None
        x, gate = ctx.saved_tensors
        dx, dgate = swiglu_backward(grad_outputs[0], x, gate)
        return (dx if ctx.needs_input_grad[0] else None), (
            dgate if ctx.needs_input_grad[1] else None
        )


def swiglu(x: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
    """Return ``silu(x) * gate`` with autograd support (swiglu.py:126-130)."""
    if not requires_autograd(x, gate):
        return _swiglu_forward(x, gate)
    return _SwiGLUAutograd.apply(x, gate)


def _check_rows(ts, name):
    ref = ts[0]
    for t in ts:
        if t.dim() != 2 or t.shape != ref.shape or t.dtype != ref.dtype or t.device != ref.device:
            raise ValueError(f"{name}: operands must be 2-D views of one shape, dtype and device")
        if t.stride(1) != 1:
            raise ValueError(f"{name}: rows must have unit column stride")


def swiglu_rows(x: torch.Tensor, gate: torch.Tensor, out: torch.Tensor) -> None:
    """``out = silu(x) * gate`` on 2-D row-strided views (``x`` and ``gate``
    sharing one row stride), e.g. the two halves of each row of a fused
    gate/up projection (``tritium_swiglu_rows_fwd``).  Not part of the
    reference's surface, whose swiglu takes separate tensors; the training
    harness's fused MLP uses it."""
    _check_rows((x, gate, out), "swiglu_rows")
    if x.stride(0) != gate.stride(0):
        raise ValueError("swiglu_rows: x and gate must share a row stride")
    _lib.call("tritium_swiglu_rows_fwd", x.data_ptr(), gate.data_ptr(), out.data_ptr(),
              x.shape[0], x.shape[1], x.stride(0), out.stride(0), _lib.dtype_code(x.dtype),
              _lib.stream_of(x))


def swiglu_rows_backward(dy, x, gate, dx, dgate) -> None:
    """Gradients of ``swiglu_rows`` into row-strided ``dx`` and ``dgate`` (which
    share a row stride, as ``x`` and ``gate`` do) -- ``tritium_swiglu_rows_bwd``."""
    _check_rows((dy, x, gate, dx, dgate), "swiglu_rows_backward")
    if x.stride(0) != gate.stride(0) or dx.stride(0) != dgate.stride(0):
        raise ValueError("swiglu_rows_backward: paired operands must share a row stride")
    _lib.call("tritium_swiglu_rows_bwd", dy.data_ptr(), x.data_ptr(), gate.data_ptr(),
              dx.data_ptr(), dgate.data_ptr(), x.shape[0], x.shape[1], dy.stride(0),
              x.stride(0), dx.stride(0), _lib.dtype_code(x.dtype), _lib.stream_of(x))

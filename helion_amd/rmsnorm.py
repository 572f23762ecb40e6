"""``rmsnorm``, ``rmsnorm_backward`` and ``residual_rmsnorm`` on gfx950 HIP kernels.

Drop-in for alkinun/helion ``tritium/ops/rmsnorm.py``: same signatures
(``rmsnorm`` 737-746, ``rmsnorm_backward`` 577-613, ``residual_rmsnorm``
749-778), same validation and messages (283-317), same autograd behaviour
(``_RMSNormAutograd`` 616-651, ``_ResidualRMSNormAutograd`` 654-734).

Differences, all numerically within the reference's own tolerances:

* dweight is reduced deterministically (fixed-order partial rows), never with
  atomics (the reference uses fp32 atomics for small row counts, 160, 192);
* the residual backward adds ``dresidual_out`` inside the dx kernel in fp32
  and rounds once, instead of rounding dx and then ``dz.add_`` (729-730).
"""

from __future__ import annotations

from typing import Any

import torch

from . import _lib
from ._utils import (
    FLOAT_DTYPES,
    check_contiguous,
    check_cuda_tensor,
    check_supported_dtype,
    next_power_of_2,
    requires_autograd,
)

SUPPORTED_DTYPES = FLOAT_DTYPES
MAX_RMSNORM_HIDDEN_NEXT_POW2 = 65536


def _check_rmsnorm_inputs(x: torch.Tensor, weight: torch.Tensor) -> int:
    """rmsnorm.py:283-317."""
    check_cuda_tensor("x", x)
    check_cuda_tensor("weight", weight)
    check_supported_dtype("x", x, SUPPORTED_DTYPES)
    check_supported_dtype("weight", weight, SUPPORTED_DTYPES)
    if x.dim() < 1:
        raise ValueError("x must have at least 1 dimension.")
    hidden = x.shape[-1]
    if weight.shape != (hidden,):
        raise ValueError(
            f"Shape mismatch: weight has shape {tuple(weight.shape)}, expected ({hidden},)."
        )
    if weight.dtype != x.dtype:
        raise ValueError(
            f"Dtype mismatch: weight has dtype {weight.dtype}, x has dtype {x.dtype}."
        )
    if weight.device != x.device:
        raise ValueError(f"Device mismatch: weight is on {weight.device}, x is on {x.device}.")
    if next_power_of_2(hidden) > MAX_RMSNORM_HIDDEN_NEXT_POW2:
        raise ValueError(
            "Unsupported hidden size: "
            f"next_power_of_2({hidden}) exceeds {MAX_RMSNORM_HIDDEN_NEXT_POW2}."
        )
    check_contiguous("x", x, "for tritium.rmsnorm")
    check_contiguous("weight", weight, "for tritium.rmsnorm")
    return hidden


def _flat_2d(x: torch.Tensor) -> tuple[torch.Tensor, int, int]:
    hidden = x.shape[-1]
    n_rows = x.numel() // hidden if hidden else 0
    return x.view(n_rows, hidden), n_rows, hidden


def _forward_kernel(
    x2d: torch.Tensor,
    residual2d: torch.Tensor | None,
    weight: torch.Tensor,
    eps: float,
) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor]:
    n_rows, hidden = x2d.shape
    out = torch.empty_like(x2d)
    residual_out = torch.empty_like(x2d) if residual2d is not None else None
    rstd = torch.empty((n_rows,), device=x2d.device, dtype=torch.float32)
    if n_rows == 0 or hidden == 0:
        return out, residual_out, rstd
    _lib.call(
        "tritium_rmsnorm_fwd",
        x2d.data_ptr(),
        _lib.ptr(residual2d),
        weight.data_ptr(),
        out.data_ptr(),
        _lib.ptr(residual_out),
        rstd.data_ptr(),
        n_rows,
        hidden,
        float(eps),
        _lib.dtype_code(x2d.dtype),
        _lib.stream_of(x2d),
    )
    return out, residual_out, rstd


def _backward_kernel(
    dy2d: torch.Tensor,
    x2d: torch.Tensor,
    weight: torch.Tensor,
    rstd: torch.Tensor | None,
    eps: float,
    *,
    compute_dweight: bool,
    dresidual2d: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor | None]:
    """dx (+ dresidual) and optionally dweight -- rmsnorm.py:383-574."""
    n_rows, hidden = x2d.shape
    dx = torch.empty_like(x2d)
    if n_rows == 0 or hidden == 0:
        if dresidual2d is not None:
            dx.copy_(dresidual2d)
        dw = torch.zeros((hidden,), device=x2d.device, dtype=weight.dtype)
        return dx, (dw if compute_dweight else None)
    dweight = torch.empty((hidden,), device=x2d.device, dtype=weight.dtype) if compute_dweight else None
    ws_bytes = _lib.lib().tritium_rmsnorm_bwd_workspace_size(n_rows, hidden) if compute_dweight else 0
    workspace = torch.empty((max(ws_bytes, 1),), device=x2d.device, dtype=torch.uint8)
    _lib.call(
        "tritium_rmsnorm_bwd",
        dy2d.data_ptr(),
        x2d.data_ptr(),
        weight.data_ptr(),
        _lib.ptr(rstd),
        _lib.ptr(dresidual2d),
        dx.data_ptr(),
        _lib.ptr(dweight),
        workspace.data_ptr(),
        ws_bytes,
        n_rows,
        hidden,
        float(eps),
        _lib.dtype_code(x2d.dtype),
        _lib.stream_of(x2d),
    )
    return dx, dweight


def _rmsnorm_forward(
    x: torch.Tensor, weight: torch.Tensor, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    """rmsnorm.py:325-349."""
    _check_rmsnorm_inputs(x, weight)
    x2d, _, _ = _flat_2d(x)
    out, _, rstd = _forward_kernel(x2d, None, weight, eps)
    return out.view_as(x), rstd


def rmsnorm_backward(
    dy: torch.Tensor,
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``(dx, dweight)`` for ``rmsnorm`` recomputing rstd from ``x``.

    rmsnorm.py:577-613.
    """
    _check_rmsnorm_inputs(x, weight)
    check_cuda_tensor("dy", dy)
    if dy.shape != x.shape:
        raise ValueError(
            f"Shape mismatch: dy has shape {tuple(dy.shape)}, x has shape {tuple(x.shape)}."
        )
    if dy.dtype != x.dtype:
        raise ValueError(f"Dtype mismatch: dy has dtype {dy.dtype}, x has dtype {x.dtype}.")
    if dy.device != x.device:
        raise ValueError(f"Device mismatch: dy is on {dy.device}, x is on {x.device}.")
    check_contiguous("dy", dy, "for tritium.rmsnorm_backward")
    x2d, n_rows, hidden = _flat_2d(x)
    dx, dweight = _backward_kernel(
        dy.view(n_rows, hidden), x2d, weight, None, eps, compute_dweight=True
    )
    return dx.view_as(x), dweight


class _RMSNormAutograd(torch.autograd.Function):
    """rmsnorm.py:616-651."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
        out, rstd = _rmsnorm_forward(x, weight, eps)
        ctx.save_for_backward(x, weight, rstd)
        ctx.eps = eps
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0] and not ctx.needs_input_grad[1]:
            return None, None, None
        x, weight, rstd = ctx.saved_tensors
        dy = grad_outputs[0]
        if not dy.is_contiguous():
            dy = dy.contiguous()
        x2d, n_rows, hidden = _flat_2d(x)
        dx, dweight = _backward_kernel(
            dy.view(n_rows, hidden),
            x2d,
            weight,
            rstd,
            ctx.eps,
            compute_dweight=ctx.needs_input_grad[1],
        )
        dx = dx.view_as(x) if ctx.needs_input_grad[0] else None
        return dx, dweight, None


def _check_residual(x: torch.Tensor, residual: torch.Tensor) -> None:
    """rmsnorm.py:664-675."""
    check_cuda_tensor("residual", residual)
    if residual.shape != x.shape:
        raise ValueError(
            f"Shape mismatch: residual has shape {tuple(residual.shape)}, "
            f"x has shape {tuple(x.shape)}."
        )
    if residual.dtype != x.dtype:
        raise ValueError(
            f"Dtype mismatch: residual has dtype {residual.dtype}, x has dtype {x.dtype}."
        )
    check_contiguous("residual", residual, "for tritium.residual_rmsnorm")


def _residual_forward(x, residual, weight, eps):
    _check_rmsnorm_inputs(x, weight)
    _check_residual(x, residual)
    x2d, n_rows, hidden = _flat_2d(x)
    out, residual_out, rstd = _forward_kernel(x2d, residual.view(n_rows, hidden), weight, eps)
    return out.view_as(x), residual_out.view_as(x), rstd


class _ResidualRMSNormAutograd(torch.autograd.Function):
    """rmsnorm.py:654-734."""

    @staticmethod
    def forward(ctx: Any, x, residual, weight, eps):
        out, residual_out, rstd = _residual_forward(x, residual, weight, eps)
        ctx.save_for_backward(residual_out, weight, rstd)
        ctx.eps = eps
        return out, residual_out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        needs = ctx.needs_input_grad
        if not needs[0] and not needs[1] and not needs[2]:
            return None, None, None, None
        residual_out, weight, rstd = ctx.saved_tensors
        dy, dresidual_out = grad_outputs[0], grad_outputs[1]
        if not dy.is_contiguous():
            dy = dy.contiguous()
        if not dresidual_out.is_contiguous():
            dresidual_out = dresidual_out.contiguous()
        z2d, n_rows, hidden = _flat_2d(residual_out)
        dz, dweight = _backward_kernel(
            dy.view(n_rows, hidden),
            z2d,
            weight,
            rstd,
            ctx.eps,
            compute_dweight=needs[2],
            dresidual2d=dresidual_out.view(n_rows, hidden),
        )
        dz = dz.view_as(residual_out)
        return (dz if needs[0] else None), (dz if needs[1] else None), dweight, None


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6) -> torch.Tensor:
    """Return ``x * rsqrt(mean(x**2) + eps) * weight`` with autograd support.

    rmsnorm.py:737-746.
    """
    if not requires_autograd(x, weight):
        out, _ = _rmsnorm_forward(x, weight, eps)
        return out
    return _RMSNormAutograd.apply(x, weight, eps)


def residual_rmsnorm(
    x: torch.Tensor,
    residual: torch.Tensor,
    weight: torch.Tensor,
    eps: float = 1e-6,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Return ``(rmsnorm(x + residual), x + residual)`` with autograd support.

    rmsnorm.py:749-778.
    """
    if not requires_autograd(x, residual, weight):
        out, residual_out, _ = _residual_forward(x, residual, weight, eps)
        return out, residual_out
    return _ResidualRMSNormAutograd.apply(x, residual, weight, eps)

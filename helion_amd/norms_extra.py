"""The reference's row ops that sit off the hot path: ``softmax``/
``softmax_backward`` and ``layernorm``/``layernorm_backward``.

Same names, signatures, validation messages and autograd contracts as
``tritium/ops/softmax.py`` and ``tritium/ops/layernorm.py``, kept for the
drop-in surface (``tritium/__init__.py:40-70``).  The config-5 model uses
neither (RMSNorm, fused linear-cross-entropy), so they run as PyTorch GPU
operations in fp32 with one rounding to the input dtype, as the reference
kernels compute; like the reference they reject CPU tensors.
"""

from __future__ import annotations

from typing import Any

import torch

from ._utils import (
    FLOAT_DTYPES,
    check_contiguous,
    check_cuda_tensor,
    check_supported_dtype,
    next_power_of_2,
    requires_autograd,
)

__all__ = ["layernorm", "layernorm_backward", "softmax", "softmax_backward"]

MAX_HIDDEN_NEXT_POW2 = 65536  # softmax.py:17, layernorm.py:19


def _check_row_input(x: torch.Tensor, op: str) -> int:
    """softmax.py:68-81 / layernorm.py:275-288."""
    check_cuda_tensor("x", x)
    check_supported_dtype("x", x, FLOAT_DTYPES)
    if x.dim() < 1:
        raise ValueError("x must have at least 1 dimension.")
    hidden_size = x.shape[-1]
    if next_power_of_2(hidden_size) > MAX_HIDDEN_NEXT_POW2:
        raise ValueError(
            "Unsupported hidden size: "
            f"next_power_of_2({hidden_size}) exceeds {MAX_HIDDEN_NEXT_POW2}."
        )
    check_contiguous("x", x, f"for tritium.{op}")
    return hidden_size


def _check_dy(dy: torch.Tensor, ref: torch.Tensor, ref_name: str, op: str) -> None:
    check_cuda_tensor("dy", dy)
    check_supported_dtype("dy", dy, FLOAT_DTYPES)
    if dy.shape != ref.shape:
        raise ValueError(
            f"Shape mismatch: dy has shape {tuple(dy.shape)}, "
            f"{ref_name} has shape {tuple(ref.shape)}."
        )
    if dy.dtype != ref.dtype:
        raise ValueError(
            f"Dtype mismatch: dy has dtype {dy.dtype}, {ref_name} has dtype {ref.dtype}."
        )
    if dy.device != ref.device:
        raise ValueError(f"Device mismatch: dy is on {dy.device}, {ref_name} is on {ref.device}.")
    check_contiguous("dy", dy, f"for tritium.{op}")


# ------------------------------------------------------------------- softmax
def _softmax_forward(x: torch.Tensor) -> torch.Tensor:
    """softmax.py:20-45, 89-99: exp(x - rowmax) / sum in fp32, stored in x's dtype."""
    _check_row_input(x, "softmax")
    if x.numel() == 0:
        return torch.empty_like(x)
    return torch.softmax(x.float(), dim=-1).to(x.dtype)


def softmax_backward(dy: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """Return ``dx = out * (dy - sum(dy * out))`` over the last dimension, in fp32
    (softmax.py:47-58, host 102-139)."""
    _check_row_input(out, "softmax")
    _check_dy(dy, out, "out", "softmax_backward")
    if out.numel() == 0:
        return torch.empty_like(out)
    o32, g32 = out.float(), dy.float()
    c = (g32 * o32).sum(dim=-1, keepdim=True)
    return (o32 * (g32 - c)).to(out.dtype)


class _SoftmaxAutograd(torch.autograd.Function):
    """softmax.py:142-158: saves the output."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor) -> torch.Tensor:
        out = _softmax_forward(x)
        ctx.save_for_backward(out)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0]:
            return (None,)
        (out,) = ctx.saved_tensors
        dy = grad_outputs[0]
        if not dy.is_contiguous():
            dy = dy.contiguous()
        return (softmax_backward(dy, out),)


def softmax(x: torch.Tensor) -> torch.Tensor:
    """Return the numerically stable softmax of ``x`` over the last dimension
    (softmax.py:161-167), reduced in fp32, with autograd support."""
    if not requires_autograd(x):
        return _softmax_forward(x)
    return _SoftmaxAutograd.apply(x)


# ----------------------------------------------------------------- layernorm
def _check_affine(name: str, param: torch.Tensor, hidden_size: int, x: torch.Tensor) -> None:
    """layernorm.py:291-312."""
    check_cuda_tensor(name, param)
    check_supported_dtype(name, param, FLOAT_DTYPES)
    if param.shape != (hidden_size,):
        raise ValueError(
            f"Shape mismatch: {name} has shape {tuple(param.shape)}, expected ({hidden_size},)."
        )
    if param.dtype != x.dtype:
        raise ValueError(f"Dtype mismatch: {name} has dtype {param.dtype}, x has dtype {x.dtype}.")
    if param.device != x.device:
        raise ValueError(f"Device mismatch: {name} is on {param.device}, x is on {x.device}.")
    check_contiguous(name, param, "for tritium.layernorm")


def _stats(x2d: torch.Tensor, eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """layernorm.py:46-50: fp32 mean, population variance, rstd = 1/sqrt(var + eps)."""
    x32 = x2d.float()
    mean = x32.mean(dim=-1)
    xc = x32 - mean[:, None]
    var = (xc * xc).mean(dim=-1)
    return mean, torch.rsqrt(var + eps)


def _layernorm_forward(x, weight, bias, eps):
    """layernorm.py:331-359: out = x_hat * w + b in fp32, stored in x's dtype;
    mean and rstd saved in fp32."""
    hidden = _check_row_input(x, "layernorm")
    _check_affine("weight", weight, hidden, x)
    _check_affine("bias", bias, hidden, x)
    x2d = x.view(-1, hidden) if hidden > 0 else x.reshape(0, 0)
    if x2d.shape[0] == 0:
        empty = torch.empty((0,), device=x.device, dtype=torch.float32)
        return torch.empty_like(x), empty, empty.clone()
    mean, rstd = _stats(x2d, eps)
    x_hat = (x2d.float() - mean[:, None]) * rstd[:, None]
    out = x_hat * weight.float() + bias.float()
    return out.to(x.dtype).view_as(x), mean, rstd


def _layernorm_grads(dy2d, x2d, weight, mean, rstd, need_dx: bool, need_affine: bool):
    """layernorm.py:62-124, 198-272: dx = rstd (g - mean(g) - x_hat mean(g x_hat)),
    g = dy w; dweight = sum_rows dy x_hat, dbias = sum_rows dy (fp32, cast to
    weight's dtype)."""
    dy32 = dy2d.float()
    x_hat = (x2d.float() - mean[:, None]) * rstd[:, None]
    dx = dweight = dbias = None
    if need_dx:
        g = dy32 * weight.float()
        c1 = g.mean(dim=-1, keepdim=True)
        c2 = (g * x_hat).mean(dim=-1, keepdim=True)
        dx = (rstd[:, None] * (g - c1 - x_hat * c2)).to(x2d.dtype)
    if need_affine:
        dweight = (dy32 * x_hat).sum(dim=0).to(weight.dtype)
        dbias = dy32.sum(dim=0).to(weight.dtype)
    return dx, dweight, dbias


def layernorm_backward(dy: torch.Tensor, x: torch.Tensor, weight: torch.Tensor,
                       eps: float = 1e-5) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Return ``(dx, dweight, dbias)`` for ``layernorm``, recomputing ``mean``
    and ``rstd`` from ``x`` (layernorm.py:563-599)."""
    hidden = _check_row_input(x, "layernorm")
    _check_affine("weight", weight, hidden, x)
    _check_dy(dy, x, "x", "layernorm_backward")
    n_rows = x.numel() // hidden if hidden > 0 else 0
    if n_rows == 0:
        zeros = torch.zeros((hidden,), device=x.device, dtype=weight.dtype)
        return torch.empty_like(x), zeros, zeros.clone()
    x2d, dy2d = x.view(n_rows, hidden), dy.view(n_rows, hidden)
    mean, rstd = _stats(x2d, eps)
    dx, dweight, dbias = _layernorm_grads(dy2d, x2d, weight, mean, rstd, True, True)
    return dx.view_as(x), dweight, dbias


class _LayerNormAutograd(torch.autograd.Function):
    """layernorm.py:603-647: saves x, weight, mean, rstd; honours needs_input_grad."""

    @staticmethod
    def forward(ctx: Any, x, weight, bias, eps):
        out, mean, rstd = _layernorm_forward(x, weight, bias, eps)
        ctx.save_for_backward(x, weight, mean, rstd)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        need = ctx.needs_input_grad
        if not (need[0] or need[1] or need[2]):
            return None, None, None, None
        x, weight, mean, rstd = ctx.saved_tensors
        dy = grad_outputs[0]
        if not dy.is_contiguous():
            dy = dy.contiguous()
        hidden = x.shape[-1]
        n_rows = x.numel() // hidden if hidden > 0 else 0
        if n_rows == 0:
            zeros = torch.zeros((hidden,), device=x.device, dtype=weight.dtype)
            return (torch.empty_like(x) if need[0] else None, zeros if need[1] else None,
                    zeros.clone() if need[2] else None, None)
        dx, dweight, dbias = _layernorm_grads(
            dy.view(n_rows, hidden), x.view(n_rows, hidden), weight, mean, rstd,
            bool(need[0]), bool(need[1] or need[2]))
        return (dx.view_as(x) if need[0] else None, dweight if need[1] else None,
                dbias if need[2] else None, None)


def layernorm(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor,
              eps: float = 1e-5) -> torch.Tensor:
    """Return ``((x - mean) * rsqrt(var + eps)) * weight + bias`` over the last
    dimension (population variance), with autograd (layernorm.py:650-665)."""
    if not requires_autograd(x, weight, bias):
        out, _, _ = _layernorm_forward(x, weight, bias, eps)
        return out
    return _LayerNormAutograd.apply(x, weight, bias, eps)

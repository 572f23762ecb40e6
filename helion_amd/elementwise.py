"""The reference's elementwise ops that sit off the hot path: ``add``, ``relu``,
``add_relu``, ``gelu``/``gelu_backward``/``add_gelu``, ``dropout``/
``dropout_backward`` and ``sgd_step``.

They keep the drop-in surface whole (``tritium/__init__.py:40-70``): same names,
signatures, validation messages and autograd contracts as
``tritium/ops/{add,relu,add_relu,gelu,dropout,sgd}.py``.  The config-5 model
uses none of them (SwiGLU MLP, dropout p = 0), so they run as PyTorch GPU
operations rather than HIP kernels of this library; like the reference they
reject CPU tensors.  Arithmetic follows the reference kernels: inputs widened
to fp32, one rounding to the output dtype.
"""

from __future__ import annotations

from typing import Any

import torch

from ._utils import (
    FLOAT_DTYPES,
    check_contiguous,
    check_cuda_tensor,
    check_same_shape_dtype_device,
    check_supported_dtype,
    requires_autograd,
)

__all__ = [
    "add",
    "add_gelu",
    "add_relu",
    "dropout",
    "dropout_backward",
    "gelu",
    "gelu_backward",
    "relu",
    "sgd_step",
]

# tanh-approximation GELU: sqrt(2/pi) and the cubic coefficient of
# Hendrycks & Gimpel (2016), as gelu.py:33-34 uses them
_GELU_K0 = 0.7978845608028654
_GELU_K1 = 0.044715


def _contiguous_grad(grad: torch.Tensor) -> torch.Tensor:
    return grad if grad.is_contiguous() else grad.contiguous()


# ----------------------------------------------------------------------- add
def _add_forward(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """add.py:37-50: fp32 sum stored in x's dtype."""
    check_same_shape_dtype_device("x", x, "y", y)
    return torch.add(x, y)


class _AddAutograd(torch.autograd.Function):
    """add.py:53-68: the gradient passes through to both inputs."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        return _add_forward(x, y)

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        grad = _contiguous_grad(grad_outputs[0])
        return (grad if ctx.needs_input_grad[0] else None,
                grad if ctx.needs_input_grad[1] else None)


def add(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Return the elementwise sum ``x + y`` with autograd support (add.py:71-76)."""
    if not requires_autograd(x, y):
        return _add_forward(x, y)
    return _AddAutograd.apply(x, y)


# ---------------------------------------------------------------------- relu
def _check_unary(x: torch.Tensor) -> None:
    check_cuda_tensor("x", x)
    check_supported_dtype("x", x, FLOAT_DTYPES)


def _check_dy_like_x(dy: torch.Tensor, x: torch.Tensor) -> None:
    check_cuda_tensor("dy", dy)
    if dy.shape != x.shape:
        raise ValueError(
            f"Shape mismatch: dy has shape {tuple(dy.shape)}, x has shape {tuple(x.shape)}."
        )


def _relu_forward(x: torch.Tensor) -> torch.Tensor:
    """relu.py:57-67: ``where(x > 0, x, 0)`` (NaN maps to 0)."""
    _check_unary(x)
    return torch.where(x > 0, x, torch.zeros((), dtype=x.dtype, device=x.device))


def _relu_backward(dy: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """relu.py:70-84: ``where(x > 0, dy, 0)`` in x's dtype."""
    _check_unary(x)
    _check_dy_like_x(dy, x)
    return torch.where(x > 0, dy, torch.zeros((), dtype=dy.dtype, device=dy.device)).to(x.dtype)


class _ReLUAutograd(torch.autograd.Function):
    """relu.py:87-107."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor) -> torch.Tensor:
        out = _relu_forward(x)
        ctx.save_for_backward(x)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0]:
            return (None,)
        (x,) = ctx.saved_tensors
        return (_relu_backward(_contiguous_grad(grad_outputs[0]), x),)


def relu(x: torch.Tensor) -> torch.Tensor:
    """Return the elementwise ReLU of ``x`` with autograd support (relu.py:110-116)."""
    if not requires_autograd(x):
        return _relu_forward(x)
    return _ReLUAutograd.apply(x)


# ------------------------------------------------------------------ add_relu
def _add_relu_forward(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """add_relu.py:21-36, 58-68: ``z = x + y`` in fp32, ``where(z > 0, z, 0)``."""
    check_same_shape_dtype_device("x", x, "y", y)
    z = x.float() + y.float()
    return torch.where(z > 0, z, torch.zeros((), device=z.device)).to(x.dtype)


class _AddReLUAutograd(torch.autograd.Function):
    """add_relu.py:71-112: the mask is ``x + y > 0`` with the sum rounded to the
    inputs' dtype (the reference forms it with a dtype-preserving ``x + y``)."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        out = _add_relu_forward(x, y)
        ctx.save_for_backward(x, y)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0] and not ctx.needs_input_grad[1]:
            return None, None
        x, y = ctx.saved_tensors
        dy = _contiguous_grad(grad_outputs[0])
        grad = torch.where(x + y > 0, dy, torch.zeros((), dtype=dy.dtype, device=dy.device))
        dx = grad.to(x.dtype) if ctx.needs_input_grad[0] else None
        dy_out = grad.to(y.dtype) if ctx.needs_input_grad[1] else None
        return dx, dy_out


def add_relu(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Return ``relu(x + y)`` with autograd support (add_relu.py:115-119)."""
    if not requires_autograd(x, y):
        return _add_relu_forward(x, y)
    return _AddReLUAutograd.apply(x, y)


# ---------------------------------------------------------------------- gelu
def _gelu_f32(z: torch.Tensor) -> torch.Tensor:
    """gelu.py:33-35: 0.5 z (1 + tanh(u)), tanh(u) written as 2 sigmoid(2u) - 1."""
    inner = _GELU_K0 * (z + _GELU_K1 * z * z * z)
    return 0.5 * z * (1.0 + (2.0 * torch.sigmoid(2.0 * inner) - 1.0))


def _dgelu_f32(z: torch.Tensor) -> torch.Tensor:
    """gelu.py:50-55: d/dz of the tanh-approximation GELU."""
    z2 = z * z
    inner = _GELU_K0 * (z + _GELU_K1 * z * z2)
    t = 2.0 * torch.sigmoid(2.0 * inner) - 1.0
    d_inner = _GELU_K0 * (1.0 + 3.0 * _GELU_K1 * z2)
    return 0.5 * (1.0 + t) + 0.5 * z * (1.0 - t * t) * d_inner


def _gelu_forward(x: torch.Tensor) -> torch.Tensor:
    """gelu.py:112-122."""
    _check_unary(x)
    return _gelu_f32(x.float()).to(x.dtype)


def gelu_backward(dy: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """Return ``dx`` for the tanh-approximation GeLU from ``x`` (gelu.py:125-143)."""
    _check_unary(x)
    _check_dy_like_x(dy, x)
    return (dy.float() * _dgelu_f32(x.float())).to(x.dtype)


def _add_gelu_forward(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """gelu.py:146-159: gelu of the fp32 sum."""
    check_same_shape_dtype_device("x", x, "y", y)
    return _gelu_f32(x.float() + y.float()).to(x.dtype)


class _GeLUAutograd(torch.autograd.Function):
    """gelu.py:179-192."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor) -> torch.Tensor:
        out = _gelu_forward(x)
        ctx.save_for_backward(x)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0]:
            return (None,)
        (x,) = ctx.saved_tensors
        return (gelu_backward(grad_outputs[0], x),)


class _AddGeLUAutograd(torch.autograd.Function):
    """gelu.py:195-220: both inputs receive ``dy * gelu'(x + y)`` (fp32 sum)."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
        out = _add_gelu_forward(x, y)
        ctx.save_for_backward(x, y)
        return out

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0] and not ctx.needs_input_grad[1]:
            return None, None
        x, y = ctx.saved_tensors
        dy = _contiguous_grad(grad_outputs[0])
        grad = dy.float() * _dgelu_f32(x.float() + y.float())
        dx = grad.to(x.dtype) if ctx.needs_input_grad[0] else None
        dy_out = grad.to(y.dtype) if ctx.needs_input_grad[1] else None
        return dx, dy_out


def gelu(x: torch.Tensor) -> torch.Tensor:
    """Return the tanh-approximation GeLU of ``x`` with autograd support (gelu.py:223-227)."""
    if not requires_autograd(x):
        return _gelu_forward(x)
    return _GeLUAutograd.apply(x)


def add_gelu(x: torch.Tensor, y: torch.Tensor) -> torch.Tensor:
    """Return ``gelu(x + y)`` with autograd support (gelu.py:230-234)."""
    if not requires_autograd(x, y):
        return _add_gelu_forward(x, y)
    return _AddGeLUAutograd.apply(x, y)


# ------------------------------------------------------------------- dropout
def _check_dropout(name: str, t: torch.Tensor, p: float) -> None:
    """dropout.py:60-68."""
    check_cuda_tensor(name, t)
    check_supported_dtype(name, t, FLOAT_DTYPES)
    if not 0.0 <= p < 1.0:
        raise ValueError(f"Dropout probability p must satisfy 0 <= p < 1, got {p}.")


def _keep_mask(shape: torch.Size, p: float, seed: int, device: torch.device) -> torch.Tensor:
    """Keep element i when u_i >= p, u = uniform [0, 1) from a generator seeded with
    ``seed`` over the flat index order; the same seed gives the same mask, so the
    backward recomputes it instead of storing it (dropout.py:35-37, 55-57; the
    reference draws u from Triton's Philox stream, this from torch's device
    generator -- same distribution and contract, different bits)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(int(seed))
    return torch.rand(shape, generator=gen, device=device, dtype=torch.float32) >= p


def _dropout_apply(t: torch.Tensor, p: float, seed: int) -> torch.Tensor:
    t = t.contiguous()
    if t.numel() == 0:
        return torch.empty_like(t)
    keep = _keep_mask(t.shape, p, seed, t.device)
    scale = 1.0 / (1.0 - p)
    return torch.where(keep, t.float() * scale, torch.zeros((), device=t.device)).to(t.dtype)


def _dropout_forward(x: torch.Tensor, p: float, seed: int) -> torch.Tensor:
    """dropout.py:71-87."""
    _check_dropout("x", x, p)
    return _dropout_apply(x, p, seed)


def dropout_backward(dy: torch.Tensor, p: float, seed: int) -> torch.Tensor:
    """Return ``dx`` for inverted dropout given the drop probability and seed
    (dropout.py:90-112): the forward's mask, recomputed from ``seed``."""
    _check_dropout("dy", dy, p)
    return _dropout_apply(dy, p, seed)


class _DropoutAutograd(torch.autograd.Function):
    """dropout.py:115-136."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, p: float, seed: int) -> torch.Tensor:
        ctx.p = p
        ctx.seed = seed
        return _dropout_forward(x, p, seed)

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        if not ctx.needs_input_grad[0]:
            return None, None, None
        return dropout_backward(_contiguous_grad(grad_outputs[0]), ctx.p, ctx.seed), None, None


def dropout(x: torch.Tensor, p: float = 0.5, seed: int | None = None) -> torch.Tensor:
    """Apply inverted dropout to ``x`` with drop probability ``p`` (dropout.py:139-159).

    Kept elements are scaled by ``1 / (1 - p)``; the mask comes from ``seed``
    (drawn from the global torch RNG when ``None``) and is recomputed in the
    backward pass.  ``p == 0`` returns ``x`` itself."""
    if p == 0:
        return x
    if seed is None:
        seed = int(torch.randint(0, 2**31, (), dtype=torch.int64).item())
    if not requires_autograd(x):
        return _dropout_forward(x, p, seed)
    return _DropoutAutograd.apply(x, p, seed)


# ----------------------------------------------------------------------- sgd
def sgd_step(param: torch.Tensor, grad: torch.Tensor, lr: float, weight_decay: float = 0.0) -> None:
    """Update ``param`` in place: ``p -= lr * (g + weight_decay * p)`` in fp32
    (sgd.py:21-35, checks 38-47, entry 50-69)."""
    check_cuda_tensor("param", param)
    check_cuda_tensor("grad", grad)
    check_supported_dtype("param", param, FLOAT_DTYPES)
    check_same_shape_dtype_device("param", param, "grad", grad)
    check_contiguous("param", param, "for tritium.sgd_step")
    check_contiguous("grad", grad, "for tritium.sgd_step")
    if param.numel() == 0:
        return
    with torch.no_grad():
        p32 = param.float()
        param.copy_(p32 - lr * (grad.float() + weight_decay * p32))

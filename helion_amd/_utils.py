"""Argument validation shared by the ops (the reference's error contract).

Mirrors alkinun/helion ``tritium/ops/_utils.py:25-78``: the same checks raise
``ValueError`` with the same message shapes, because the reference's tests
match on them ("must be a CUDA tensor", "must be contiguous", "must have one of
these dtypes", "Shape mismatch", "Dtype mismatch", "Device mismatch").  On
ROCm builds of torch the device type of a GPU tensor is still ``"cuda"``.
"""

from __future__ import annotations

from collections.abc import Iterable

import torch

FLOAT_DTYPES = (torch.float16, torch.bfloat16, torch.float32)
INDEX_DTYPES = (torch.int32, torch.int64)


def next_power_of_2(n: int) -> int:
    return 1 if n <= 1 else 1 << (n - 1).bit_length()


def check_cuda_tensor(name: str, tensor: torch.Tensor) -> None:
    """_utils.py:25-27 (``is_cuda``: device type "cuda", without building a device object)."""
    if not tensor.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor.")


def check_contiguous(name: str, tensor: torch.Tensor, reason: str) -> None:
    """_utils.py:30-32."""
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous {reason}.")


def _dtype_names(dtypes: Iterable[torch.dtype]) -> str:
    return ", ".join(str(d).replace("torch.", "") for d in dtypes)


def check_supported_dtype(name: str, tensor: torch.Tensor, supported) -> None:
    """_utils.py:39-46."""
    if tensor.dtype not in supported:
        raise ValueError(f"{name} must have one of these dtypes: {_dtype_names(supported)}.")


def check_same_shape_dtype_device(lhs_name, lhs, rhs_name, rhs) -> None:
    """_utils.py:49-74."""
    check_cuda_tensor(lhs_name, lhs)
    check_cuda_tensor(rhs_name, rhs)
    if lhs.shape != rhs.shape:
        raise ValueError(
            f"Shape mismatch: {lhs_name} has shape {tuple(lhs.shape)}, "
            f"{rhs_name} has shape {tuple(rhs.shape)}."
        )
    if lhs.dtype != rhs.dtype:
        raise ValueError(
            f"Dtype mismatch: {lhs_name} has dtype {lhs.dtype}, "
            f"{rhs_name} has dtype {rhs.dtype}."
        )
    if lhs.device != rhs.device:
        raise ValueError(
            f"Device mismatch: {lhs_name} is on {lhs.device}, {rhs_name} is on {rhs.device}."
        )


def check_same_device(name: str, tensor: torch.Tensor, ref_name: str, ref: torch.Tensor) -> None:
    if tensor.device != ref.device:
        raise ValueError(
            f"Device mismatch: {name} is on {tensor.device}, {ref_name} is on {ref.device}."
        )


def requires_autograd(*tensors: torch.Tensor) -> bool:
    """_utils.py:77-78."""
    return torch.is_grad_enabled() and any(t.requires_grad for t in tensors)

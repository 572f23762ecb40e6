"""``rope`` and ``rope_`` on a gfx950 HIP kernel.

Drop-in for alkinun/helion ``tritium/ops/rope.py``: same signatures (``rope``
363-394, ``rope_`` 397-408), validation and messages (93-198), autograd
(``_RoPEAutograd`` 294-360, whose backward is the inverse rotation).

One deliberate tightening: without ``position_ids`` the host knows every
position (``t + position_offset``) and raises ``ValueError`` when the cos/sin
tables are too short, where the reference would read past them.  With
``position_ids`` the check would need a device->host sync, so the kernel
instead writes NaN for a token whose position has no table row.
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

SUPPORTED_DTYPES = FLOAT_DTYPES
SUPPORTED_POSITION_DTYPES = INDEX_DTYPES
MAX_ROPE_BLOCK_SIZE = 65536


def _check_position_ids(position_ids, q, n_tokens) -> None:
    """rope.py:93-116."""
    if position_ids is None:
        return
    check_cuda_tensor("position_ids", position_ids)
    check_supported_dtype("position_ids", position_ids, SUPPORTED_POSITION_DTYPES)
    if position_ids.device != q.device:
        raise ValueError(
            f"Device mismatch: position_ids is on {position_ids.device}, q is on {q.device}."
        )
    if position_ids.shape != (n_tokens,):
        raise ValueError(
            f"Shape mismatch: position_ids has shape {tuple(position_ids.shape)}, "
            f"expected ({n_tokens},)."
        )
    check_contiguous("position_ids", position_ids, "for tritium.rope")


def _check_rope_inputs(q, k, cos, sin, position_ids) -> tuple[int, int, int, int]:
    """rope.py:119-198."""
    for name, t in (("q", q), ("k", k), ("cos", cos), ("sin", sin)):
        check_cuda_tensor(name, t)
    for name, t in (("q", q), ("k", k), ("cos", cos), ("sin", sin)):
        check_supported_dtype(name, t, SUPPORTED_DTYPES)
    if q.shape != k.shape:
        raise ValueError(
            f"Shape mismatch: q has shape {tuple(q.shape)}, k has shape {tuple(k.shape)}."
        )
    if q.dtype != k.dtype:
        raise ValueError(f"Dtype mismatch: q has dtype {q.dtype}, k has dtype {k.dtype}.")
    for name, t in (("k", k), ("cos", cos), ("sin", sin)):
        if t.device != q.device:
            raise ValueError(f"Device mismatch: {name} is on {t.device}, q is on {q.device}.")
    if q.dim() == 2:
        n_tokens, head_dim = q.shape
        n_heads = 1
    elif q.dim() == 3:
        n_tokens, n_heads, head_dim = q.shape
    else:
        raise ValueError(
            "q and k must be shaped (n_tokens, head_dim) or (n_tokens, n_heads, head_dim)."
        )
    if head_dim % 2 != 0:
        raise ValueError("head_dim must be even for tritium.rope.")
    half = head_dim // 2
    block = next_power_of_2(half)
    if block > MAX_ROPE_BLOCK_SIZE:
        raise ValueError(
            f"Unsupported head_dim: next_power_of_2({half}) is {block}, "
            f"which exceeds {MAX_ROPE_BLOCK_SIZE}."
        )
    if cos.dim() != 2 or sin.dim() != 2:
        raise ValueError("cos and sin must be 2D tensors shaped (max_position, head_dim / 2).")
    if cos.shape != sin.shape:
        raise ValueError(
            f"Shape mismatch: cos has shape {tuple(cos.shape)}, sin has shape {tuple(sin.shape)}."
        )
    if cos.shape[1] != half:
        raise ValueError(
            f"Shape mismatch: cos last dimension is {cos.shape[1]}, expected {half}."
        )
    check_contiguous("q", q, "for tritium.rope")
    check_contiguous("k", k, "for tritium.rope")
    check_contiguous("cos", cos, "for tritium.rope")
    check_contiguous("sin", sin, "for tritium.rope")
    _check_position_ids(position_ids, q, n_tokens)
    return n_tokens, n_heads, head_dim, half


def _launch(q, k, cos, sin, position_ids, position_offset, interleaved, inverse, q_out, k_out):
    n_tokens, n_heads, head_dim, _ = _check_rope_inputs(q, k, cos, sin, position_ids)
    if position_offset < 0:
        raise ValueError("position_offset must be non-negative.")
    if q.numel() == 0:
        return
    max_position = cos.shape[0]
    if position_ids is None and n_tokens - 1 + position_offset >= max_position:
        raise ValueError(
            f"cos/sin have {max_position} positions, but position "
            f"{n_tokens - 1 + position_offset} is needed."
        )
    if sin.dtype != cos.dtype:
        sin = sin.to(cos.dtype)
    if position_ids is None:
        kind = 0
    else:
        kind = 1 if position_ids.dtype == torch.int32 else 2
    _lib.call(
        "tritium_rope",
        q.data_ptr(),
        k.data_ptr(),
        cos.data_ptr(),
        sin.data_ptr(),
        _lib.ptr(position_ids),
        kind,
        q_out.data_ptr(),
        k_out.data_ptr(),
        n_tokens,
        n_heads,
        head_dim,
        max_position,
        int(position_offset),
        int(bool(interleaved)),
        int(bool(inverse)),
        _lib.dtype_code(q.dtype),
        _lib.dtype_code(cos.dtype),
        _lib.stream_of(q),
    )


def rope_rows(q, k, cos, sin, position_ids, q_out, k_out, *, inverse: bool,
              in_token_stride: int, out_token_stride: int) -> None:
    """Rotate (or, with ``inverse``, un-rotate) token rows of q and k into
    q_out/k_out, where each operand is addressed as token * stride + head *
    head_dim + i with its own token stride -- e.g. q and k read in place from a
    fused [tokens, 3, heads, head_dim] projection (``tritium_rope_strided``).
    Not part of the reference's surface (its rope takes contiguous tensors
    only, rope.py:192-195): the training harness's fused split uses it.  q,
    k, q_out, k_out are [tokens, heads, head_dim]-shaped views with those
    strides and a unit head_dim stride; positions as in ``rope``.  q and
    q_out may both be None: k alone is rotated (for attention_rope_q, which
    rotates q as it loads it)."""
    if (q is None) != (q_out is None):
        raise ValueError("rope_rows: q and q_out are both given or both None (k alone)")
    n_tokens, n_heads, head_dim = k.shape
    for t in (q, q_out, k_out):
        if t is not None and (t.shape != k.shape or t.dtype != k.dtype or t.device != k.device):
            raise ValueError("rope_rows: q, k, q_out, k_out must share shape, dtype and device")
    for t, ts in ((q, in_token_stride), (k, in_token_stride), (q_out, out_token_stride),
                  (k_out, out_token_stride)):
        if t is not None and t.stride() != (ts, head_dim, 1):
            raise ValueError(f"rope_rows: expected strides {(ts, head_dim, 1)}, got {t.stride()}")
    if n_tokens == 0:
        return
    if sin.dtype != cos.dtype:
        sin = sin.to(cos.dtype)
    kind = 0 if position_ids is None else (1 if position_ids.dtype == torch.int32 else 2)
    _lib.call(
        "tritium_rope_strided", _lib.ptr(q), k.data_ptr(), cos.data_ptr(), sin.data_ptr(),
        _lib.ptr(position_ids), kind, _lib.ptr(q_out), k_out.data_ptr(), n_tokens, n_heads,
        head_dim, cos.shape[0], 0, 0, int(bool(inverse)), int(in_token_stride),
        int(out_token_stride), _lib.dtype_code(k.dtype), _lib.dtype_code(cos.dtype),
        _lib.stream_of(k),
    )


def _rope_forward(q, k, cos, sin, position_ids, position_offset, interleaved, inverse):
    """rope.py:201-247 (out of place)."""
    q_out = torch.empty_like(q)
    k_out = torch.empty_like(k)
    _launch(q, k, cos, sin, position_ids, position_offset, interleaved, inverse, q_out, k_out)
    return q_out, k_out


class _RoPEAutograd(torch.autograd.Function):
    """rope.py:294-360."""

    @staticmethod
    def forward(ctx: Any, q, k, cos, sin, position_ids, position_offset, interleaved):
        q_out, k_out = _rope_forward(
            q, k, cos, sin, position_ids, position_offset, interleaved, inverse=False
        )
        ctx.save_for_backward(cos, sin)
        ctx.position_ids = position_ids
        ctx.position_offset = position_offset
        ctx.interleaved = interleaved
        return q_out, k_out

    @staticmethod
    def backward(ctx: Any, *grad_outputs):
        dq_out, dk_out = grad_outputs
        cos, sin = ctx.saved_tensors
        dq = dk = None
        if dq_out is not None or dk_out is not None:
            if dq_out is None:
                dq_out = torch.zeros_like(dk_out)
            if dk_out is None:
                dk_out = torch.zeros_like(dq_out)
            if not dq_out.is_contiguous():
                dq_out = dq_out.contiguous()
            if not dk_out.is_contiguous():
                dk_out = dk_out.contiguous()
            dq, dk = _rope_forward(
                dq_out, dk_out, cos, sin, ctx.position_ids, ctx.position_offset,
                ctx.interleaved, inverse=True,
            )
        if not ctx.needs_input_grad[0]:
            dq = None
        if not ctx.needs_input_grad[1]:
            dk = None
        return dq, dk, None, None, None, None, None


def rope(
    q: torch.Tensor,
    k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    position_ids: torch.Tensor | None = None,
    position_offset: int = 0,
    interleaved: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Apply rotary embeddings to q and k over the last dimension (rope.py:363-394)."""
    if not requires_autograd(q, k):
        return _rope_forward(
            q, k, cos, sin, position_ids, position_offset, interleaved, inverse=False
        )
    return _RoPEAutograd.apply(q, k, cos, sin, position_ids, position_offset, interleaved)


def rope_(
    q: torch.Tensor,
    k: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    *,
    position_ids: torch.Tensor | None = None,
    position_offset: int = 0,
    interleaved: bool = False,
) -> None:
    """Apply rotary embeddings to q and k in-place (rope.py:397-408)."""
    _launch(q, k, cos, sin, position_ids, position_offset, interleaved, False, q, k)

"""Embedding backward with a tied output head, on a gfx950 HIP kernel.

The reference's ``Embedding`` (alkinun/helion ``helion/nn.py:24-28``) is the
gather ``weight[ids]`` with torch's autograd backward (a sort of the ids and a
scatter-add); the benchmark's model (``examples/common.py``) ties that weight
to the output head, so autograd also adds the head's weight gradient in a
separate pass.  :func:`embedding_backward` does the scatter-add and that add
in one deterministic kernel (``tritium_embedding_bwd``); the training
harness's tied embedding uses it.  Not part of the reference's
``tritium.ops`` surface (the reference has no embedding op).
"""

from __future__ import annotations

import torch

from . import _lib
from ._utils import check_contiguous, check_cuda_tensor

INDEX_DTYPES = (torch.int32, torch.int64)


def embedding_backward(ids: torch.Tensor, dx: torch.Tensor, dw: torch.Tensor,
                       out: torch.Tensor | None = None) -> torch.Tensor:
    """``dw + scatter_add(ids, dx)`` for ``ids [n]``, ``dx [n, dim]`` (row
    stride any multiple of 1, unit column stride) and ``dw [vocab, dim]``,
    summed in fp32 in token order and rounded once into ``dw``'s dtype.
    ``out`` (default: a new tensor) may be ``dw`` itself.  Ids outside
    ``[0, vocab)`` add nothing."""
    for name, t in (("ids", ids), ("dx", dx), ("dw", dw)):
        check_cuda_tensor(name, t)
    if ids.dtype not in INDEX_DTYPES:
        raise ValueError(f"ids must have one of these dtypes: {INDEX_DTYPES}, got {ids.dtype}.")
    if dw.dim() != 2 or dx.dim() != 2:
        raise ValueError("dx must be [n_tokens, dim] and dw [vocab, dim].")
    n, dim = dx.shape
    if ids.numel() != n or dw.shape[1] != dim:
        raise ValueError(
            f"Shape mismatch: ids {tuple(ids.shape)}, dx {tuple(dx.shape)}, dw {tuple(dw.shape)}."
        )
    if dx.dtype != dw.dtype:
        raise ValueError(f"Dtype mismatch: dx has dtype {dx.dtype}, dw has dtype {dw.dtype}.")
    if dx.device != dw.device or ids.device != dw.device:
        raise ValueError("Device mismatch: ids, dx and dw must be on one device.")
    check_contiguous("dw", dw, "for embedding_backward")
    if dx.stride(1) != 1:
        dx = dx.contiguous()
    ids = ids.contiguous()
    if out is None:
        out = torch.empty_like(dw)
    elif out.shape != dw.shape or out.dtype != dw.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor like dw.")
    vocab = dw.shape[0]
    ws_bytes = _lib.lib().tritium_embedding_bwd_workspace_size(n, vocab, dim)
    ws = torch.empty((max(ws_bytes, 1),), device=dw.device, dtype=torch.uint8)
    _lib.call(
        "tritium_embedding_bwd", ids.data_ptr(), 1 if ids.dtype == torch.int32 else 2, n,
        dx.data_ptr(), dx.stride(0) if n > 0 else dim, dw.data_ptr(), out.data_ptr(), vocab, dim,
        ws.data_ptr(), ws_bytes, _lib.dtype_code(dw.dtype), _lib.stream_of(dw),
    )
    return out

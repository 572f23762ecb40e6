"""``attention`` on gfx950 HIP kernels (bf16/fp16 MFMA for head_dim 16-256;
fp32, and 16-bit head_dims 512 and 1024, on a SIMT path).

Drop-in for alkinun/helion ``tritium/ops/attention.py``: same signature
(``attention(q, k, v, *, is_causal=True)`` 739-757), validation and messages
(``_check_attention_inputs`` 220-281), autograd (``_AttentionAutograd``
705-736), GQA, ``q_len != kv_len``, strided q/k/v (the module path passes
``transpose(1, 2)`` views, helion/nn.py:212-220) and the KV-cache
``q_len == 1`` call (helion/nn.py:275-280).

Differences:

* ``dq``, ``dk`` and ``dv`` are written with their own strides.  The
  reference stores ``dq`` as if it were contiguous while allocating it with
  q's strides (attention.py:625-629 vs 645), which permutes it for the
  module's transposed views; here it is correct for any layout;
* ``dk``/``dv`` are reduced in registers (no fp32 atomics) and the results are
  bitwise deterministic;
* head_dim above 1024 is rejected (the reference's autotuned Triton kernel
  has no fixed bound, but its register tiles would not fit either).
"""

from __future__ import annotations

import collections
import ctypes
from typing import Any

import torch

from . import _lib
from ._utils import FLOAT_DTYPES, check_cuda_tensor, check_supported_dtype, requires_autograd

SUPPORTED_DTYPES = FLOAT_DTYPES
MAX_HEAD_DIM = 1024
# The backward stores dS (2 bytes per visible (query, key) pair) for head_dim
# 128 when that workspace stays within this many bytes; above it (long
# sequences) it recomputes S and dP in its dQ kernel instead.
DS_WORKSPACE_MAX_BYTES = 8 << 30


def _check_attention_inputs(q, k, v) -> tuple[int, int, int, int, int, int]:
    """attention.py:220-281."""
    for name, t in (("q", q), ("k", k), ("v", v)):
        check_cuda_tensor(name, t)
        check_supported_dtype(name, t, SUPPORTED_DTYPES)
    if q.dim() != 4:
        raise ValueError("q must be a 4D tensor shaped (batch, n_heads, q_seq_len, head_dim).")
    batch, n_heads, q_len, head_dim = q.shape
    ks = k.shape
    n_kv_heads = ks[1] if len(ks) == 4 else 0
    kv_len = ks[2] if len(ks) == 4 else 0
    qdtype, qdev = q.dtype, q.device
    for name, t in (("k", k), ("v", v)):
        s = t.shape
        if len(s) != 4:
            raise ValueError(
                f"{name} must be a 4D tensor shaped (batch, n_kv_heads, kv_seq_len, head_dim)."
            )
        if s[0] != batch:
            raise ValueError(f"Shape mismatch: {name} has batch {s[0]}, expected {batch}.")
        if s[2] != kv_len:
            raise ValueError(f"Shape mismatch: {name} has seq_len {s[2]}, expected {kv_len}.")
        if s[3] != head_dim:
            raise ValueError(f"Shape mismatch: {name} has head_dim {s[3]}, expected {head_dim}.")
        if s[1] != n_kv_heads:
            raise ValueError(
                f"Shape mismatch: {name} has {s[1]} kv heads, expected {n_kv_heads}."
            )
        if t.dtype != qdtype:
            raise ValueError(f"Dtype mismatch: {name} has dtype {t.dtype}, q has dtype {qdtype}.")
        if t.device != qdev:
            raise ValueError(f"Device mismatch: {name} is on {t.device}, q is on {qdev}.")
    if n_kv_heads == 0 or n_heads % n_kv_heads != 0:
        raise ValueError(
            f"n_heads ({n_heads}) must be divisible by n_kv_heads ({n_kv_heads})."
        )
    if head_dim < 16 or (head_dim & (head_dim - 1)) != 0:
        raise ValueError(f"head_dim must be a power of 2 >= 16, got {head_dim}.")
    if head_dim > MAX_HEAD_DIM:
        raise ValueError(f"head_dim must be <= {MAX_HEAD_DIM}, got {head_dim}.")
    return batch, n_heads, n_kv_heads, q_len, kv_len, head_dim


def _unit_last(t: torch.Tensor) -> torch.Tensor:
    """The kernels address rows through (batch, head, seq) strides; head_dim
    must be the unit-stride dimension."""
    return t if t.stride(-1) == 1 else t.contiguous()


def _rows_aligned(t: torch.Tensor) -> bool:
    """Unit head_dim stride, 16-byte aligned base and row strides (what the MFMA
    kernels need of every operand to take it in place)."""
    es = t.element_size()
    st = t.stride()
    return (st[3] == 1 and t.data_ptr() % 16 == 0
            and (st[0] * es) % 16 == 0 and (st[1] * es) % 16 == 0 and (st[2] * es) % 16 == 0)


_Strides12 = ctypes.c_int64 * 12


def _strides(*ts: torch.Tensor):
    """(batch, head, seq) strides of each tensor as a host int64 array (read by
    the entry point before it returns)."""
    vals: list[int] = []
    for t in ts:
        vals.extend(t.stride()[:3])
    if len(vals) == 12:
        return _Strides12(*vals)
    return (ctypes.c_int64 * len(vals))(*vals)


# Decode workspaces, one per (device, stream), grown on demand: calls on one
# stream never overlap, so each reuses its stream's buffer instead of
# allocating one per call (the partials are written before they are read).
# Only the _DECODE_WS_KEEP most recently used streams keep theirs: a caller
# that makes a stream per request retains at most that many buffers, each the
# size of the largest call seen on its stream.  An evicted buffer goes back to
# torch's caching allocator, ordered on the stream it was allocated on.
_DECODE_WS: "collections.OrderedDict[tuple[int, int], torch.Tensor]" = collections.OrderedDict()
_DECODE_WS_KEEP = 4


def _decode_workspace(dev: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    n = max(nbytes, 4) // 4
    if torch.cuda.is_current_stream_capturing():
        return torch.empty((n,), device=dev, dtype=torch.float32)
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), stream)
    buf = _DECODE_WS.get(key)
    if buf is None or buf.numel() < n:
        buf = torch.empty((n,), device=dev, dtype=torch.float32)
        _DECODE_WS[key] = buf
    _DECODE_WS.move_to_end(key)
    while len(_DECODE_WS) > _DECODE_WS_KEEP:
        _DECODE_WS.popitem(last=False)
    return buf


def _attention_forward(q, k, v, is_causal: bool):
    """attention.py:284-351."""
    batch, n_heads, n_kv_heads, q_len, kv_len, head_dim = _check_attention_inputs(q, k, v)
    q, k, v = _unit_last(q), _unit_last(k), _unit_last(v)
    o = torch.empty_like(q)
    if o.stride(-1) != 1:
        o = torch.empty(q.shape, device=q.device, dtype=q.dtype)
    lse = torch.empty((batch, n_heads, q_len), device=q.device, dtype=torch.float32)
    if q_len == 0 or batch == 0:
        return o, lse
    strides = _strides(q, k, v, o)
    if (q_len == 1 and not is_causal and kv_len > 0 and q.dtype != torch.float32
            and head_dim in (64, 128) and n_heads // n_kv_heads <= 8
            and all(_rows_aligned(t) for t in (q, k, v))):
        # decode: one query row per head against a K/V cache, split over the keys
        ws_bytes = _lib.lib().tritium_attention_decode_workspace_size(
            batch, n_heads, n_kv_heads, kv_len, head_dim)
        stream = _lib.stream_of(q)
        ws = _decode_workspace(q.device, stream, ws_bytes)
        _lib.call(
            "tritium_attention_decode", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
            lse.data_ptr(), ws.data_ptr(), ws_bytes, batch, n_heads, n_kv_heads, kv_len,
            head_dim, strides, _lib.dtype_code(q.dtype), stream,
        )
        return o, lse
    _lib.call(
        "tritium_attention_fwd",
        q.data_ptr(),
        k.data_ptr(),
        v.data_ptr(),
        o.data_ptr(),
        lse.data_ptr(),
        batch,
        n_heads,
        n_kv_heads,
        q_len,
        kv_len,
        head_dim,
        strides,
        int(bool(is_causal)),
        _lib.dtype_code(q.dtype),
        _lib.stream_of(q),
    )
    return o, lse


def _ds_workspace(q, batch, n_heads, q_len, kv_len, head_dim, is_causal):
    """The dS workspace of the backward (tensor, bytes), or (None, 0) where the
    shape takes none or it would exceed DS_WORKSPACE_MAX_BYTES."""
    n = _lib.lib().tritium_attention_bwd_workspace_size(
        batch, n_heads, q_len, kv_len, head_dim, int(bool(is_causal)), _lib.dtype_code(q.dtype))
    if not 0 < n <= DS_WORKSPACE_MAX_BYTES:
        return None, 0
    return torch.empty((n,), device=q.device, dtype=torch.uint8), n


def _attention_backward_impl(do, q, k, v, o, lse, is_causal: bool):
    """attention.py:632-702, with correct strided outputs and no atomics."""
    batch, n_heads, n_kv_heads, q_len, kv_len, head_dim = _check_attention_inputs(q, k, v)
    q, k, v, o, do = (_unit_last(t) for t in (q, k, v, o, do))
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    if q_len == 0 or batch == 0 or kv_len == 0:
        return dq.zero_(), dk.zero_(), dv.zero_()
    delta = torch.empty((batch * n_heads * q_len,), device=q.device, dtype=torch.float32)
    strides = _strides(q, k, v, o, do, dq, dk, dv)
    ws, ws_bytes = _ds_workspace(q, batch, n_heads, q_len, kv_len, head_dim, is_causal)
    _lib.call(
        "tritium_attention_bwd_ws",
        do.data_ptr(),
        q.data_ptr(),
        k.data_ptr(),
        v.data_ptr(),
        o.data_ptr(),
        lse.data_ptr(),
        dq.data_ptr(),
        dk.data_ptr(),
        dv.data_ptr(),
        delta.data_ptr(),
        ws.data_ptr() if ws is not None else None,
        ws_bytes,
        batch,
        n_heads,
        n_kv_heads,
        q_len,
        kv_len,
        head_dim,
        strides,
        int(bool(is_causal)),
        _lib.dtype_code(q.dtype),
        _lib.stream_of(q),
    )
    return dq, dk, dv


class _AttentionAutograd(torch.autograd.Function):
    """attention.py:705-736."""

    @staticmethod
    def forward(ctx: Any, q, k, v, is_causal: bool):
        o, lse = _attention_forward(q, k, v, is_causal)
        ctx.save_for_backward(q, k, v, o, lse)
        ctx.is_causal = is_causal
        return o

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        do = grad_outputs[0]
        q, k, v, o, lse = ctx.saved_tensors
        # attention.py:726-727 copies a non-contiguous upstream gradient; the kernels read
        # dO through its own (batch, head, seq) strides, so a copy is needed only when
        # those strides would break 16-byte row alignment (e.g. not the transposed
        # [batch, seq, heads, head_dim] view a module passes)
        if not do.is_contiguous() and not _rows_aligned(do):
            do = do.contiguous()
        dq, dk, dv = _attention_backward_impl(do, q, k, v, o, lse, ctx.is_causal)
        return (
            dq if ctx.needs_input_grad[0] else None,
            dk if ctx.needs_input_grad[1] else None,
            dv if ctx.needs_input_grad[2] else None,
            None,
        )


def attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    *,
    is_causal: bool = True,
) -> torch.Tensor:
    """Compute scaled dot-product attention over the last two dimensions.

    q: (batch, n_heads, q_seq_len, head_dim); k, v: (batch, n_kv_heads,
    kv_seq_len, head_dim) with n_heads divisible by n_kv_heads (GQA).
    head_dim must be a power of 2 >= 16.  The causal mask is top-left aligned
    (query i sees keys 0..i), as in attention.py:112-113.
    """
    if not requires_autograd(q, k, v):
        o, _ = _attention_forward(q, k, v, is_causal)
        return o
    return _AttentionAutograd.apply(q, k, v, is_causal)


# ------------------------------------------------------- RoPE on q's load --
# Not part of the reference's surface: its model rotates q and k into new
# tensors and then calls attention (helion/nn.py:196-220).  These run that
# sequence with q rotated as the attention kernels load it, so no rotated
# copy of q is written in the forward or kept for the backward; k arrives
# rotated (tritium_rope_strided rotates it alone).


def _check_rope_q(q, k, v, cos, sin, position_ids):
    batch, n_heads, n_kv_heads, q_len, kv_len, head_dim = _check_attention_inputs(q, k, v)
    if q.dtype not in (torch.bfloat16, torch.float16) or head_dim not in (64, 128):
        raise ValueError("attention with rope on q needs bf16/fp16 tensors with head_dim 64 or "
                         f"128, got {q.dtype} and head_dim {head_dim}")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not _rows_aligned(t):
            raise ValueError(f"attention with rope on q: {name} needs a unit head_dim stride and "
                             "16-byte aligned rows")
    for name, t in (("cos", cos), ("sin", sin)):
        if (t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != head_dim // 2
                or not t.is_contiguous() or t.device != q.device):
            raise ValueError(f"attention with rope on q: {name} must be a contiguous float32 "
                             f"[max_position, {head_dim // 2}] tensor on {q.device}")
    if cos.shape != sin.shape:
        raise ValueError("attention with rope on q: cos and sin shapes differ")
    if position_ids is not None:
        if (position_ids.dtype not in (torch.int32, torch.int64) or not position_ids.is_contiguous()
                or position_ids.numel() != batch * q_len or position_ids.device != q.device):
            raise ValueError("attention with rope on q: position_ids must be a contiguous int32 "
                             f"or int64 tensor of batch * q_len = {batch * q_len} positions")
    return batch, n_heads, n_kv_heads, q_len, kv_len, head_dim


def _pos_args(position_ids):
    if position_ids is None:
        return None, 0
    return position_ids.data_ptr(), (1 if position_ids.dtype == torch.int32 else 2)


def attention_rope_fwd(q, k, v, cos, sin, position_ids, is_causal: bool, o=None):
    """Forward of attention(rope(q), k, v): q unrotated, k rotated; returns
    (o, lse).  ``o`` may be given (any layout with 16-byte aligned rows)."""
    batch, n_heads, n_kv_heads, q_len, kv_len, head_dim = _check_rope_q(q, k, v, cos, sin,
                                                                         position_ids)
    if o is None:
        o = torch.empty((batch, q_len, n_heads, head_dim), device=q.device,
                        dtype=q.dtype).transpose(1, 2)
    lse = torch.empty((batch, n_heads, q_len), device=q.device, dtype=torch.float32)
    if q_len == 0 or batch == 0:
        return o, lse
    pos_ptr, kind = _pos_args(position_ids)
    _lib.call("tritium_attention_fwd_rope", q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
              lse.data_ptr(), batch, n_heads, n_kv_heads, q_len, kv_len, head_dim,
              _strides(q, k, v, o), int(bool(is_causal)), _lib.dtype_code(q.dtype),
              cos.data_ptr(), sin.data_ptr(), pos_ptr, kind, cos.shape[0], _lib.stream_of(q))
    return o, lse


def attention_rope_bwd(do, q, k, v, o, lse, cos, sin, position_ids, is_causal: bool,
                       dq=None, dk=None, dv=None):
    """Backward of ``attention_rope_fwd``: dq is the gradient of the unrotated
    q.  dq/dk/dv may be given as strided views (16-byte aligned rows)."""
    batch, n_heads, n_kv_heads, q_len, kv_len, head_dim = _check_rope_q(q, k, v, cos, sin,
                                                                         position_ids)
    dq = torch.empty_like(q) if dq is None else dq
    dk = torch.empty_like(k) if dk is None else dk
    dv = torch.empty_like(v) if dv is None else dv
    if q_len == 0 or batch == 0 or kv_len == 0:
        for t in (dq, dk, dv):
            t.zero_()
        return dq, dk, dv
    if not _rows_aligned(do):
        do = do.contiguous()
    delta = torch.empty((batch * n_heads * q_len,), device=q.device, dtype=torch.float32)
    q_rot = torch.empty((batch, n_heads, q_len, head_dim), device=q.device, dtype=q.dtype)
    pos_ptr, kind = _pos_args(position_ids)
    ws, ws_bytes = _ds_workspace(q, batch, n_heads, q_len, kv_len, head_dim, is_causal)
    _lib.call("tritium_attention_bwd_rope_ws", do.data_ptr(), q.data_ptr(), k.data_ptr(),
              v.data_ptr(), o.data_ptr(), lse.data_ptr(), dq.data_ptr(), dk.data_ptr(),
              dv.data_ptr(), delta.data_ptr(), q_rot.data_ptr(),
              ws.data_ptr() if ws is not None else None, ws_bytes, batch, n_heads,
              n_kv_heads, q_len, kv_len, head_dim, _strides(q, k, v, o, do, dq, dk, dv),
              int(bool(is_causal)), _lib.dtype_code(q.dtype), cos.data_ptr(), sin.data_ptr(),
              pos_ptr, kind, cos.shape[0], _lib.stream_of(q))
    return dq, dk, dv


class _AttentionRopeQ(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, q, k, v, cos, sin, position_ids, is_causal: bool):
        o, lse = attention_rope_fwd(q, k, v, cos, sin, position_ids, is_causal)
        ctx.save_for_backward(q, k, v, o, lse, cos, sin, position_ids)
        ctx.is_causal = is_causal
        return o

    @staticmethod
    def backward(ctx: Any, *grad_outputs: torch.Tensor):
        q, k, v, o, lse, cos, sin, position_ids = ctx.saved_tensors
        dq, dk, dv = attention_rope_bwd(grad_outputs[0], q, k, v, o, lse, cos, sin, position_ids,
                                        ctx.is_causal)
        return dq, dk, dv, None, None, None, None


def attention_rope_q(q, k, v, cos, sin, position_ids=None, *, is_causal: bool = True):
    """``attention(rope(q), k, v, is_causal=...)`` with q rotated as the kernels
    load it: q unrotated (batch, n_heads, q_len, head_dim), k already
    rotated, cos/sin float32 [max_position, head_dim / 2] (non-interleaved
    halves, as ``rope``), position_ids one per (batch, query row) in
    batch-major order or None (position = query row).  The gradient of q is
    that of the unrotated q.  bf16/fp16 with head_dim 64 or 128."""
    if not requires_autograd(q, k, v):
        return attention_rope_fwd(q, k, v, cos, sin, position_ids, is_causal)[0]
    return _AttentionRopeQ.apply(q, k, v, cos, sin, position_ids, is_causal)

"""Rotary position embedding forward/inverse (test infrastructure).

Follows alkinun/helion ``tritium/ops/rope.py``:

* position of token t is ``position_ids[t] + offset`` or ``t + offset``
  (rope.py:47-50);
* cos/sin rows are indexed by that position and upcast to fp32 (rope.py:52-57);
* pairs are ``(x[i], x[i+half])`` or, interleaved, ``(x[2i], x[2i+1])``
  (rope.py:60-65);
* forward rotation ``(a*c - b*s, b*c + a*s)``, inverse (the backward)
  ``(a*c + b*s, b*c - a*s)`` (rope.py:76-85), computed in fp32 and stored in
  the input dtype.

Pinned by (tests/test_oracle.py, test_rope_*): the complex-multiplication restatement
``(a + i b) * exp(+-i theta)``, identity at position 0, conservation of every
pair's norm, ``inverse(forward(x)) == x`` in float64, torch autograd of the
forward (which must equal the inverse rotation: the reference never checks
backward values, tests/tritium/test_rope.py:109-121), and the reference's test
formula (tests/tritium/test_rope.py:11-35) in the golden fixtures.
"""

from __future__ import annotations

import numpy as np

from .numerics import quantize


def make_cos_sin(max_seq_len: int, head_dim: int, theta: float = 10000.0):
    """fp32 cos/sin tables ``[max_seq_len, head_dim/2]`` -- test_rope.py:38-45."""
    half = head_dim // 2
    inv_freq = (1.0 / (theta ** (np.arange(half, dtype=np.float32) / np.float32(half)))).astype(
        np.float32
    )
    t = np.arange(max_seq_len, dtype=np.float32)
    freqs = np.outer(t, inv_freq).astype(np.float32)
    return np.cos(freqs).astype(np.float32), np.sin(freqs).astype(np.float32)


def positions(n_tokens: int, position_ids=None, position_offset: int = 0) -> np.ndarray:
    """Per-token table row -- rope.py:47-50."""
    if position_ids is None:
        return np.arange(n_tokens, dtype=np.int64) + position_offset
    return np.asarray(position_ids, dtype=np.int64) + position_offset


def apply(
    x: np.ndarray,
    cos: np.ndarray,
    sin: np.ndarray,
    position_ids=None,
    position_offset: int = 0,
    interleaved: bool = False,
    inverse: bool = False,
    dtype: str = "f32",
) -> np.ndarray:
    """Rotate one tensor ``x`` of shape ``[T, D]`` or ``[T, H, D]`` -- rope.py:42-90."""
    x3 = np.asarray(x, dtype=np.float32)
    squeeze = x3.ndim == 2
    if squeeze:
        x3 = x3[:, None, :]
    n_tokens, _, head_dim = x3.shape
    half = head_dim // 2
    pos = positions(n_tokens, position_ids, position_offset)
    c = cos.astype(np.float32)[pos][:, None, :]
    s = sin.astype(np.float32)[pos][:, None, :]
    if interleaved:
        a, b = x3[..., 0::2], x3[..., 1::2]
    else:
        a, b = x3[..., :half], x3[..., half:]
    if inverse:
        first, second = a * c + b * s, b * c - a * s
    else:
        first, second = a * c - b * s, b * c + a * s
    out = np.empty_like(x3)
    if interleaved:
        out[..., 0::2], out[..., 1::2] = first, second
    else:
        out[..., :half], out[..., half:] = first, second
    out = quantize(out, dtype)
    return out[:, 0, :] if squeeze else out


def forward(q, k, cos, sin, position_ids=None, position_offset=0, interleaved=False,
            dtype="f32"):
    """``rope(q, k, ...)`` -- rope.py:363-394."""
    kw = dict(position_ids=position_ids, position_offset=position_offset,
              interleaved=interleaved, dtype=dtype)
    return apply(q, cos, sin, **kw), apply(k, cos, sin, **kw)


def backward(dq_out, dk_out, cos, sin, position_ids=None, position_offset=0,
             interleaved=False, dtype="f32"):
    """``_RoPEAutograd.backward``: the inverse rotation of the grads -- rope.py:345-354."""
    kw = dict(position_ids=position_ids, position_offset=position_offset,
              interleaved=interleaved, inverse=True, dtype=dtype)
    return apply(dq_out, cos, sin, **kw), apply(dk_out, cos, sin, **kw)

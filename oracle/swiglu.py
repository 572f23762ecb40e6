"""SwiGLU forward and backward (test infrastructure).

Follows alkinun/helion ``tritium/ops/swiglu.py``: ``silu(x) * gate`` in fp32
(swiglu.py:32-35); backward ``dx = dy * gate * sig * (1 + x * (1 - sig))``,
``dgate = dy * silu(x)`` (swiglu.py:51-58); the first argument gets the silu.

Pinned by (tests/test_oracle.py, test_swiglu_*): torch ``F.silu(x) * gate`` and its
autograd (tests/tritium/test_swiglu.py:9-10, 25-36), the special case x = 0
(``out = 0``, ``dgate = 0``, ``dx = dy * gate / 2``), a float64
finite-difference check, and the golden fixtures.
"""

from __future__ import annotations

import numpy as np

from .numerics import quantize


def _sigmoid(x: np.ndarray) -> np.ndarray:
    return (np.float32(1.0) / (np.float32(1.0) + np.exp(-x))).astype(np.float32)


def forward(x: np.ndarray, gate: np.ndarray, dtype: str = "f32") -> np.ndarray:
    """``silu(x) * gate`` -- swiglu.py:32-35."""
    x = x.astype(np.float32)
    return quantize(x * _sigmoid(x) * gate.astype(np.float32), dtype)


def backward(dy: np.ndarray, x: np.ndarray, gate: np.ndarray, dtype: str = "f32"):
    """``(dx, dgate)`` -- swiglu.py:51-58."""
    x = x.astype(np.float32)
    dy = dy.astype(np.float32)
    gate = gate.astype(np.float32)
    sig = _sigmoid(x)
    silu = x * sig
    dsilu = sig * (np.float32(1.0) + x * (np.float32(1.0) - sig))
    return quantize(dy * gate * dsilu, dtype), quantize(dy * silu, dtype)

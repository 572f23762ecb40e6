"""RMSNorm / residual RMSNorm forward and backward (test infrastructure).

Follows alkinun/helion ``tritium/ops/rmsnorm.py``:

* forward ``_rmsnorm_forward_kernel`` rmsnorm.py:45-51 -- fp32 ``mean(x^2)``,
  ``rstd = 1 / sqrt(mean + eps)``, ``y = x * rstd * w`` stored in x's dtype,
  ``rstd`` saved in fp32;
* residual forward ``_residual_rmsnorm_forward_kernel`` rmsnorm.py:72-83 --
  ``z = x + r`` in fp32, normalised from the fp32 ``z``; ``z`` is stored in
  x's dtype and that rounded ``z`` is what the backward sees (rmsnorm.py:697);
* backward ``_rmsnorm_backward_dx_kernel`` rmsnorm.py:121-129 and
  ``_rmsnorm_dweight_stage1_kernel`` rmsnorm.py:253 --
  ``dx = rstd*(dy*w) - (rstd^3/H) * x * sum(dy*w*x)``,
  ``dw = sum_rows(dy * x * rstd)`` in fp32, cast to w's dtype (rmsnorm.py:439);
* standalone ``rmsnorm_backward`` recomputes rstd from x (rmsnorm.py:184-185);
* residual backward ``dz = rmsnorm_bwd(dy) + dresidual_out``, returned for both
  x and residual (rmsnorm.py:720-734).

Pinned by (tests/test_oracle.py, test_rmsnorm_*): torch's ``F.rms_norm`` library
routine, the closed form for a constant row ``y = w*c/sqrt(c^2+eps)``, torch
autograd of the forward (an independent derivation of dx and dw), a float64
finite-difference gradient check, and the reference's own test formulas
(tests/tritium/test_rmsnorm.py:12-48) in the golden fixtures.
"""

from __future__ import annotations

import numpy as np

from .numerics import quantize


def _rows(x: np.ndarray, acc=np.float32) -> np.ndarray:
    return np.asarray(x).astype(acc).reshape(-1, x.shape[-1])


def rstd_of(x2d: np.ndarray, eps: float, acc=np.float32) -> np.ndarray:
    """Per-row ``1/sqrt(mean(x^2)+eps)`` -- rmsnorm.py:46-47."""
    x2d = x2d.astype(acc)
    mean_sq = (x2d * x2d).sum(axis=1, dtype=acc) / acc(x2d.shape[1])
    return (acc(1.0) / np.sqrt(mean_sq + acc(eps))).astype(acc)


def forward(x: np.ndarray, w: np.ndarray, eps: float = 1e-6, dtype: str = "f32",
            acc=np.float32):
    """Return ``(y, rstd)``; y rounded to ``dtype`` -- rmsnorm.py:45-51.

    ``acc`` is the arithmetic width: float32 as the reference kernel, or
    float64 for a truth value to measure float32 kernels against.
    """
    x2d = _rows(x, acc)
    rstd = rstd_of(x2d, eps, acc)
    y = x2d * rstd[:, None] * w.astype(acc)[None, :]
    return quantize(y, dtype).reshape(x.shape), rstd


def residual_forward(
    x: np.ndarray, r: np.ndarray, w: np.ndarray, eps: float = 1e-6, dtype: str = "f32",
    acc=np.float32,
):
    """Return ``(y, z, rstd)`` with ``z = x + r`` -- rmsnorm.py:72-83."""
    z = _rows(x, acc) + _rows(r, acc)
    rstd = rstd_of(z, eps, acc)
    y = z * rstd[:, None] * w.astype(acc)[None, :]
    return (
        quantize(y, dtype).reshape(x.shape),
        quantize(z, dtype).reshape(x.shape),
        rstd,
    )


def backward(
    dy: np.ndarray,
    x: np.ndarray,
    w: np.ndarray,
    rstd: np.ndarray | None = None,
    eps: float = 1e-6,
    dtype: str = "f32",
    w_dtype: str | None = None,
    acc=np.float32,
):
    """Return ``(dx, dw)`` -- rmsnorm.py:121-129 (dx) and 253, 279, 439 (dw).

    ``rstd=None`` recomputes it from x as the standalone ``rmsnorm_backward``
    does (rmsnorm.py:184-185).
    """
    x2d = _rows(x, acc)
    dy2d = _rows(dy, acc)
    hidden = x2d.shape[1]
    if rstd is None:
        rstd = rstd_of(x2d, eps, acc)
    rstd = rstd.astype(acc)[:, None]
    wf = w.astype(acc)[None, :]
    weighted = dy2d * wf
    c = (weighted * x2d).sum(axis=1, dtype=acc)[:, None]
    dx = rstd * weighted - (rstd * rstd * rstd / acc(hidden)) * x2d * c
    dw = (dy2d * x2d * rstd).sum(axis=0, dtype=acc)
    return (
        quantize(dx, dtype).reshape(x.shape),
        quantize(dw, w_dtype or dtype),
    )


def residual_backward(
    dy: np.ndarray,
    dz_out: np.ndarray,
    z: np.ndarray,
    w: np.ndarray,
    rstd: np.ndarray,
    dtype: str = "f32",
    acc=np.float32,
):
    """Return ``(dz, dw)``: ``dz = rmsnorm_bwd(dy) + dresidual_out`` -- rmsnorm.py:718-734.

    The reference rounds the rmsnorm dx to the storage dtype before the add
    (rmsnorm.py:729-730); both roundings are reproduced here.
    """
    dx, dw = backward(dy, z, w, rstd=rstd, dtype=dtype, acc=acc)
    dz = quantize(_rows(dx, acc) + _rows(dz_out, acc), dtype).reshape(z.shape)
    return dz, dw

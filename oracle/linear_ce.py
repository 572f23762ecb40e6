"""Fused linear + cross-entropy forward and backward (test infrastructure).

Follows alkinun/helion ``tritium/ops/cross_entropy.py``:

* forward (cross_entropy.py:219-293): ``logits = hidden @ weight^T`` with fp32
  accumulation, per-row ``lse = max + ln(sum exp(logits - max))``,
  ``nll = lse - logits[target]``, mean over rows;
* backward (cross_entropy.py:103-131 and 937-957):
  ``G = (exp(logits - lse) - onehot(target)) * grad_out / denominator``,
  ``dhidden = G @ weight``, ``dweight = G^T @ hidden``.

``ignore_index`` is NOT in the reference (it never checks for ignored targets,
cross_entropy.py:240-244, 281-289); the semantics here are PyTorch's
``F.cross_entropy(..., ignore_index=-100, reduction="mean")``: ignored rows
contribute nothing to the loss or the gradients and the mean divides by the
number of non-ignored rows (all rows ignored gives NaN, as torch does).  With
no ignored target the result is the reference's.

Arithmetic is float64 by default (the fp32-or-better reference the north-star
tolerance is quoted against).

Pinned by (tests/test_oracle.py, test_linear_ce_*): torch
``F.cross_entropy(F.linear(h, W).float(), t, ignore_index=-100)`` and its
autograd (tests/tritium/test_cross_entropy.py:72, 93), the closed form for
``W = 0`` (``loss = ln V``, ``dH = 0``, ``dW = (1/V - onehot)^T h / N_valid``),
an all-ignored batch giving NaN, a float64 finite-difference gradient check,
and the golden fixtures.
"""

from __future__ import annotations

import numpy as np

IGNORE_INDEX = -100


def forward(hidden, weight, target, ignore_index: int = IGNORE_INDEX, acc=np.float64):
    """Return ``(loss, lse)`` -- cross_entropy.py:219-293 plus torch ignore_index."""
    h = hidden.reshape(-1, hidden.shape[-1]).astype(acc)
    w = weight.astype(acc)
    t = np.asarray(target).reshape(-1).astype(np.int64)
    logits = h @ w.T
    m = logits.max(axis=1)
    lse = m + np.log(np.exp(logits - m[:, None]).sum(axis=1))
    valid = t != ignore_index
    n_valid = int(valid.sum())
    rows = np.nonzero(valid)[0]
    nll = lse[rows] - logits[rows, t[rows]]
    loss = nll.sum() / n_valid if n_valid > 0 else np.float64("nan")
    return loss, lse


def backward(grad_out, hidden, weight, target, lse, ignore_index: int = IGNORE_INDEX,
             acc=np.float64):
    """Return ``(dhidden, dweight)`` -- cross_entropy.py:127-131, 937-957."""
    h = hidden.reshape(-1, hidden.shape[-1]).astype(acc)
    w = weight.astype(acc)
    t = np.asarray(target).reshape(-1).astype(np.int64)
    valid = t != ignore_index
    n_valid = int(valid.sum())
    logits = h @ w.T
    g = np.exp(logits - np.asarray(lse, dtype=acc)[:, None])
    rows = np.nonzero(valid)[0]
    g[rows, t[rows]] -= 1.0
    scale = float(grad_out) / n_valid if n_valid > 0 else float("nan")
    g *= scale
    g[~valid] = 0.0
    return (g @ w).reshape(hidden.shape), g.T @ h

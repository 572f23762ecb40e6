"""Fused AdamW step (test infrastructure).

Follows alkinun/helion ``tritium/ops/adamw.py``: moments in fp32
(adamw.py:45-48), decoupled weight decay applied to the pre-update parameter
before the Adam term (adamw.py:50), ``denom = sqrt(v / bc2) + eps`` and
``step_size = lr / bc1`` (adamw.py:51-53) with the bias corrections computed on
the host in float64 (adamw.py:133-134).

Pinned by (tests/test_oracle.py, test_adamw_*): ``torch.optim.AdamW(foreach=False)``
over several steps (tests/tritium/test_adamw.py:19-27 compares against it), and
the step-1 closed form from zero moments
``p1 = p*(1 - lr*wd) - lr * g / (|g| + eps)``.
"""

from __future__ import annotations

import numpy as np

from .numerics import quantize


def bias_corrections(beta1: float, beta2: float, step: int) -> tuple[float, float]:
    """Host-side float64 bias corrections -- adamw.py:133-134."""
    return 1.0 - beta1**step, 1.0 - beta2**step


def step(
    p: np.ndarray,
    g: np.ndarray,
    m: np.ndarray,
    v: np.ndarray,
    *,
    lr: float,
    beta1: float = 0.9,
    beta2: float = 0.999,
    eps: float = 1e-8,
    weight_decay: float = 0.01,
    step: int = 1,
    dtype: str = "f32",
):
    """Return updated ``(p, m, v)``; p rounded to ``dtype`` -- adamw.py:40-54."""
    bc1, bc2 = bias_corrections(beta1, beta2, step)
    f = np.float32
    pf = p.astype(np.float32)
    gf = g.astype(np.float32)
    m = (f(beta1) * m.astype(np.float32) + f(1.0 - beta1) * gf).astype(np.float32)
    v = (f(beta2) * v.astype(np.float32) + f(1.0 - beta2) * gf * gf).astype(np.float32)
    pf = pf - f(lr) * f(weight_decay) * pf
    denom = np.sqrt(v / f(bc2)) + f(eps)
    pf = pf - f(lr / bc1) * m / denom
    return quantize(pf, dtype), m, v

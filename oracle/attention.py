"""Scaled dot-product attention forward and backward (test infrastructure).

Follows alkinun/helion ``tritium/ops/attention.py``:

* forward (attention.py:69-141): per (batch, head) with GQA head mapping
  ``kv_head = head // (n_heads // n_kv_heads)`` (attention.py:73);
  ``scores = (q @ k^T) * scale`` with ``scale = head_dim ** -0.5``
  (attention.py:109, 314); top-left causal mask ``q_pos >= kv_pos``
  (attention.py:112-113); softmax; ``o = P @ v``; ``lse = m + ln(l)``
  (attention.py:139) in natural-log units;
* backward (attention.py:486-494, 600-614): ``P = exp(scores - lse)``,
  ``dP = dO @ v^T``, ``D_i = rowsum(P * dP)``, ``dS = P * (dP - D_i)``,
  ``dV = P^T @ dO``, ``dQ = dS @ k * scale``, ``dK = dS^T @ q * scale``; the
  GQA group's heads are summed into their kv head (the reference's atomics,
  attention.py:499-506, 616-623).

Arithmetic is float64 by default (``acc=np.float64``), the "fp32 reference" the
north-star tolerance (max-abs 2e-2 for bf16) is quoted against; ``acc=np.float32``
gives the reference kernels' own accumulation width.

Pinned by (tests/test_oracle.py, test_attention_*): torch
``F.scaled_dot_product_attention`` with ``repeat_interleave`` for GQA and its
autograd (tests/tritium/test_attention.py:9-21, 100-107), ``T = 1`` gives
``o = v``, causal row 0 gives ``o[0] = v[0]``, uniform v rows give ``o = v``,
``lse >= max score``, a float64 finite-difference gradient check, and the
golden fixtures.
"""

from __future__ import annotations

import numpy as np


def _mask(tq: int, tkv: int, is_causal: bool) -> np.ndarray:
    qp = np.arange(tq)[:, None]
    kp = np.arange(tkv)[None, :]
    return (qp >= kp) if is_causal else np.ones((tq, tkv), dtype=bool)


def forward(q, k, v, is_causal: bool = True, acc=np.float64):
    """Return ``(o, lse)`` for q ``[B,H,Tq,D]``, k/v ``[B,Hkv,Tkv,D]``.

    attention.py:69-141 (decode branch attention.py:174-217 is the same math
    for ``Tq == 1``).
    """
    b, h, tq, d = q.shape
    hkv, tkv = k.shape[1], k.shape[2]
    group = h // hkv
    scale = d ** -0.5
    mask = _mask(tq, tkv, is_causal)
    o = np.zeros((b, h, tq, d), dtype=acc)
    lse = np.zeros((b, h, tq), dtype=acc)
    for bi in range(b):
        for hi in range(h):
            kh = hi // group
            qf = q[bi, hi].astype(acc)
            kf = k[bi, kh].astype(acc)
            vf = v[bi, kh].astype(acc)
            s = (qf @ kf.T) * acc(scale)
            s = np.where(mask, s, -np.inf)
            m = s.max(axis=1, keepdims=True)
            p = np.exp(s - m)
            l = p.sum(axis=1, keepdims=True)
            o[bi, hi] = (p @ vf) / l
            lse[bi, hi] = (m + np.log(l))[:, 0]
    return o, lse


def backward(do, q, k, v, lse, is_causal: bool = True, acc=np.float64):
    """Return ``(dq, dk, dv)`` -- attention.py:486-506 and 600-629."""
    b, h, tq, d = q.shape
    hkv, tkv = k.shape[1], k.shape[2]
    group = h // hkv
    scale = d ** -0.5
    mask = _mask(tq, tkv, is_causal)
    dq = np.zeros((b, h, tq, d), dtype=acc)
    dk = np.zeros((b, hkv, tkv, d), dtype=acc)
    dv = np.zeros((b, hkv, tkv, d), dtype=acc)
    for bi in range(b):
        for hi in range(h):
            kh = hi // group
            qf = q[bi, hi].astype(acc)
            kf = k[bi, kh].astype(acc)
            vf = v[bi, kh].astype(acc)
            dof = do[bi, hi].astype(acc)
            s = (qf @ kf.T) * acc(scale)
            p = np.where(mask, np.exp(s - lse[bi, hi].astype(acc)[:, None]), 0.0)
            dp = dof @ vf.T
            di = (p * dp).sum(axis=1, keepdims=True)
            ds = p * (dp - di)
            dq[bi, hi] = (ds @ kf) * acc(scale)
            dk[bi, kh] += (ds.T @ qf) * acc(scale)
            dv[bi, kh] += p.T @ dof
    return dq, dk, dv

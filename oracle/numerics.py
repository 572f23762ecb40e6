"""Storage-dtype rounding used by every oracle function (test infrastructure).

numpy has no bfloat16, so bf16 values are carried in float32 arrays and rounded
with the IEEE round-to-nearest-even rule on the upper 16 bits, which is what
``tl.store`` of an fp32 value into a bf16 pointer does (and what the HIP
kernels' ``v_cvt_pk_bf16_f32`` does).
"""

from __future__ import annotations

import numpy as np

DTYPES = ("f32", "f16", "bf16")
# "f64" keeps float64 values unrounded: a truth value for finite-difference checks.


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), as float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = rounded.astype(np.uint32).view(np.float32).copy()
    nan = np.isnan(x)
    if nan.any():
        out[nan] = np.float32("nan")
    return out


def quantize(x: np.ndarray, dtype: str) -> np.ndarray:
    """Return float32 ``x`` rounded to the storage dtype ``dtype``."""
    if dtype == "f64":
        return np.array(x, dtype=np.float64)
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        return x.copy()
    if dtype == "f16":
        return x.astype(np.float16).astype(np.float32)
    if dtype == "bf16":
        return bf16_round(x)
    raise ValueError(f"unknown dtype {dtype!r}")


def seeded_normal(seed: int, shape, scale: float = 1.0, mean: float = 0.0) -> np.ndarray:
    """Float32 N(mean, scale^2) samples from a seeded numpy Generator."""
    rng = np.random.default_rng(seed)
    return (mean + scale * rng.standard_normal(shape)).astype(np.float32)

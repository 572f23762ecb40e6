"""Shared helpers for the test-suite (seeded inputs, conversions, tolerances)."""

from __future__ import annotations

import numpy as np
import torch

DTYPES = [torch.float32, torch.float16, torch.bfloat16]
NAME = {torch.float32: "f32", torch.float16: "f16", torch.bfloat16: "bf16"}

# north-star / reference tolerances: fp32 1e-5 relative (AdamW, RMSNorm);
# fp16 2e-2 and bf16 3e-2 (tests/tritium/test_rmsnorm.py:51-62, tests/_utils.py:14-17)
TOL = {torch.float32: (1e-5, 1e-5), torch.float16: (2e-2, 2e-2), torch.bfloat16: (3e-2, 3e-2)}


def randn(shape, dtype=torch.float32, seed=0, device="cuda", scale=1.0, mean=0.0):
    """N(mean, scale^2) drawn on a seeded CPU generator, then cast and moved."""
    g = torch.Generator().manual_seed(seed)
    t = torch.randn(shape, generator=g, dtype=torch.float32) * scale + mean
    return t.to(dtype).to(device)


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_close(actual: torch.Tensor, expected, rtol, atol, msg=""):
    exp = torch.as_tensor(np.asarray(expected, dtype=np.float32))
    torch.testing.assert_close(
        actual.detach().float().cpu(), exp.reshape(actual.shape), rtol=rtol, atol=atol,
        msg=(lambda m: f"{msg}: {m}") if msg else None,
    )

"""``matmul`` / ``matmul_vec`` (vendor GEMM) against a float64 CPU product,
mirroring the reference's tests/tritium/test_matmul.py: its shapes, the
non-contiguous second operand ``weight.T`` that ``helion.Linear`` passes,
autograd, no-grad, and the error contract.  Tolerances are the reference's
(tests/_utils.py:14-17): fp32 1e-5, fp16/bf16 2e-2."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import helion_amd as tritium
from _helpers import DTYPES, np32, randn

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _close(actual, expected64, dtype):
    # the reference rounds the fp32 product to the output dtype before comparing
    exp = torch.from_numpy(np.asarray(expected64, dtype=np.float32)).to(dtype).float()
    tol = TOL[dtype]
    torch.testing.assert_close(actual.detach().float().cpu(), exp, rtol=tol, atol=tol)


def _np64(t):
    return np32(t).astype(np.float64)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("m", "n", "k"), [(16, 16, 16), (64, 64, 64), (128, 256, 32), (33, 17, 9)])
def test_matmul_forward(dtype, m, n, k):
    a, b = randn((m, k), dtype, 1), randn((k, n), dtype, 2)
    _close(tritium.matmul(a, b), _np64(a) @ _np64(b), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_accepts_non_contiguous_second_input(dtype):
    a, weight = randn((64, 64), dtype, 3), randn((48, 64), dtype, 4)
    b = weight.T
    assert not b.is_contiguous()
    _close(tritium.matmul(a, b), _np64(a) @ _np64(b), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("n", "k"), [(16, 16), (96, 64), (1024, 384), (65, 33)])
def test_matmul_vec_forward(dtype, n, k):
    a, b = randn((k,), dtype, 5), randn((k, n), dtype, 6)
    _close(tritium.matmul_vec(a, b), _np64(a) @ _np64(b), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_vec_accepts_non_contiguous_second_input(dtype):
    a, weight = randn((64,), dtype, 7), randn((96, 64), dtype, 8)
    b = weight.T
    assert not b.is_contiguous()
    _close(tritium.matmul_vec(a, b), _np64(a) @ _np64(b), dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("m", "n", "k"), [(64, 64, 64), (128, 32, 17)])
def test_matmul_autograd(dtype, m, n, k):
    a = randn((m, k), dtype, 9).requires_grad_(True)
    b = randn((k, n), dtype, 10).requires_grad_(True)
    g = randn((m, n), dtype, 11)
    tritium.matmul(a, b).backward(g)
    A, B, G = _np64(a), _np64(b), _np64(g)
    _close(a.grad, G @ B.T, dtype)
    _close(b.grad, A.T @ G, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
def test_matmul_vec_autograd(dtype):
    a = randn((64,), dtype, 12).requires_grad_(True)
    b = randn((64, 32), dtype, 13).requires_grad_(True)
    g = randn((32,), dtype, 14)
    tritium.matmul_vec(a, b).backward(g)
    A, B, G = _np64(a), _np64(b), _np64(g)
    _close(a.grad, B @ G, dtype)
    _close(b.grad, np.outer(A, G), dtype)


def test_matmul_needs_input_grad_and_no_grad():
    a = randn((16, 16), torch.float32, 15).requires_grad_(True)
    b = randn((16, 16), torch.float32, 16)
    tritium.matmul(a, b).sum().backward()
    assert a.grad is not None and b.grad is None
    with torch.no_grad():
        assert not tritium.matmul(a, b).requires_grad


def test_matmul_empty_and_zero_k():
    assert tritium.matmul(randn((0, 8), seed=1), randn((8, 5), seed=2)).shape == (0, 5)
    out = tritium.matmul(randn((3, 0), seed=1), randn((0, 5), seed=2))
    assert out.shape == (3, 5) and torch.count_nonzero(out) == 0


def test_matmul_error_contract():
    with pytest.raises(ValueError, match="Shape mismatch"):
        tritium.matmul(randn((4, 8)), randn((4, 8)))
    with pytest.raises(ValueError, match="Dtype mismatch"):
        tritium.matmul(randn((4, 8)), randn((8, 4), torch.float16))
    with pytest.raises(ValueError, match="must be a 2D tensor"):
        tritium.matmul(randn((4,)), randn((4, 8)))
    with pytest.raises(ValueError, match="must be a 1D tensor"):
        tritium.matmul_vec(randn((2, 4)), randn((4, 8)))
    with pytest.raises(ValueError, match="must have one of these dtypes"):
        tritium.matmul(randn((4, 4)).to(torch.int32), randn((4, 4)).to(torch.int32))

"""RMSNorm HIP kernels vs the CPU oracle (parity), mirroring the reference's
tests/tritium/test_rmsnorm.py (dtypes, hidden sizes, row counts, residual,
non-contiguous dy, empty input) at north-star tolerances."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import helion_amd as tritium
import oracle
from _helpers import DTYPES, NAME, TOL, assert_close, np32, randn

pytestmark = pytest.mark.gpu

HIDDEN = [1, 7, 768, 1024, 1536, 4096, 5120, 11008, 16384, 40000]
ROWS = [1, 16, 128, 1030]


def _inputs(n_rows, hidden, dtype, seed=0):
    x = randn((n_rows, hidden), dtype, seed)
    w = randn((hidden,), dtype, seed + 1, scale=0.02, mean=1.0)
    dy = randn((n_rows, hidden), dtype, seed + 2)
    return x, w, dy


def _truth_acc(dtype):
    return np.float64 if dtype == torch.float32 else np.float32


# every (hidden, rows) pair whose CPU oracle run stays within a 4M-element budget
SHAPES = [(h, r) for h in HIDDEN for r in ROWS if h * r <= 4_000_000]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("hidden", "n_rows"), SHAPES)
def test_rmsnorm_forward_backward(dtype, hidden, n_rows):
    x, w, dy = _inputs(n_rows, hidden, dtype)
    xs = x.clone().requires_grad_(True)
    ws = w.clone().requires_grad_(True)
    y = tritium.rmsnorm(xs, ws, 1e-6)
    y.backward(dy)
    acc = _truth_acc(dtype)
    ey, _ = oracle.rmsnorm.forward(np32(x), np32(w), 1e-6, NAME[dtype], acc=acc)
    edx, edw = oracle.rmsnorm.backward(np32(dy), np32(x), np32(w), None, 1e-6, NAME[dtype], acc=acc)
    rtol, atol = TOL[dtype]
    assert_close(y, ey, rtol, atol, "y")
    assert_close(xs.grad, edx, rtol, atol, "dx")
    # dw sums n_rows terms: the reference test widens fp32 to 2e-4 (test_rmsnorm.py:56-58)
    dw_tol = (1e-5, 1e-5) if dtype == torch.float32 else (3e-2, 3e-2)
    if dtype != torch.float32:
        # judged relative to the scale of the sum, as the reference's bf16 tolerances are
        scale = max(1.0, float(np.abs(edw).max()))
        dw_tol = (3e-2, 3e-2 * scale)
    assert_close(ws.grad, edw, *dw_tol, msg="dw")


@pytest.mark.parametrize("dtype", DTYPES)
def test_rmsnorm_backward_standalone_recomputes_rstd(dtype):
    x, w, dy = _inputs(64, 4096, dtype, seed=5)
    dx, dw = tritium.rmsnorm_backward(dy, x, w, 1e-6)
    acc = _truth_acc(dtype)
    edx, edw = oracle.rmsnorm.backward(np32(dy), np32(x), np32(w), None, 1e-6, NAME[dtype], acc=acc)
    rtol, atol = TOL[dtype]
    assert_close(dx, edx, rtol, atol, "dx")
    scale = max(1.0, float(np.abs(edw).max()))
    assert_close(dw, edw, rtol, atol * (1 if dtype == torch.float32 else scale), "dw")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("hidden", [768, 4096, 333])
def test_residual_rmsnorm(dtype, hidden):
    n = 96
    x, w, dy = _inputs(n, hidden, dtype, seed=11)
    r = randn((n, hidden), dtype, 21)
    dz_out = randn((n, hidden), dtype, 22)
    xs, rs, ws = (t.clone().requires_grad_(True) for t in (x, r, w))
    y, z = tritium.residual_rmsnorm(xs, rs, ws, 1e-6)
    torch.autograd.backward((y, z), (dy, dz_out))
    acc = _truth_acc(dtype)
    ey, ez, rstd = oracle.rmsnorm.residual_forward(np32(x), np32(r), np32(w), 1e-6, NAME[dtype], acc=acc)
    edz, edw = oracle.rmsnorm.residual_backward(np32(dy), np32(dz_out), ez, np32(w), rstd,
                                                NAME[dtype], acc=acc)
    rtol, atol = TOL[dtype]
    assert_close(y, ey, rtol, atol, "y")
    assert_close(z, ez, rtol, atol, "z")
    # the kernel adds dresidual in fp32 and rounds once; the reference rounds twice
    assert_close(xs.grad, edz, rtol, atol * (1 if dtype == torch.float32 else 2), "dx")
    torch.testing.assert_close(xs.grad, rs.grad, rtol=0, atol=0)
    scale = max(1.0, float(np.abs(edw).max()))
    assert_close(ws.grad, edw, rtol, atol * (1 if dtype == torch.float32 else scale), "dw")


def test_rmsnorm_noncontiguous_dy_and_3d():
    x, w, _ = _inputs(2 * 8 * 4, 256, torch.float32, seed=3)
    x = x.view(2, 32, 256).requires_grad_(True)
    dy = randn((2, 256, 32), torch.float32, 4).transpose(1, 2)
    assert not dy.is_contiguous()
    y = tritium.rmsnorm(x, w, 1e-6)
    y.backward(dy)
    edx, _ = oracle.rmsnorm.backward(np32(dy), np32(x), np32(w), None, 1e-6, "f32", acc=np.float64)
    assert_close(x.grad, edx, 1e-5, 1e-5)


def test_rmsnorm_empty_rows():
    x = torch.empty((0, 64), device="cuda")
    w = torch.ones(64, device="cuda", requires_grad=True)
    y = tritium.rmsnorm(x, w)
    assert y.shape == (0, 64)
    dx, dw = tritium.rmsnorm_backward(torch.empty_like(x), x, w.detach())
    assert dx.shape == (0, 64) and torch.count_nonzero(dw) == 0


def test_rmsnorm_config1_shape():
    # BASELINE config 1 at its own shape: x [4096, 768] fp32, w = 1 + N(0, 0.02), eps 1e-6
    x, w, dy = _inputs(4096, 768, torch.float32, seed=0)
    xs = x.clone().requires_grad_(True)
    ws = w.clone().requires_grad_(True)
    y = tritium.rmsnorm(xs, ws, 1e-6)
    y.backward(dy)
    ey, _ = oracle.rmsnorm.forward(np32(x), np32(w), 1e-6, "f32", acc=np.float64)
    edx, edw = oracle.rmsnorm.backward(np32(dy), np32(x), np32(w), None, 1e-6, "f32", acc=np.float64)
    assert_close(y, ey, 1e-5, 1e-5, "y")
    assert_close(xs.grad, edx, 1e-5, 1e-5, "dx")
    assert_close(ws.grad, edw, 1e-5, 1e-5, "dw")


def test_rmsnorm_deterministic():
    x, w, dy = _inputs(4096, 4096, torch.bfloat16, seed=9)
    r1 = tritium.rmsnorm_backward(dy, x, w)
    r2 = tritium.rmsnorm_backward(dy, x, w)
    assert torch.equal(r1[0], r2[0]) and torch.equal(r1[1], r2[1])

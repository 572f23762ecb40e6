"""GPU parity of the public ops off the hot path.

``cross_entropy``/``cross_entropy_backward`` run this library's HIP kernels:
checked against float64 CPU logsumexp / softmax of the same logits (the
formula of tests/tritium/test_cross_entropy.py:15-60, F.cross_entropy on fp32
logits) at vocabularies on both sides of the one-wavefront / one-block split,
with vector and element-wise row paths, int32 and int64 targets, plus the
known answer for zero logits (loss = ln V, dlogits = (1/V - onehot)/N).

The torch-implemented ops (add, relu, add_relu, gelu, add_gelu, dropout,
sgd_step, softmax, layernorm) mirror the reference's own tests
(tests/tritium/test_{add,relu,add_relu,gelu,dropout,sgd,softmax,layernorm}.py)
with its tolerances (tests/_utils.py:14-17: fp32 1e-5, fp16/bf16 2e-2).
"""

from __future__ import annotations

import importlib
import math

import pytest
import torch
import torch.nn.functional as F

import helion_amd as tritium
from _helpers import DTYPES, randn

pytestmark = pytest.mark.gpu

ce_mod = importlib.import_module("helion_amd.cross_entropy")

REF_TOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _close(actual, expected, dtype=None, tol=None):
    t = tol if tol is not None else REF_TOL[dtype or actual.dtype]
    torch.testing.assert_close(actual.detach().float().cpu(), expected.detach().float().cpu(),
                               rtol=t, atol=t)


# ------------------------------------------------------------- cross_entropy
CE_SHAPES = [(1, 10), (7, 100), (64, 1000), (33, 8191), (16, 8192), (8, 50304), (3, 131072),
             (5, 12345), (300, 257), (128, 1024), (16, 512), (1, 8),
             # dispatch edges of the forward: rows of >= 8192 elements are cut into spans
             # (a (max, sum) pair per span, merged in span order) when there are fewer rows
             # than two workgroups per compute unit (512 on a 256-CU part), otherwise a
             # 256-lane block per row; shorter rows get one wavefront each
             (511, 8192), (512, 8192), (513, 8192), (511, 8191), (2, 16384), (2, 16376)]


def _targets(n, v, seed, dtype=torch.int64):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, v, (n,), generator=g).to(dtype).cuda()


def _ce_ref(logits, target):
    x = logits.detach().double().cpu()
    t = target.long().cpu()
    lse = torch.logsumexp(x, dim=-1)
    nll = lse - x.gather(1, t[:, None])[:, 0]
    return nll.mean(), lse, torch.softmax(x, dim=-1)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("n", "v"), CE_SHAPES)
def test_cross_entropy_forward_backward(dtype, n, v):
    print(f"[ce] {dtype} n={n} v={v}", flush=True)
    logits = randn((n, v), dtype, seed=n + v, scale=2.0)
    target = _targets(n, v, seed=v, dtype=torch.int32 if v % 2 else torch.int64)
    loss = tritium.cross_entropy(logits, target)
    ref_loss, ref_lse, ref_p = _ce_ref(logits, target)
    assert loss.dtype == torch.float32 and loss.shape == ()
    _close(loss, ref_loss, tol=1e-5)
    _, lse = ce_mod._cross_entropy_forward(logits, target)
    _close(lse, ref_lse, tol=1e-5)
    g = torch.tensor(0.75, device="cuda")
    dl = tritium.cross_entropy_backward(g, logits, target, lse)
    onehot = F.one_hot(target.long().cpu(), v).double()
    expected = ((ref_p - onehot) * (0.75 / n)).to(dtype)
    assert dl.dtype == dtype and dl.shape == logits.shape
    _close(dl, expected, dtype, tol=1e-5 if dtype == torch.float32 else 1e-2 / n)


@pytest.mark.parametrize("dtype", DTYPES)
def test_cross_entropy_autograd_matches_torch(dtype):
    # tests/tritium/test_cross_entropy.py:43-60
    logits = randn((24, 3000), dtype, seed=3).requires_grad_(True)
    target = _targets(24, 3000, seed=4)
    tritium.cross_entropy(logits, target).backward()
    ref = logits.detach().float().cpu().requires_grad_(True)
    F.cross_entropy(ref, target.cpu()).backward()
    _close(logits.grad, ref.grad, dtype)


def test_cross_entropy_zero_logits_known_answer():
    n, v = 6, 5000
    logits = torch.zeros((n, v), device="cuda", dtype=torch.bfloat16)
    target = _targets(n, v, seed=9)
    loss, lse = ce_mod._cross_entropy_forward(logits, target)
    assert abs(float(loss) - math.log(v)) < 1e-5
    dl = tritium.cross_entropy_backward(torch.tensor(1.0, device="cuda"), logits, target, lse).float().cpu()
    exp = torch.full((n, v), 1.0 / v / n)
    exp[torch.arange(n), target.cpu()] -= 1.0 / n
    torch.testing.assert_close(dl, exp.to(torch.bfloat16).float(), rtol=0, atol=0)


def test_cross_entropy_edge_cases():
    # no rows: zero loss (cross_entropy.py:540-544); an out-of-range target gives NaN
    empty = torch.empty((0, 7), device="cuda")
    assert float(tritium.cross_entropy(empty, torch.empty(0, dtype=torch.long, device="cuda"))) == 0.0
    logits = randn((2, 16), seed=1)
    bad = torch.tensor([3, 16], device="cuda")
    assert math.isnan(float(tritium.cross_entropy(logits, bad)))
    assert not tritium.cross_entropy(logits, torch.tensor([3, 15], device="cuda")).isnan()


def test_cross_entropy_forward_rejects_small_workspace():
    # The C entry takes the workspace size and refuses a buffer smaller than
    # tritium_cross_entropy_fwd_workspace_size before launching anything.
    lib = importlib.import_module("helion_amd._lib")
    n, v = 16, 32768  # few long rows: one (max, sum) pair per span
    logits = randn((n, v), torch.bfloat16, seed=5)
    target = _targets(n, v, seed=6)
    code = lib.dtype_code(logits.dtype)
    need = lib.lib().tritium_cross_entropy_fwd_workspace_size(n, v, code)
    assert need > n * 4
    loss = torch.empty((), device="cuda")
    lse = torch.empty((n,), device="cuda")
    work = torch.empty((need // 4 + 1,), device="cuda")
    with pytest.raises(RuntimeError, match="workspace"):
        lib.call("tritium_cross_entropy_fwd_ws", logits.data_ptr(), target.data_ptr(), 2,
                 loss.data_ptr(), lse.data_ptr(), work.data_ptr(), n * 4, n, v, code,
                 lib.stream_of(logits))
    lib.call("tritium_cross_entropy_fwd_ws", logits.data_ptr(), target.data_ptr(), 2,
             loss.data_ptr(), lse.data_ptr(), work.data_ptr(), need, n, v, code,
             lib.stream_of(logits))
    ref_loss, ref_lse, _ = _ce_ref(logits, target)
    _close(loss, ref_loss, tol=1e-5)
    _close(lse, ref_lse, tol=1e-5)


def test_cross_entropy_no_autograd_when_not_needed():
    logits = randn((4, 10), seed=2).requires_grad_(True)
    with torch.no_grad():
        assert not tritium.cross_entropy(logits, _targets(4, 10, 1)).requires_grad


# --------------------------------------------------------------- elementwise
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 16, 1024, 4096])
def test_add_relu_family_forward(dtype, n):
    x, y = randn(n, dtype, seed=n), randn(n, dtype, seed=n + 1)
    _close(tritium.add(x, y), x + y)
    _close(tritium.relu(x), torch.relu(x))
    _close(tritium.add_relu(x, y), torch.relu(x + y))


@pytest.mark.parametrize("dtype", DTYPES)
def test_add_relu_family_autograd(dtype):
    x = randn(1024, dtype, seed=1).requires_grad_(True)
    y = randn(1024, dtype, seed=2).requires_grad_(True)
    tritium.add(x, y).backward(torch.ones_like(x))
    _close(x.grad, torch.ones_like(x))
    _close(y.grad, torch.ones_like(y))
    x.grad = y.grad = None
    dy = randn(1024, dtype, seed=3)
    tritium.add_relu(x, y).backward(dy)
    mask = (x + y).detach() > 0
    _close(x.grad, torch.where(mask, dy, torch.zeros_like(dy)))
    _close(y.grad, torch.where(mask, dy, torch.zeros_like(dy)))
    x.grad = None
    tritium.relu(x).backward(dy)
    _close(x.grad, torch.where(x.detach() > 0, dy, torch.zeros_like(dy)))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 16, 1024, 8192])
def test_gelu_forward_and_backward(dtype, n):
    # tests/tritium/test_gelu.py:9-50
    x, y, dy = randn(n, dtype, seed=n), randn(n, dtype, seed=n + 1), randn(n, dtype, seed=n + 2)
    _close(tritium.gelu(x), F.gelu(x.float(), approximate="tanh").to(dtype))
    _close(tritium.add_gelu(x, y), F.gelu(x.float() + y.float(), approximate="tanh").to(dtype))
    xr = x.float().clone().requires_grad_(True)  # a copy: .float() of fp32 is x itself
    F.gelu(xr, approximate="tanh").backward(dy.float())
    _close(tritium.gelu_backward(dy, x), xr.grad.to(dtype))
    xa = x.clone().requires_grad_(True)
    ya = y.clone().requires_grad_(True)
    tritium.add_gelu(xa, ya).backward(dy)
    zr = (x.float() + y.float()).requires_grad_(True)
    F.gelu(zr, approximate="tanh").backward(dy.float())
    _close(xa.grad, zr.grad.to(dtype))
    _close(ya.grad, zr.grad.to(dtype))


@pytest.mark.parametrize("dtype", DTYPES)
def test_sgd_step(dtype):
    # tests/tritium/test_sgd.py:9-36
    param, grad = randn(4096, dtype, seed=1), randn(4096, dtype, seed=2)
    ref = (param.float() - 1e-2 * (grad.float() + 0.1 * param.float())).to(dtype)
    tritium.sgd_step(param, grad, 1e-2, weight_decay=0.1)
    _close(param, ref)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_dropout_contract(dtype, p):
    # tests/tritium/test_dropout.py:19-98
    x, dy = randn(8192, dtype, seed=5), randn(8192, dtype, seed=6)
    out = tritium.dropout(x, p, seed=7)
    kept = out != 0
    scale = 1.0 / (1.0 - p)
    _close(out[kept], (x[kept].float() * scale).to(dtype))
    assert abs(float(kept.float().mean()) - (1 - p)) < 0.02 + 0.05 * (1 - p)
    dx = tritium.dropout_backward(dy, p, 7)
    _close(dx, torch.where(kept, dy.float() * scale, torch.zeros(())).to(dtype))
    xa = x.clone().requires_grad_(True)
    tritium.dropout(xa, p, seed=7).backward(dy)
    _close(xa.grad, dx)


def test_dropout_seeds_and_layout():
    x = randn(8192, seed=1)
    assert torch.equal(tritium.dropout(x, 0.3, seed=123), tritium.dropout(x, 0.3, seed=123))
    assert not torch.equal(tritium.dropout(x, 0.5, seed=1), tritium.dropout(x, 0.5, seed=2))
    torch.manual_seed(0)
    a = tritium.dropout(x, 0.5)
    torch.manual_seed(0)
    assert torch.equal(a, tritium.dropout(x, 0.5))
    xt = randn((1024, 16), seed=2).T
    out = tritium.dropout(xt, 0.5, seed=4)
    assert out.shape == xt.shape and out.is_contiguous()
    kept = out != 0
    _close(out[kept], xt.contiguous()[kept] * 2.0)
    assert tritium.dropout(torch.empty(0, device="cuda"), 0.5, seed=0).shape == (0,)


# ------------------------------------------------------------ softmax / norm
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("rows", "hidden"), [(1, 7), (64, 1000), (8, 4096), (3, 65536)])
def test_softmax_forward_backward(dtype, rows, hidden):
    # tests/tritium/test_softmax.py:41-90
    x, dy = randn((rows, hidden), dtype, seed=1, scale=3.0), randn((rows, hidden), dtype, seed=2)
    out = tritium.softmax(x)
    ref = torch.softmax(x.double(), dim=-1)
    _close(out, ref.to(dtype), dtype)
    o64 = out.double()
    dx_ref = o64 * (dy.double() - (dy.double() * o64).sum(-1, keepdim=True))
    _close(tritium.softmax_backward(dy, out), dx_ref.to(dtype), dtype)
    xa = x.clone().requires_grad_(True)
    tritium.softmax(xa).backward(dy.t().contiguous().t())  # non-contiguous upstream grad
    _close(xa.grad, dx_ref.to(dtype), dtype)


def test_softmax_large_values_are_stable():
    x = torch.tensor([[1000.0, 1001.0, 1002.0]], device="cuda")
    _close(tritium.softmax(x), torch.softmax(x, -1))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("rows", "hidden"), [(1, 64), (37, 768), (16, 4096)])
def test_layernorm_forward_backward(dtype, rows, hidden):
    # tests/tritium/test_layernorm.py:77-140
    x = randn((rows, hidden), dtype, seed=1)
    w = randn(hidden, dtype, seed=2, scale=0.1, mean=1.0)
    b = randn(hidden, dtype, seed=3, scale=0.1)
    dy = randn((rows, hidden), dtype, seed=4)
    xr, wr, br = (t.double().cpu().requires_grad_(True) for t in (x, w, b))
    ref = F.layer_norm(xr, (hidden,), wr, br, eps=1e-5)
    ref.backward(dy.double().cpu())
    _close(tritium.layernorm(x, w, b), ref.to(dtype), dtype)
    dx, dw, db = tritium.layernorm_backward(dy, x, w)
    _close(dx, xr.grad.to(dtype), dtype)
    tol = REF_TOL[dtype] * max(1.0, rows / 16)
    _close(dw, wr.grad.to(dtype), tol=tol)
    _close(db, br.grad.to(dtype), tol=tol)
    xa, wa, ba = (t.clone().requires_grad_(True) for t in (x, w, b))
    tritium.layernorm(xa, wa, ba).backward(dy)
    _close(xa.grad, xr.grad.to(dtype), dtype)
    _close(wa.grad, wr.grad.to(dtype), tol=tol)


def test_layernorm_only_needs_dx():
    # tests/tritium/test_layernorm.py:243-257
    x = randn((8, 256), seed=1).requires_grad_(True)
    w, b = randn(256, seed=2), randn(256, seed=3)
    tritium.layernorm(x, w, b).sum().backward()
    assert x.grad is not None and w.grad is None and b.grad is None


@pytest.mark.parametrize(("n", "v"), [(128, 1024), (3, 131072), (700, 8192)])
def test_cross_entropy_forward_repeated_calls(n, v):
    # calls of different sizes in a row (per-row and row-span paths, the span
    # count changing with the row count) each match the float64 reference, and a
    # repeated call is bitwise identical (fixed-order merges and mean)
    shapes = [(n, v), (max(1, n // 2), v), (n, v)]
    for i, (nn, vv) in enumerate(shapes):
        logits = randn((nn, vv), torch.bfloat16, seed=i + nn, scale=2.0)
        target = _targets(nn, vv, seed=i)
        loss, lse = ce_mod._cross_entropy_forward(logits, target)
        ref_loss, ref_lse, _ = _ce_ref(logits, target)
        _close(loss, ref_loss, tol=1e-5)
        _close(lse, ref_lse, tol=1e-5)
        loss2, _ = ce_mod._cross_entropy_forward(logits, target)
        assert torch.equal(loss, loss2)

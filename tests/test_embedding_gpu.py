"""Embedding backward with a tied head (tritium_embedding_bwd) against the float64
oracle (oracle.embedding.backward, pinned to torch's F.embedding autograd):
dw_out = dw_in + scatter_add(ids, dx), fp32 sums rounded once.  Covers int32 and
int64 ids, dims below, at and past one 1024-column chunk (12, 300, 768, 1000,
1100), repeated and very frequent ids (140 repeats of one id),
out-of-range ids, in-place and out-of-place, strided dx rows, empty input, and
bitwise determinism.  Tolerance: fp32 1e-5 relative; 16-bit one rounding of the
exact sum (half an ulp, plus the fp32 sum's own error)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from _helpers import NAME, np32, randn
from helion_amd.embedding import embedding_backward

pytestmark = pytest.mark.gpu


def _check(got, want, dtype):
    got = np32(got).astype(np.float64)
    want = np.asarray(want, dtype=np.float64)
    if dtype == torch.float32:
        tol = 1e-5 * (1 + np.abs(want))
    else:
        ulp = 2.0 ** (-8 if dtype == torch.bfloat16 else -11)
        tol = ulp * np.abs(want) + 1e-6
    bad = np.abs(got - want) > tol
    assert not bad.any(), f"{bad.sum()} entries off, max err {np.abs(got - want).max():.3e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim", [12, 300, 768, 1000, 1100])
@pytest.mark.parametrize("id_dtype", [torch.int32, torch.int64])
def test_embedding_backward_against_oracle(dtype, dim, id_dtype):
    print(f"[embedding bwd] {dtype} dim={dim} ids={id_dtype}", flush=True)
    vocab, n = 1001, 700
    g = torch.Generator().manual_seed(dim)
    ids = torch.randint(0, vocab, (n,), generator=g)
    ids[::5] = 17  # a frequent id: 140 repeats in one row
    ids = ids.to(id_dtype).cuda()
    dx = randn((n, dim), dtype, seed=1)
    dw = randn((vocab, dim), dtype, seed=2)
    out = embedding_backward(ids, dx, dw)
    want = oracle.embedding.backward(np32(ids).astype(np.int64), np32(dx), np32(dw),
                                     NAME[dtype])
    _check(out, want, dtype)
    # in place gives the same values, and only touched rows change
    dw2 = dw.clone()
    embedding_backward(ids, dx, dw2, out=dw2)
    assert torch.equal(dw2, out)


def test_embedding_backward_strided_rows_and_out_of_range_ids():
    vocab, dim, n = 300, 64, 130
    base = randn((n, dim + 24), torch.bfloat16, seed=3)
    dx = base[:, 8:8 + dim]  # row stride dim + 24
    ids = torch.randint(-5, vocab + 5, (n,), generator=torch.Generator().manual_seed(4)).cuda()
    dw = randn((vocab, dim), torch.bfloat16, seed=5)
    out = embedding_backward(ids, dx, dw)
    want = oracle.embedding.backward(np32(ids).astype(np.int64), np32(dx), np32(dw), "bf16")
    _check(out, want, torch.bfloat16)


def test_embedding_backward_deterministic_and_empty():
    vocab, dim, n = 2000, 768, 16384
    ids = torch.randint(0, vocab, (n,), generator=torch.Generator().manual_seed(6)).cuda()
    dx = randn((n, dim), torch.bfloat16, seed=7)
    dw = randn((vocab, dim), torch.bfloat16, seed=8)
    a = embedding_backward(ids, dx, dw)
    b = embedding_backward(ids, dx, dw)
    assert torch.equal(a, b)
    empty = embedding_backward(ids[:0], dx[:0], dw)
    assert torch.equal(empty, dw)


def test_embedding_backward_matches_torch_autograd_for_a_tied_weight():
    # the harness's use: gather forward, tied head gradient added in the backward
    vocab, dim, b, s = 500, 96, 4, 64
    g = torch.Generator().manual_seed(9)
    w = (torch.randn((vocab, dim), generator=g) * 0.02).cuda()
    tok = torch.randint(0, vocab, (b, s), generator=g).cuda()
    dx = torch.randn((b, s, dim), generator=g).cuda()
    dhead = torch.randn((vocab, dim), generator=g).cuda()
    ws = w.clone().requires_grad_(True)
    ((torch.nn.functional.embedding(tok, ws) * dx).sum() + (ws * dhead).sum()).backward()
    got = embedding_backward(tok.reshape(-1), dx.reshape(-1, dim), dhead.clone())
    torch.testing.assert_close(got, ws.grad, rtol=1e-5, atol=1e-5)

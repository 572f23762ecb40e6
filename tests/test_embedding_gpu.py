"""Embedding backward with a tied head (tritium_embedding_bwd) against the float64
oracle (oracle.embedding.backward, pinned to torch's F.embedding autograd):
dw_out = dw_in + scatter_add(ids, dx), fp32 sums rounded once.  Covers int32 and
int64 ids, dims below, at and past one 1024-column chunk (12, 300, 768, 1000,
1100), repeated and very frequent ids (140 repeats of one id; one id on half
of 6000 tokens; one id on every token), runs crossing the bucketed list's
16-position windows,
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


def _check(got, want, dtype, sum_bound=None):
    """sum_bound: per-entry bound on the fp32 summation error of a row with many
    tokens (added to the tolerance), see _sum_bound."""
    got = np32(got).astype(np.float64)
    want = np.asarray(want, dtype=np.float64)
    if dtype == torch.float32:
        tol = 1e-5 * (1 + np.abs(want))
    else:
        ulp = 2.0 ** (-8 if dtype == torch.bfloat16 else -11)
        tol = ulp * np.abs(want) + 1e-6
    if sum_bound is not None:
        tol = tol + sum_bound
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


def _sum_bound(ids, dx, vocab):
    """4 sqrt(n_v) u sum_i |dx_i| per entry of row v, u = 2^-24: the usual
    statistical bound on the rounding error of an fp32 sum of n_v terms (a row
    named by thousands of tokens can lose more than the 1e-5 relative of a
    short sum where its terms cancel; a dropped or doubled token would still
    be off by about one |dx| entry, far above this)."""
    ids = np32(ids).astype(np.int64)
    a = np.abs(np32(dx).astype(np.float64))
    cnt = np.bincount(ids, minlength=vocab).astype(np.float64)
    s = np.zeros((vocab, a.shape[1]))
    np.add.at(s, ids, a)
    return 4.0 * np.sqrt(cnt)[:, None] * 2.0 ** -24 * s


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("dim", [64, 768, 1100])
def test_embedding_backward_skewed_ids(dtype, dim):
    # one id on half of the tokens (padding or end of text in real batches), a
    # second one on a quarter, runs that cross the 16-position windows of the
    # bucketed list at every offset, and runs of length 15-17 around one window
    print(f"[embedding skewed] {dtype} dim={dim}", flush=True)
    vocab, n = 5000, 6000
    g = torch.Generator().manual_seed(dim + 11)
    ids = torch.randint(0, vocab, (n,), generator=g)
    ids[torch.randperm(n, generator=g)[: n // 2]] = 3
    ids[torch.randperm(n, generator=g)[: n // 4]] = vocab - 1
    ids[:15] = 100
    ids[15:31] = 101
    ids[31:48] = 102
    ids = ids.cuda()
    dx = randn((n, dim), dtype, seed=12)
    dw = randn((vocab, dim), dtype, seed=13)
    out = embedding_backward(ids, dx, dw)
    want = oracle.embedding.backward(np32(ids).astype(np.int64), np32(dx), np32(dw),
                                     NAME[dtype])
    _check(out, want, dtype, _sum_bound(ids, dx, vocab))
    assert torch.equal(out, embedding_backward(ids, dx, dw))  # bitwise deterministic


def test_embedding_backward_one_id_everywhere():
    # every token names the same row: one run across every window of the list
    vocab, dim, n = 7, 256, 4099
    ids = torch.full((n,), 5, dtype=torch.int64).cuda()
    dx = randn((n, dim), torch.float32, seed=14)
    dw = randn((vocab, dim), torch.float32, seed=15)
    out = embedding_backward(ids, dx, dw)
    want = oracle.embedding.backward(np32(ids).astype(np.int64), np32(dx), np32(dw), "f32")
    _check(out, want, torch.float32, _sum_bound(ids, dx, vocab))
    assert torch.equal(out[:5], dw[:5]) and torch.equal(out[6:], dw[6:])


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

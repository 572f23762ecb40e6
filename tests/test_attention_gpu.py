"""Attention HIP kernels (MFMA bf16/fp16, SIMT fp32) vs the float64 oracle,
mirroring the reference's tests/tritium/test_attention.py (head dims, GQA,
non-causal, KV-cache decode, autograd) plus the module's strided layout, ragged
lengths, q_len != kv_len and head_dim 128.  Tolerance: bf16/fp16 max-abs 2e-2
(+2e-2 relative, as tests/_utils.py:14-17), fp32 1e-5."""

from __future__ import annotations

import importlib
import numpy as np
import pytest
import torch

import helion_amd as tritium
import oracle
from _helpers import DTYPES, assert_close, np32, randn

pytestmark = pytest.mark.gpu

ATOL = {torch.float32: 1e-5, torch.float16: 2e-2, torch.bfloat16: 2e-2}


def _check(dtype, b, h, hkv, tq, tkv, d, causal, seed=0, grads=True, layout="bhtd"):
    def make(n, t, s):
        if layout == "bthd":  # what helion.Attention passes: view(b, s, n, d).transpose(1, 2)
            return randn((b, t, n, d), dtype, s).transpose(1, 2)
        return randn((b, n, t, d), dtype, s)

    q, k, v = make(h, tq, seed), make(hkv, tkv, seed + 1), make(hkv, tkv, seed + 2)
    do = randn((b, h, tq, d), dtype, seed + 3)
    qs, ks, vs = (t.detach().requires_grad_(grads) for t in (q, k, v))
    o = tritium.attention(qs, ks, vs, is_causal=causal)
    eo, lse = oracle.attention.forward(np32(q), np32(k), np32(v), causal)
    tol = ATOL[dtype]
    assert_close(o, eo, tol, tol, "o")
    if not grads:
        return
    o.backward(do)
    edq, edk, edv = oracle.attention.backward(np32(do), np32(q), np32(k), np32(v), lse, causal)
    assert_close(qs.grad, edq, tol, tol, "dq")
    assert_close(ks.grad, edk, tol, tol, "dk")
    assert_close(vs.grad, edv, tol, tol, "dv")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [16, 32, 64, 128])
@pytest.mark.parametrize(("batch", "n_heads", "seq"), [(1, 4, 64), (2, 8, 128)])
def test_attention_forward_backward(dtype, head_dim, batch, n_heads, seq):
    _check(dtype, batch, n_heads, n_heads, seq, seq, head_dim, True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("causal", [True, False])
def test_attention_head_dim_256(dtype, causal):
    # the MFMA path at head_dim 256 (forward kernel with one wavefront per SIMD,
    # dQ kernel, dV and dK as two passes): several tiles, GQA, ragged lengths
    _check(dtype, 2, 4, 4, 192, 192, 256, causal, seed=21)
    _check(dtype, 1, 4, 2, 77, 130, 256, causal, seed=22)
    _check(dtype, 1, 2, 2, 130, 70, 256, causal, seed=23, layout="bthd")


@pytest.mark.parametrize("dtype", DTYPES)
def test_attention_grouped_query(dtype):
    _check(dtype, 2, 8, 2, 128, 128, 64, True, seed=4)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", [False, True])
def test_attention_ragged_and_unequal_lengths(dtype, causal):
    _check(dtype, 1, 2, 2, 77, 77, 64, causal, seed=7)
    _check(dtype, 1, 2, 1, 50, 200, 128, causal, seed=8)
    _check(dtype, 1, 2, 2, 200, 50, 32, causal, seed=9)


@pytest.mark.parametrize("dtype", DTYPES)
def test_attention_non_causal(dtype):
    _check(dtype, 1, 4, 4, 64, 64, 32, False, seed=10)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_attention_module_layout_strided(dtype):
    # the reference's strided-dq bug (attention.py:625-629 vs 645) must not recur
    _check(dtype, 2, 4, 4, 96, 96, 64, True, seed=11, layout="bthd")
    _check(dtype, 2, 4, 2, 130, 130, 128, True, seed=12, layout="bthd")


@pytest.mark.parametrize("dtype", DTYPES)
def test_attention_kv_cache_single_query(dtype):
    b, h, kv_len, d = 2, 4, 64, 32
    cache_k = randn((b, h, 80, d), dtype, 1)
    cache_v = randn((b, h, 80, d), dtype, 2)
    k, v = cache_k[:, :, :kv_len], cache_v[:, :, :kv_len]  # strided cache slices
    q = k[:, :, -1:, :].contiguous()
    o = tritium.attention(q, k, v, is_causal=False)
    eo, _ = oracle.attention.forward(np32(q), np32(k), np32(v), False)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert_close(o, eo, tol, tol)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize(("b", "h", "hkv", "kv_len"),
                         [(1, 4, 4, 1), (2, 8, 4, 7), (1, 6, 2, 300), (2, 16, 4, 5000),
                          (1, 8, 1, 2500), (3, 32, 32, 1030)])
def test_attention_decode_split_kv(dtype, head_dim, b, h, hkv, kv_len):
    # q_len 1 against strided cache slices takes the split-KV decode kernels (groups of 1,
    # 2, 3 (padded to 4), 4 and 8 query heads per kv head); o and lse against the oracle
    print(f"[decode] {dtype} d={head_dim} b={b} h={h} hkv={hkv} L={kv_len}", flush=True)
    cache_k = randn((b, hkv, kv_len + 40, head_dim), dtype, 3)
    cache_v = randn((b, hkv, kv_len + 40, head_dim), dtype, 4)
    k, v = cache_k[:, :, :kv_len], cache_v[:, :, :kv_len]
    q = randn((b, 1, h, head_dim), dtype, 5).transpose(1, 2)  # the module's layout
    o = tritium.attention(q, k, v, is_causal=False)
    eo, e_lse = oracle.attention.forward(np32(q), np32(k), np32(v), False)
    assert_close(o, eo, 2e-2, 2e-2, "o")
    from helion_amd.attention import _attention_forward
    _, lse = _attention_forward(q, k, v, False)
    assert_close(lse, e_lse, 1e-4, 1e-4, "lse")


def test_attention_decode_grads_through_general_backward():
    # the decode forward's (o, lse) feed the general backward kernels
    b, h, hkv, kv_len, d = 2, 8, 2, 333, 128
    q = randn((b, h, 1, d), torch.bfloat16, 7).requires_grad_(True)
    k = randn((b, hkv, kv_len, d), torch.bfloat16, 8).requires_grad_(True)
    v = randn((b, hkv, kv_len, d), torch.bfloat16, 9).requires_grad_(True)
    do = randn((b, h, 1, d), torch.bfloat16, 10)
    tritium.attention(q, k, v, is_causal=False).backward(do)
    eo, lse = oracle.attention.forward(np32(q), np32(k), np32(v), False)
    edq, edk, edv = oracle.attention.backward(np32(do), np32(q), np32(k), np32(v), lse, False)
    assert_close(q.grad, edq, 2e-2, 2e-2, "dq")
    assert_close(k.grad, edk, 2e-2, 2e-2, "dk")
    assert_close(v.grad, edv, 2e-2, 2e-2, "dv")


def test_attention_decode_workspace_cache_is_bounded():
    # one workspace per (device, stream), only the most recent few streams keep theirs;
    # each stream's decode still matches the oracle
    att = importlib.import_module("helion_amd.attention")
    b, h, hkv, kv_len, d = 1, 4, 2, 700, 64
    q = randn((b, h, 1, d), torch.bfloat16, 11)
    k = randn((b, hkv, kv_len, d), torch.bfloat16, 12)
    v = randn((b, hkv, kv_len, d), torch.bfloat16, 13)
    eo, _ = oracle.attention.forward(np32(q), np32(k), np32(v), False)
    streams = [torch.cuda.Stream() for _ in range(att._DECODE_WS_KEEP + 3)]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(st):
            o = tritium.attention(q, k, v, is_causal=False)
        torch.cuda.current_stream().wait_stream(st)
        assert_close(o, eo, 2e-2, 2e-2, "o")
        assert len(att._DECODE_WS) <= att._DECODE_WS_KEEP
    keys = list(att._DECODE_WS)
    assert keys[-1][1] == streams[-1].cuda_stream


def test_attention_large_head_bf16_t1024():
    _check(torch.bfloat16, 1, 2, 2, 1024, 1024, 128, True, seed=13)


@pytest.mark.parametrize("causal", [False, True])
def test_attention_gqa_many_tiles_ragged(causal):
    # several kv and query workgroups per head, GQA group of 4, length not a tile multiple
    _check(torch.bfloat16, 1, 8, 2, 700, 700, 128, causal, seed=14)
    _check(torch.float16, 2, 4, 1, 333, 333, 64, causal, seed=15)


# head_dim 128 backward: dK/dV store dS and dQ is formed from it (the default
# where the workspace fits), or the dQ kernel recomputes S and dP (workspace
# limit 0).  Both against the oracle: ragged tiles, Tq < Tkv and Tq > Tkv
# (the causal mask is top-left), GQA, a single row.
DS_SHAPES = [(1, 2, 2, 77, 77), (1, 2, 1, 50, 200), (1, 2, 1, 200, 50), (2, 4, 2, 333, 333),
             (1, 2, 2, 64, 64), (1, 1, 1, 1, 1), (1, 2, 2, 129, 127), (1, 4, 4, 384, 384)]


@pytest.mark.parametrize("head_dim", [128])
@pytest.mark.parametrize("stored", [True, False])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize(("b", "h", "hkv", "tq", "tkv"), DS_SHAPES)
def test_attention_backward_stored_and_recomputed_ds(monkeypatch, stored, causal, b, h, hkv, tq,
                                                     tkv, head_dim):
    A = importlib.import_module("helion_amd.attention")
    if not stored:
        monkeypatch.setattr(A, "DS_WORKSPACE_MAX_BYTES", 0)
    _check(torch.bfloat16, b, h, hkv, tq, tkv, head_dim, causal, seed=31 + tq + tkv)


@pytest.mark.parametrize("head_dim", [64, 128])
def test_attention_longest_first_order(head_dim):
    # causal grids whose (batch, head) count is a multiple of the 8 XCDs take their
    # tiles longest first across each XCD's slices (at head_dim 128 the dQ-from-dS
    # kernel in groups of four slices: 6 per XCD here, a group of 4 and one of 2);
    # the order must not change the results.  GQA: dK/dV over 24 kv slices.
    _check(torch.bfloat16, 2, 24, 24, 512, 512, head_dim, True, seed=41)
    _check(torch.bfloat16, 2, 24, 12, 512, 512, head_dim, True, seed=42)


def test_attention_persistent_dkdv_pairs():
    # head_dim 128 grids with >= 2 kv tiles per compute unit and (batch, kv head)s in
    # multiples of the 8 XCDs run the persistent dK/dV kernel, which deals the kv-tile
    # pairs (t, n - 1 - t) of each head round-robin: 4 kv tiles per head (2 pairs), then 5
    # (an odd count: the middle tile is a work unit of its own) and GQA over 128 kv heads
    _check(torch.bfloat16, 4, 32, 32, 512, 512, 128, True, seed=51)
    _check(torch.bfloat16, 4, 32, 32, 640, 640, 128, True, seed=52)
    _check(torch.bfloat16, 8, 32, 16, 512, 512, 128, True, seed=53)


def test_attention_stored_ds_deterministic_fp16():
    q = randn((2, 4, 300, 128), torch.float16, 1).requires_grad_(True)
    k = randn((2, 2, 300, 128), torch.float16, 2).requires_grad_(True)
    v = randn((2, 2, 300, 128), torch.float16, 3).requires_grad_(True)
    grads = []
    for _ in range(2):
        q.grad = k.grad = v.grad = None
        tritium.attention(q, k, v).sum().backward()
        grads.append((q.grad.clone(), k.grad.clone(), v.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def test_attention_invariants():
    # T = 1 -> o = v; causal row 0 -> o[0] = v[0]; uniform v rows -> o = v
    q = randn((1, 2, 1, 64), torch.bfloat16, 1)
    k = randn((1, 2, 1, 64), torch.bfloat16, 2)
    v = randn((1, 2, 1, 64), torch.bfloat16, 3)
    assert torch.equal(tritium.attention(q, k, v), v)
    q = randn((1, 2, 130, 64), torch.bfloat16, 4)
    k = randn((1, 2, 130, 64), torch.bfloat16, 5)
    v = randn((1, 2, 1, 64), torch.bfloat16, 6).expand(1, 2, 130, 64).contiguous()
    o = tritium.attention(q, k, v)
    assert_close(o, np32(v), 1e-2, 1e-2)
    v2 = randn((1, 2, 130, 64), torch.bfloat16, 7)
    o2 = tritium.attention(q, k, v2)
    assert torch.equal(o2[:, :, 0], v2[:, :, 0])


def test_attention_deterministic():
    q = randn((1, 4, 256, 64), torch.bfloat16, 1).requires_grad_(True)
    k = randn((1, 4, 256, 64), torch.bfloat16, 2).requires_grad_(True)
    v = randn((1, 4, 256, 64), torch.bfloat16, 3).requires_grad_(True)
    grads = []
    for _ in range(2):
        q.grad = k.grad = v.grad = None
        tritium.attention(q, k, v).sum().backward()
        grads.append((q.grad.clone(), k.grad.clone(), v.grad.clone()))
    for a, b in zip(*grads):
        assert torch.equal(a, b)


def _check_heads(dtype, b, h, hkv, t, d, causal, heads, seed, grads=False):
    """Run the full (b, h, t, d) problem, check the listed (batch, kv head)
    slices -- with every query head of each kv head's group -- against the
    oracle (the problem is independent per (batch, kv head))."""
    group = h // hkv
    q, k, v = randn((b, h, t, d), dtype, seed), randn((b, hkv, t, d), dtype, seed + 1), \
        randn((b, hkv, t, d), dtype, seed + 2)
    do = randn((b, h, t, d), dtype, seed + 3)
    qs, ks, vs = (x.detach().requires_grad_(grads) for x in (q, k, v))
    o = tritium.attention(qs, ks, vs, is_causal=causal)
    if grads:
        o.backward(do)
    tol = ATOL[dtype]
    for bi, kh in heads:
        hq = slice(kh * group, (kh + 1) * group)
        sel = lambda x, hs: np32(x[bi:bi + 1, hs])  # noqa: E731
        eo, lse = oracle.attention.forward(sel(q, hq), sel(k, slice(kh, kh + 1)),
                                           sel(v, slice(kh, kh + 1)), causal)
        assert_close(o[bi:bi + 1, hq], eo, tol, tol, f"o[{bi},{kh}]")
        if grads:
            edq, edk, edv = oracle.attention.backward(
                sel(do, hq), sel(q, hq), sel(k, slice(kh, kh + 1)), sel(v, slice(kh, kh + 1)),
                lse, causal)
            assert_close(qs.grad[bi:bi + 1, hq], edq, tol, tol, f"dq[{bi},{kh}]")
            assert_close(ks.grad[bi:bi + 1, kh:kh + 1], edk, tol, tol, f"dk[{bi},{kh}]")
            assert_close(vs.grad[bi:bi + 1, kh:kh + 1], edv, tol, tol, f"dv[{bi},{kh}]")


# head_dim 128 problems with at least 4 workgroups of (256-row query tile
# pairs) per CU take the 8-wavefront ping-pong forward and dQ kernels; these
# grids (1024 workgroups) reach them on a 256-CU part, with one and with an
# odd number of query tiles, ragged lengths, GQA and the non-causal mask.
def test_attention_pingpong_grid():
    _check_heads(torch.bfloat16, 4, 256, 256, 256, 128, True,
                 [(0, 0), (1, 77), (3, 255)], seed=21, grads=True)
    _check_heads(torch.float16, 2, 256, 64, 731, 128, True, [(0, 0), (1, 63)], seed=22,
                 grads=True)
    _check_heads(torch.bfloat16, 2, 256, 256, 600, 128, False, [(0, 5), (1, 250)], seed=23)

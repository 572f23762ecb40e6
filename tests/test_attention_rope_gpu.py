"""Attention with RoPE applied to q as the kernels load it (attention_rope_q:
tritium_attention_fwd_rope / tritium_attention_bwd_rope) against the
reference's sequence -- rope on q and k, then attention (helion/nn.py:196-220)
-- run two ways: this library's rope kernel followed by its attention (the
forward and dK/dV must match bitwise, since the rotation rounds alike; both
take the stored-dS backward, or both the recomputing one), and
the float64 oracle (oracle.rope, then oracle.attention; dq through the
inverse rotation).  Tolerance as the attention tests: max-abs 2e-2 + 2e-2
relative for 16-bit."""

from __future__ import annotations

import importlib

import numpy as np
import pytest
import torch

import helion_amd as tritium
import oracle
from _helpers import NAME, assert_close, np32, randn
from helion_amd.attention import attention_rope_q
from helion_amd.rope import rope_rows

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _tables(max_pos, d):
    c, s = oracle.rope.make_cos_sin(max_pos, d)
    return torch.from_numpy(c).cuda(), torch.from_numpy(s).cuda()


def _rope_tokens(x, cos, sin, pos, inverse=False):
    """x: [b, n, t, d] as a transposed view of [b, t, n, d] memory -> rotated, same layout."""
    b, n, t, d = x.shape
    rows = x.transpose(1, 2).contiguous().view(b * t, n, d)
    out = torch.empty_like(rows)
    rope_rows(None, rows, cos, sin, pos, None, out, inverse=inverse, in_token_stride=n * d,
              out_token_stride=n * d)
    return out.view(b, t, n, d).transpose(1, 2)


def _inputs(dtype, b, h, hkv, t, d, seed):
    q = randn((b, t, h, d), dtype, seed).transpose(1, 2)
    k = randn((b, t, hkv, d), dtype, seed + 1).transpose(1, 2)
    v = randn((b, t, hkv, d), dtype, seed + 2).transpose(1, 2)
    do = randn((b, t, h, d), dtype, seed + 3).transpose(1, 2)
    return q, k, v, do


def _positions(kind, b, t, max_pos, seed):
    if kind == 0:
        return None, np.tile(np.arange(t), b)
    g = torch.Generator().manual_seed(seed)
    p = torch.randint(0, max_pos, (b * t,), generator=g)
    p = p.to(torch.int32 if kind == 1 else torch.int64)
    return p.cuda(), p.numpy().astype(np.int64)


def _run(dtype, b, h, hkv, t, d, kind, seed=0, oracle_check=True):
    print(f"[attention rope] {dtype} b={b} h={h} hkv={hkv} t={t} d={d} pos_kind={kind}", flush=True)
    max_pos = max(2 * t, 64)
    cos, sin = _tables(max_pos, d)
    pos, pos_np = _positions(kind, b, t, max_pos, seed + 9)
    pos_arg = torch.tile(torch.arange(t), (b,)).cuda() if pos is None else pos
    q, k, v, do = _inputs(dtype, b, h, hkv, t, d, seed)
    k_rot = _rope_tokens(k, cos, sin, pos_arg)
    # fused: q rotated on load
    qs, ks, vs = (x.detach().requires_grad_(True) for x in (q, k_rot, v))
    o = attention_rope_q(qs, ks, vs, cos, sin, pos, is_causal=True)
    o.backward(do)
    # composition: rope kernel, then attention
    q_rot = _rope_tokens(q, cos, sin, pos_arg)
    qc, kc, vc = (x.detach().requires_grad_(True) for x in (q_rot, k_rot, v))
    oc = tritium.attention(qc, kc, vc, is_causal=True)
    oc.backward(do)
    assert torch.equal(o, oc), "forward differs from rope + attention"
    assert torch.equal(ks.grad, kc.grad) and torch.equal(vs.grad, vc.grad), "dk/dv differ"
    # dq: the fused path un-rotates fp32 accumulators and rounds once; the composition
    # rounds dq of the rotated q first, then its rotation (two roundings, each within
    # 2^-8 of the largest element it mixes)
    dq_comp = _rope_tokens(qc.grad, cos, sin, pos_arg, inverse=True).float()
    torch.testing.assert_close(qs.grad.float(), dq_comp, rtol=1.6e-2,
                               atol=float(1e-2 * dq_comp.abs().max()))
    if not oracle_check:
        return
    # float64 oracle: the rope kernel's rotation (rounded to the dtype), then attention
    cs, sn = np32(cos), np32(sin)
    tok = lambda x: np32(x.transpose(1, 2)).reshape(b * t, x.shape[1], d)
    unt = lambda a, n: a.reshape(b, t, n, d).transpose(0, 2, 1, 3)
    eq = unt(oracle.rope.apply(tok(q), cs, sn, position_ids=pos_np, dtype=NAME[dtype]), h)
    ek = np32(k_rot)
    eo, lse = oracle.attention.forward(eq, ek, np32(v), True)
    assert_close(o, eo, TOL, TOL, "o")
    edq_rot, edk, edv = oracle.attention.backward(np32(do), eq, ek, np32(v), lse, True)
    edq = unt(oracle.rope.apply(edq_rot.transpose(0, 2, 1, 3).reshape(b * t, h, d), cs, sn,
                                position_ids=pos_np, inverse=True), h)
    assert_close(qs.grad, edq, TOL, TOL, "dq")
    assert_close(ks.grad, edk, TOL, TOL, "dk")
    assert_close(vs.grad, edv, TOL, TOL, "dv")


@pytest.mark.parametrize("stored", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("pos_kind", [0, 1, 2])
def test_attention_rope_q_matches_rope_then_attention(monkeypatch, dtype, head_dim, pos_kind,
                                                      stored):
    if not stored:  # the recomputing backward (no dS workspace)
        monkeypatch.setattr(importlib.import_module("helion_amd.attention"),
                            "DS_WORKSPACE_MAX_BYTES", 0)
    _run(dtype, 2, 4, 4, 130, head_dim, pos_kind, seed=head_dim + pos_kind)


@pytest.mark.parametrize("stored", [True, False])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_attention_rope_q_grouped_query_ragged(monkeypatch, head_dim, stored):
    if not stored:
        monkeypatch.setattr(importlib.import_module("helion_amd.attention"),
                            "DS_WORKSPACE_MAX_BYTES", 0)
    _run(torch.bfloat16, 1, 8, 2, 77, head_dim, 2, seed=3)


def test_attention_rope_q_pingpong_forward_size():
    # enough query tiles for the 8-wavefront ping-pong forward (attn_fwd_pp); compared with
    # rope + attention only (the float64 oracle would take minutes here)
    _run(torch.bfloat16, 8, 32, 32, 2048, 128, 0, seed=5, oracle_check=False)


def test_attention_rope_q_out_of_range_position_gives_nan_rows():
    b, h, t, d = 1, 2, 64, 64
    cos, sin = _tables(64, d)
    q, k, v, _ = _inputs(torch.bfloat16, b, h, h, t, d, 11)
    pos = torch.arange(t, device="cuda")
    pos[5] = 64  # one past the table
    k_rot = _rope_tokens(k, cos, sin, torch.arange(t, device="cuda"))
    o = attention_rope_q(q, k_rot, v, cos, sin, pos, is_causal=True)
    bad = torch.isnan(o.float()).any(dim=-1)[0, 0]
    assert bad[5] and not bad[:5].any()


def test_attention_rope_q_rejects_what_it_cannot_run():
    q = randn((1, 2, 16, 32), torch.bfloat16, 1)
    cos, sin = _tables(16, 32)
    with pytest.raises(ValueError, match="head_dim 64 or 128"):
        attention_rope_q(q, q, q, cos, sin)
    q = randn((1, 2, 16, 64), torch.float32, 1)
    cos, sin = _tables(16, 64)
    with pytest.raises(ValueError, match="bf16/fp16"):
        attention_rope_q(q, q, q, cos, sin)

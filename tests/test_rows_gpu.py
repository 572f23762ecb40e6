"""RoPE, SwiGLU and AdamW HIP kernels vs the CPU oracle (parity), mirroring the
reference's tests/tritium/test_{rope,swiglu,adamw}.py at north-star tolerances."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import helion_amd as tritium
import oracle
from _helpers import DTYPES, NAME, TOL, assert_close, np32, randn

pytestmark = pytest.mark.gpu


# ------------------------------------------------------------------- RoPE --
def _tables(max_pos, head_dim, dtype=torch.float32):
    c, s = oracle.rope.make_cos_sin(max_pos, head_dim)
    return torch.from_numpy(c).to(dtype).cuda(), torch.from_numpy(s).to(dtype).cuda()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [2, 6, 32, 64, 128])
@pytest.mark.parametrize("layout", ["2d", "3d"])
@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_forward(dtype, head_dim, layout, interleaved):
    n_tokens, n_heads = 37, 3
    shape = (n_tokens, head_dim) if layout == "2d" else (n_tokens, n_heads, head_dim)
    q = randn(shape, dtype, 1)
    k = randn(shape, dtype, 2)
    cos, sin = _tables(64, head_dim)
    qo, ko = tritium.rope(q, k, cos, sin, interleaved=interleaved)
    eq, ek = oracle.rope.forward(np32(q), np32(k), np32(cos), np32(sin),
                                 interleaved=interleaved, dtype=NAME[dtype])
    rtol, atol = TOL[dtype]
    assert_close(qo, eq, rtol, atol, "q")
    assert_close(ko, ek, rtol, atol, "k")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("pos_dtype", [torch.int32, torch.int64])
@pytest.mark.parametrize("table_dtype", [torch.float32, torch.bfloat16])
def test_rope_position_ids_offset_and_backward(dtype, pos_dtype, table_dtype):
    b, s, h, d = 3, 50, 4, 128
    q = randn((b * s, h, d), dtype, 3).requires_grad_(True)
    k = randn((b * s, h, d), dtype, 4).requires_grad_(True)
    cos, sin = _tables(64, d, table_dtype)
    pos = torch.arange(s, device="cuda", dtype=pos_dtype).repeat(b)
    qo, ko = tritium.rope(q, k, cos, sin, position_ids=pos, position_offset=7)
    dqo, dko = randn((b * s, h, d), dtype, 5), randn((b * s, h, d), dtype, 6)
    torch.autograd.backward((qo, ko), (dqo, dko))
    npos = np32(pos).astype(np.int64)
    kw = dict(position_ids=npos, position_offset=7, dtype=NAME[dtype])
    eq, ek = oracle.rope.forward(np32(q), np32(k), np32(cos), np32(sin), **kw)
    edq, edk = oracle.rope.backward(np32(dqo), np32(dko), np32(cos), np32(sin), **kw)
    rtol, atol = TOL[dtype]
    assert_close(qo, eq, rtol, atol, "q")
    assert_close(ko, ek, rtol, atol, "k")
    assert_close(q.grad, edq, rtol, atol, "dq")
    assert_close(k.grad, edk, rtol, atol, "dk")


def test_rope_inplace_matches_out_of_place():
    q = randn((128, 32, 128), torch.bfloat16, 8)
    k = randn((128, 32, 128), torch.bfloat16, 9)
    cos, sin = _tables(128, 128)
    qo, ko = tritium.rope(q, k, cos, sin)
    tritium.rope_(q, k, cos, sin)
    assert torch.equal(q, qo) and torch.equal(k, ko)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("head_dim", [64, 6])
def test_rope_rows_in_fused_qkv_matches_rope(dtype, head_dim):
    # tritium_rope_strided: q, k read in place from [tokens, 3, heads, head_dim] and the
    # inverse rotation written back into it give exactly what rope does on contiguous copies
    from helion_amd.rope import rope_rows
    t, h = 300, 5
    qkv = randn((t, 3, h, head_dim), dtype, 21)
    cos, sin = _tables(512, head_dim)
    pos = torch.randint(0, 512, (t,), generator=torch.Generator().manual_seed(3)).cuda()
    q, k = torch.empty((t, h, head_dim), device="cuda", dtype=dtype), torch.empty((t, h, head_dim), device="cuda", dtype=dtype)
    rope_rows(qkv[:, 0], qkv[:, 1], cos, sin, pos, q, k, inverse=False,
              in_token_stride=3 * h * head_dim, out_token_stride=h * head_dim)
    eq, ek = tritium.rope(qkv[:, 0].contiguous(), qkv[:, 1].contiguous(), cos, sin, position_ids=pos)
    assert torch.equal(q, eq) and torch.equal(k, ek)
    back = torch.full_like(qkv, 7.0)
    rope_rows(q, k, cos, sin, pos, back[:, 0], back[:, 1], inverse=True,
              in_token_stride=h * head_dim, out_token_stride=3 * h * head_dim)
    from helion_amd.rope import _rope_forward
    iq, ik = _rope_forward(q, k, cos, sin, pos, 0, False, True)
    assert torch.equal(back[:, 0], iq) and torch.equal(back[:, 1], ik)
    assert torch.equal(back[:, 2], torch.full_like(back[:, 2], 7.0))  # v rows untouched


def test_fused_qkv_rope_attention_matches_unbind_rope_attention():
    # the training harness's attention block (gpt._QKVRopeAttention: k rotated once out of
    # the fused projection, q rotated by the attention kernels as they load it, v read in
    # place) against unbind + rope on contiguous copies + attention, forward and backward
    from helion_amd.gpt import _QKVRopeAttention
    b, s, h, d = 2, 96, 3, 64
    cos, sin = _tables(128, d)
    pos = torch.arange(s, device="cuda").repeat(b)
    base = randn((b, s, 3, h, d), torch.bfloat16, 5)
    go = randn((b, s, h, d), torch.bfloat16, 10)
    x1 = base.clone().requires_grad_(True)
    o1 = _QKVRopeAttention.apply(x1, cos, sin, pos, pos)
    o1.backward(go)
    # q's positions taken as the row index (no position table) are the same positions
    x3 = base.clone().requires_grad_(True)
    o3 = _QKVRopeAttention.apply(x3, cos, sin, pos, None)
    o3.backward(go)
    assert torch.equal(o1, o3) and torch.equal(x1.grad, x3.grad)
    x2 = base.clone().requires_grad_(True)
    qv, kv, vv = x2.unbind(2)
    q2, k2 = tritium.rope(qv.reshape(b * s, h, d).contiguous(), kv.reshape(b * s, h, d).contiguous(),
                          cos, sin, position_ids=pos)
    o2 = tritium.attention(q2.view(b, s, h, d).transpose(1, 2), k2.view(b, s, h, d).transpose(1, 2),
                           vv.transpose(1, 2), is_causal=True).transpose(1, 2)
    o2.backward(go)
    # the rotation rounds as the rope kernel does: forward, dk and dv are bitwise equal
    assert torch.equal(o1, o2)
    assert torch.equal(x1.grad[:, :, 1], x2.grad[:, :, 1])
    assert torch.equal(x1.grad[:, :, 2], x2.grad[:, :, 2])
    # dq is un-rotated from its fp32 accumulators (one rounding instead of two)
    dq2 = x2.grad[:, :, 0].float()
    torch.testing.assert_close(x1.grad[:, :, 0].float(), dq2, rtol=1.6e-2,
                               atol=float(1e-2 * dq2.abs().max()))


def test_rope_rows_k_alone_matches_rope():
    # q = q_out = None rotates k alone (the attention with rope on q's load needs only k)
    from helion_amd.rope import rope_rows
    t, h, d = 130, 4, 128
    k = randn((t, h, d), torch.bfloat16, 41)
    cos, sin = _tables(256, d)
    pos = torch.randint(0, 256, (t,), generator=torch.Generator().manual_seed(4)).cuda()
    out = torch.empty_like(k)
    rope_rows(None, k, cos, sin, pos, None, out, inverse=False, in_token_stride=h * d,
              out_token_stride=h * d)
    _, ek = tritium.rope(k, k, cos, sin, position_ids=pos)
    assert torch.equal(out, ek)


def test_rope_out_of_range_position_is_nan_not_a_fault():
    q = randn((4, 2, 16), torch.float32, 1)
    cos, sin = _tables(8, 16)
    pos = torch.tensor([0, 1, 100, 3], device="cuda")
    qo, _ = tritium.rope(q, q, cos, sin, position_ids=pos)
    assert torch.isnan(qo[2]).all() and not torch.isnan(qo[[0, 1, 3]]).any()
    with pytest.raises(ValueError, match="positions"):
        tritium.rope(q, q, cos, sin, position_offset=6)


# ----------------------------------------------------------------- SwiGLU --
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("rows", "cols"), [(37, 3072), (5, 4100), (3, 7), (1, 300000)])
def test_swiglu_rows_matches_swiglu(dtype, rows, cols):
    # tritium_swiglu_rows_*: x and gate as the two halves of each row of a fused projection,
    # gradients written back into that layout -- exactly what swiglu does on copies
    from helion_amd.swiglu import swiglu_rows, swiglu_rows_backward
    gu = randn((rows, 2 * cols), dtype, 31)
    dy = randn((rows, cols), dtype, 32)
    out = torch.empty((rows, cols), device="cuda", dtype=dtype)
    swiglu_rows(gu[:, :cols], gu[:, cols:], out)
    x, g = gu[:, :cols].contiguous(), gu[:, cols:].contiguous()
    dgu = torch.full_like(gu, 3.0)
    swiglu_rows_backward(dy, gu[:, :cols], gu[:, cols:], dgu[:, :cols], dgu[:, cols:])
    ex, eg = tritium.swiglu_backward(dy, x, g)
    pairs = [(out, tritium.swiglu(x, g)), (dgu[:, :cols], ex), (dgu[:, cols:], eg)]
    if cols % (16 // x.element_size()) == 0:
        # both sides run the 16-byte-vector path: identical arithmetic
        assert all(torch.equal(a, e) for a, e in pairs)
    else:
        # element-wise rows against the vector path on the copy: same formula, compiled apart
        rtol, atol = TOL[dtype]
        for a, e in pairs:
            assert_close(a, np32(e), rtol, atol)


def test_fused_gate_up_matches_two_projections():
    # the training harness's fused MLP input (gpt._GateUpSwiGLU) against swiglu on two halves
    from helion_amd.gpt import _GateUpSwiGLU
    gu = randn((96, 2 * 512), torch.bfloat16, 33)
    dy = randn((96, 512), torch.bfloat16, 34)
    a = gu.clone().requires_grad_(True)
    _GateUpSwiGLU.apply(a).backward(dy)
    b = gu.clone().requires_grad_(True)
    tritium.swiglu(b[:, :512], b[:, 512:]).backward(dy)
    assert torch.equal(a.grad, b.grad)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 7, 16, 1024, 8193, 1 << 20])
def test_swiglu_forward_backward(dtype, n):
    x = randn((n,), dtype, 1).requires_grad_(True)
    g = randn((n,), dtype, 2).requires_grad_(True)
    dy = randn((n,), dtype, 3)
    out = tritium.swiglu(x, g)
    out.backward(dy)
    eo = oracle.swiglu.forward(np32(x), np32(g), NAME[dtype])
    edx, edg = oracle.swiglu.backward(np32(dy), np32(x), np32(g), NAME[dtype])
    rtol, atol = TOL[dtype]
    assert_close(out, eo, rtol, atol, "out")
    assert_close(x.grad, edx, rtol, atol, "dx")
    assert_close(g.grad, edg, rtol, atol, "dgate")


def test_swiglu_unaligned_views():
    base = randn((4099,), torch.bfloat16, 4)
    x, g = base[1:4097], base[2:4098]
    out = tritium.swiglu(x, g)
    assert_close(out, oracle.swiglu.forward(np32(x), np32(g), "bf16"), 3e-2, 3e-2)
    dx, dg = tritium.swiglu_backward(x, x, g)
    edx, edg = oracle.swiglu.backward(np32(x), np32(x), np32(g), "bf16")
    assert_close(dx, edx, 3e-2, 3e-2)
    assert_close(dg, edg, 3e-2, 3e-2)


# ------------------------------------------------------------------ AdamW --
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("n", [1, 128, 4096, 10007])
def test_adamw_step(dtype, n):
    p = randn((n,), dtype, 1)
    g = randn((n,), dtype, 2)
    m = torch.zeros(n, device="cuda")
    v = torch.zeros(n, device="cuda")
    hp = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    ep, em, ev = np32(p), np32(m), np32(v)
    for step in (1, 2, 3):
        tritium.adamw_step(p, g, m, v, step=step, **hp)
        ep, em, ev = oracle.adamw.step(ep, np32(g), em, ev, step=step, dtype=NAME[dtype], **hp)
    rtol, atol = TOL[dtype]
    assert_close(p, ep, rtol, atol, "param")
    assert_close(m, em, 1e-5, 1e-7, "exp_avg")
    assert_close(v, ev, 1e-5, 1e-9, "exp_avg_sq")


def test_adamw_multi_matches_single_and_oracle():
    shapes = [(3,), (50257, 8), (768,), (5, 7), (4096,), (1,), (0,), (3072, 3)]
    dtypes = [torch.float32, torch.float32, torch.bfloat16, torch.float16,
              torch.float32, torch.float32, torch.float32, torch.float32]
    params = [randn(s, d, i) for i, (s, d) in enumerate(zip(shapes, dtypes))]
    grads = [randn(s, d, 100 + i) * 1e-2 for i, (s, d) in enumerate(zip(shapes, dtypes))]
    ms = [torch.zeros(s, device="cuda") for s in shapes]
    vs = [torch.zeros(s, device="cuda") for s in shapes]
    ref_p = [p.clone() for p in params]
    ref_m = [m.clone() for m in ms]
    ref_v = [v.clone() for v in vs]
    hp = dict(lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    for step in (1, 2):
        tritium.adamw_step_multi(params, grads, ms, vs, step=step, **hp)
        for p, g, m, v in zip(ref_p, grads, ref_m, ref_v):
            tritium.adamw_step(p, g, m, v, step=step, **hp)
    for a, b in zip(params + ms + vs, ref_p + ref_m + ref_v):
        assert torch.equal(a, b)
    ep, em, ev = oracle.adamw.step(np32(params[1]), np32(grads[1]),
                                   np32(ms[1]), np32(vs[1]), step=3, **hp)
    tritium.adamw_step_multi(params, grads, ms, vs, step=3, **hp)
    assert_close(params[1], ep, 1e-5, 1e-5)


@pytest.mark.parametrize("dtype", DTYPES)
def test_adamw_multi_misaligned_and_ragged(dtype):
    # tensors starting one element past a 16-byte boundary (the element path in every
    # chunk) beside aligned ones whose sizes straddle the 256-element workgroup chunks;
    # bitwise equal to the single-tensor kernel, and the oracle after 2 steps
    flat = randn((1 + 1000 + 300 + 7,), dtype, 90)
    mis = [flat[1:1001], flat[1001:1301], flat[1301:1308]]
    params = mis + [randn((n,), dtype, 91 + n) for n in (255, 256, 257, 1027)]
    grads = [randn(tuple(p.shape), dtype, 200 + i) * 1e-2 for i, p in enumerate(params)]
    ms = [torch.zeros(p.shape, device="cuda") for p in params]
    vs = [torch.zeros(p.shape, device="cuda") for p in params]
    # the single-tensor reference on copies with the same alignment (the same code path:
    # the element path and the vector groups may contract the update into FMAs differently)
    flat_ref = flat.clone()
    ref = [(flat_ref[1:1001], ms[0].clone(), vs[0].clone()),
           (flat_ref[1001:1301], ms[1].clone(), vs[1].clone()),
           (flat_ref[1301:1308], ms[2].clone(), vs[2].clone())]
    ref += [(p.clone(), m.clone(), v.clone()) for p, m, v in zip(params[3:], ms[3:], vs[3:])]
    states = [(np32(p), np32(m), np32(v)) for p, m, v in zip(params, ms, vs)]
    gnp = [np32(g) for g in grads]
    hp = dict(lr=6e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)
    for step in (1, 2):
        tritium.adamw_step_multi(params, grads, ms, vs, step=step, **hp)
        for (p, m, v), g in zip(ref, grads):
            tritium.adamw_step(p, g, m, v, step=step, **hp)
        states = [oracle.adamw.step(ep, eg, em, ev, step=step, dtype=NAME[dtype], **hp)
                  for (ep, em, ev), eg in zip(states, gnp)]
    for (rp, rm, rv), p, m, v in zip(ref, params, ms, vs):
        assert torch.equal(p, rp) and torch.equal(m, rm) and torch.equal(v, rv)
    rtol, atol = TOL[dtype]
    for p, (ep, _, _) in zip(params, states):
        assert_close(p, ep, rtol, atol, "param")


@pytest.mark.parametrize("gdtype", [torch.bfloat16, torch.float16])
def test_adamw_mixed_matches_fp32_step(gdtype):
    # tritium_adamw_step_mixed: same update as adamw_step on the widened gradient; the
    # shadow is the updated fp32 param rounded once; ragged sizes take the element path
    from helion_amd.adamw import adamw_step_mixed
    # (tensors of one or many 256-element workgroup chunks, with and without a ragged
    # last chunk or a last group of fewer than 4 elements)
    shapes = [(4096,), (33, 7), (1,), (768, 768), (5000,), (8193,), (3, 8191), (16384,),
              (255,), (257,), (1027,)]
    ps = [randn(s, torch.float32, 40 + i, scale=0.02) for i, s in enumerate(shapes)]
    gs = [randn(s, gdtype, 50 + i, scale=1e-2) for i, s in enumerate(shapes)]
    ms = [randn(s, torch.float32, 60 + i, scale=1e-3) for i, s in enumerate(shapes)]
    vs = [randn(s, torch.float32, 70 + i, scale=1e-3).abs() for i, s in enumerate(shapes)]
    sh = [torch.zeros(s, device="cuda", dtype=gdtype) for s in shapes]
    ref = [(p.clone(), g.float(), m.clone(), v.clone()) for p, g, m, v in zip(ps, gs, ms, vs)]
    kw = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=10)
    adamw_step_mixed(ps, gs, ms, vs, sh, **kw)
    for (rp, rg, rm, rv), p, m, v, s_ in zip(ref, ps, ms, vs, sh):
        tritium.adamw_step(rp, rg, rm, rv, **kw)
        for a, e in ((p, rp), (m, rm), (v, rv)):
            torch.testing.assert_close(a, e, rtol=1e-6, atol=1e-9)
        assert torch.equal(s_, p.to(gdtype))


def test_adamw_mixed_misaligned_views():
    # tensors that start 4 bytes past a 16-byte boundary take the element path in every
    # chunk (the kernel's vector groups need 16-byte aligned fp32 and 8-byte aligned
    # 16-bit rows); results as adamw_step on the widened gradient
    from helion_amd.adamw import adamw_step_mixed
    sizes = [1000, 300, 7]
    def views(dtype, seed, scale):
        flat = randn((sum(sizes) + 1,), dtype, seed, scale=scale)
        out, off = [], 1
        for n in sizes:
            out.append(flat[off:off + n])
            off += n
        return out
    ps, gs = views(torch.float32, 80, 0.02), views(torch.bfloat16, 81, 1e-2)
    ms, vs = views(torch.float32, 82, 1e-3), [v.abs() for v in views(torch.float32, 83, 1e-3)]
    sh = views(torch.bfloat16, 84, 1.0)
    assert all(p.data_ptr() % 16 != 0 for p in ps)
    ref = [(p.clone(), g.float(), m.clone(), v.clone()) for p, g, m, v in zip(ps, gs, ms, vs)]
    kw = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1, step=3)
    adamw_step_mixed(ps, gs, ms, vs, sh, **kw)
    for (rp, rg, rm, rv), p, m, v, s_ in zip(ref, ps, ms, vs, sh):
        tritium.adamw_step(rp, rg, rm, rv, **kw)
        for a, e in ((p, rp), (m, rm), (v, rv)):
            torch.testing.assert_close(a, e, rtol=1e-6, atol=1e-9)
        assert torch.equal(s_, p.to(torch.bfloat16))


def test_adamw_step1_closed_form():
    # from zero moments, step 1: p1 = p*(1 - lr*wd) - lr * g / (|g| + eps)
    n = 4096
    p = randn((n,), torch.float32, 1)
    g = randn((n,), torch.float32, 2)
    m, v = torch.zeros(n, device="cuda"), torch.zeros(n, device="cuda")
    lr, wd, eps = 1e-3, 0.1, 1e-8
    expect = np32(p) * (1 - lr * wd) - lr * np32(g) / (np.abs(np32(g)) + eps)
    tritium.adamw_step(p, g, m, v, lr=lr, beta1=0.9, beta2=0.95, eps=eps, weight_decay=wd, step=1)
    assert_close(p, expect, 1e-5, 1e-6)

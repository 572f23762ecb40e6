"""Pin the CPU oracle (the checker every GPU parity test trusts).

Each oracle function is checked against, as applicable:

* the golden fixtures in tests/golden/ -- float64 outputs of torch's library
  routines (F.rms_norm, F.scaled_dot_product_attention, F.cross_entropy,
  torch.optim.AdamW, complex multiplication) and their autograd, which is
  what the reference's own tests compare its kernels against;
* closed forms and invariants the mathematics fixes (constant rows, W = 0,
  x = 0, T = 1, position 0, norm preservation, inverse(forward) = identity);
* float64 finite differences of the oracle's own forward;
* the storage rounding rule against torch's own bfloat16/float16 casts.

The "planted mistake" tests alter an oracle function on the CPU (a dropped
term, a swapped sign, a wrong denominator) and assert that the pinning
checks above reject it, so the pins are shown to be sensitive.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def fixture(name):
    with np.load(os.path.join(GOLDEN, f"{name}.npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def close(a, b, tol=1e-10):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return a.shape == b.shape and bool(np.all(np.abs(a - b) <= tol * (1 + np.abs(b))))


def fd_grad(f, x, dy, eps=1e-6):
    """Directional finite difference: sum(dy * df/dx) along random unit direction u."""
    rng = np.random.default_rng(0)
    u = rng.standard_normal(x.shape)
    u /= np.linalg.norm(u)
    plus = np.sum(dy * f(x + eps * u))
    minus = np.sum(dy * f(x - eps * u))
    return (plus - minus) / (2 * eps), u


# --------------------------------------------------------------- numerics --
def test_bf16_round_matches_torch_cast():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(10000).astype(np.float32) * 10,
        np.array([0.0, -0.0, 1e-40, 3.0e38, np.inf, -np.inf], dtype=np.float32),
        # exact ties: the low 16 bits are 0x8000 -> round half to even
        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], dtype=np.float32),
    ])
    ref = torch.from_numpy(x).bfloat16().float().numpy()
    np.testing.assert_array_equal(oracle.numerics.bf16_round(x), ref)
    assert np.isnan(oracle.numerics.bf16_round(np.array([np.nan], dtype=np.float32)))[0]


def test_quantize_f16_matches_torch_cast():
    x = np.random.default_rng(2).standard_normal(5000).astype(np.float32) * 100
    ref = torch.from_numpy(x).half().float().numpy()
    np.testing.assert_array_equal(oracle.numerics.quantize(x, "f16"), ref)


# ---------------------------------------------------------------- rmsnorm --
def test_rmsnorm_against_torch_rms_norm_golden():
    g = fixture("rmsnorm")
    y, rstd = oracle.rmsnorm.forward(g["x"], g["w"], float(g["eps"]), acc=np.float64)
    dx, dw = oracle.rmsnorm.backward(g["dy"], g["x"], g["w"], None, float(g["eps"]), acc=np.float64,
                                     dtype="f32")
    # forward/backward are stored through float32 by the oracle's rounding step
    assert close(y, g["y"], 1e-6) and close(dx, g["dx"], 1e-6) and close(dw, g["dw"], 1e-6)


def test_rmsnorm_constant_row_closed_form():
    c, eps = 0.37, 1e-6
    x = np.full((3, 64), c)
    w = np.linspace(0.5, 1.5, 64)
    y, _ = oracle.rmsnorm.forward(x, w, eps, acc=np.float64)
    assert close(y, w[None, :] * c / np.sqrt(c * c + eps) * np.ones((3, 1)), 1e-6)


def test_rmsnorm_backward_matches_finite_differences():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((4, 32))
    w = 1 + 0.1 * rng.standard_normal(32)
    dy = rng.standard_normal((4, 32))

    def f(xx):
        return oracle.rmsnorm.forward(xx, w, 1e-6, "f64", acc=np.float64)[0]

    dx, dw = oracle.rmsnorm.backward(dy, x, w, None, 1e-6, "f64", acc=np.float64)
    fd, u = fd_grad(f, x, dy)
    assert abs(fd - np.sum(dx * u)) < 1e-7
    fdw, uw = fd_grad(lambda ww: oracle.rmsnorm.forward(x, ww, 1e-6, "f64", acc=np.float64)[0], w, dy)
    assert abs(fdw - np.sum(dw * uw)) < 1e-7


def test_residual_rmsnorm_backward_is_rmsnorm_backward_plus_residual_grad():
    rng = np.random.default_rng(4)
    x, r = rng.standard_normal((5, 48)), rng.standard_normal((5, 48))
    w, dy, dz = 1 + 0.1 * rng.standard_normal(48), rng.standard_normal((5, 48)), rng.standard_normal((5, 48))
    y, z, rstd = oracle.rmsnorm.residual_forward(x, r, w, 1e-6, acc=np.float64)
    assert close(z, x + r, 1e-6)
    dzr, dwr = oracle.rmsnorm.residual_backward(dy, dz, z, w, rstd, acc=np.float64)
    dx, dw = oracle.rmsnorm.backward(dy, z, w, rstd, acc=np.float64)
    assert close(dzr, dx + dz, 1e-6) and close(dwr, dw, 1e-12)


# ------------------------------------------------------------------- rope --
def _rope_fixture_check(apply_fn):
    g = fixture("rope")
    ok = True
    for il in (0, 1):
        q_out = apply_fn(g["q"], g["cos"], g["sin"], position_ids=g["pos"], interleaved=bool(il))
        dq = apply_fn(g["dq_out"], g["cos"], g["sin"], position_ids=g["pos"], interleaved=bool(il),
                      inverse=True)
        ok &= close(q_out, g[f"q_out_{il}"], 1e-5) and close(dq, g[f"dq_{il}"], 1e-5)
    return ok


def test_rope_against_complex_multiplication_golden():
    # backward of a rotation = rotation by the opposite angle (autograd of the complex form)
    assert _rope_fixture_check(oracle.rope.apply)


def test_rope_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((12, 2, 32)).astype(np.float32)
    cos, sin = oracle.rope.make_cos_sin(64, 32)
    pos = rng.integers(0, 64, 12)
    y = oracle.rope.apply(x, cos, sin, position_ids=pos)
    half = 16
    # pair norms preserved
    assert np.allclose(x[..., :half] ** 2 + x[..., half:] ** 2, y[..., :half] ** 2 + y[..., half:] ** 2,
                       rtol=1e-5, atol=1e-5)
    # inverse(forward) = identity
    back = oracle.rope.apply(y, cos, sin, position_ids=pos, inverse=True)
    assert np.allclose(back, x, atol=1e-5)
    # position 0 is the identity
    y0 = oracle.rope.apply(x, cos, sin, position_ids=np.zeros(12, dtype=np.int64))
    assert np.array_equal(y0, x)


def test_rope_tables_match_float64_angles():
    # cos/sin of t * theta^(-2i/d) (tests/tritium/test_rope.py:38-45); the float32
    # recipe rounds the angle, an error that grows with the position t
    c, s = oracle.rope.make_cos_sin(2048, 128)
    tc, ts = oracle.torch_ref.make_cos_sin(2048, 128)
    ang = np.outer(np.arange(2048.0), 1.0 / 10000.0 ** (np.arange(64) / 64.0))
    bound = 8 * ang * 2.0 ** -24 + 1e-6
    for table, fn in ((c, np.cos), (s, np.sin), (tc.numpy(), np.cos), (ts.numpy(), np.sin)):
        assert np.all(np.abs(table - fn(ang)) <= bound)


# ----------------------------------------------------------------- swiglu --
def test_swiglu_against_torch_silu_golden():
    g = fixture("swiglu")
    out = oracle.swiglu.forward(g["x"], g["gate"])
    dx, dgate = oracle.swiglu.backward(g["dy"], g["x"], g["gate"])
    assert close(out, g["out"], 1e-5) and close(dx, g["dx"], 1e-5) and close(dgate, g["dgate"], 1e-5)


def test_swiglu_zero_input_closed_form():
    gate = np.linspace(-2, 2, 11).astype(np.float32)
    dy = np.linspace(1, 3, 11).astype(np.float32)
    x = np.zeros(11, dtype=np.float32)
    assert np.all(oracle.swiglu.forward(x, gate) == 0)
    dx, dgate = oracle.swiglu.backward(dy, x, gate)
    assert np.all(dgate == 0) and np.allclose(dx, dy * gate / 2, atol=1e-7)


# ------------------------------------------------------------------ adamw --
def test_adamw_against_torch_optim_golden():
    g = fixture("adamw")
    p, m, v = g["p0"].astype(np.float32), np.zeros_like(g["p0"], np.float32), np.zeros_like(g["p0"], np.float32)
    for step in (1, 2, 3):
        p, m, v = oracle.adamw.step(p, g["g"][step - 1].astype(np.float32), m, v, lr=float(g["lr"]),
                                    beta1=float(g["beta1"]), beta2=float(g["beta2"]),
                                    eps=float(g["eps"]), weight_decay=float(g["wd"]), step=step)
    assert np.allclose(p, g["p3"], rtol=1e-5, atol=1e-7)
    assert np.allclose(m, g["m3"], rtol=1e-5, atol=1e-9)
    assert np.allclose(v, g["v3"], rtol=1e-5, atol=1e-12)


def test_adamw_step1_closed_form():
    rng = np.random.default_rng(6)
    p = rng.standard_normal(100).astype(np.float32)
    gr = rng.standard_normal(100).astype(np.float32)
    lr, wd, eps = 1e-3, 0.1, 1e-8
    p1, _, _ = oracle.adamw.step(p, gr, np.zeros(100, np.float32), np.zeros(100, np.float32), lr=lr,
                                 beta1=0.9, beta2=0.95, eps=eps, weight_decay=wd, step=1)
    assert np.allclose(p1, p * (1 - lr * wd) - lr * gr / (np.abs(gr) + eps), rtol=1e-5, atol=1e-7)


# -------------------------------------------------------------- attention --
def test_attention_against_sdpa_golden():
    g = fixture("attention")
    for causal in (1, 0):
        o, lse = oracle.attention.forward(g["q"], g["k"], g["v"], bool(causal))
        dq, dk, dv = oracle.attention.backward(g["do"], g["q"], g["k"], g["v"], lse, bool(causal))
        assert close(o, g[f"o_{causal}"]) and close(lse, g[f"lse_{causal}"])
        assert close(dq, g[f"dq_{causal}"]) and close(dk, g[f"dk_{causal}"]) and close(dv, g[f"dv_{causal}"])


def test_attention_invariants():
    rng = np.random.default_rng(7)
    q = rng.standard_normal((1, 2, 1, 16))
    k = rng.standard_normal((1, 2, 1, 16))
    v = rng.standard_normal((1, 2, 1, 16))
    o, lse = oracle.attention.forward(q, k, v, True)
    assert close(o, v)  # T = 1
    q = rng.standard_normal((1, 2, 9, 16))
    k = rng.standard_normal((1, 2, 9, 16))
    v = rng.standard_normal((1, 2, 9, 16))
    o, lse = oracle.attention.forward(q, k, v, True)
    assert close(o[:, :, 0], v[:, :, 0])  # causal row 0 sees only key 0
    s = np.einsum("bhqd,bhkd->bhqk", q, k) * 16 ** -0.5
    assert np.all(lse >= np.max(np.where(np.tril(np.ones((9, 9), bool)), s, -np.inf), -1) - 1e-12)
    vu = np.broadcast_to(v[:, :, :1], v.shape).copy()
    assert close(oracle.attention.forward(q, k, vu, True)[0], vu)  # uniform values


# --------------------------------------------------------------- linear-CE --
def test_linear_ce_against_cross_entropy_golden():
    g = fixture("linear_ce")
    loss, lse = oracle.linear_ce.forward(g["hidden"], g["weight"], g["target"])
    dh, dw = oracle.linear_ce.backward(float(g["grad_out"]), g["hidden"], g["weight"], g["target"], lse)
    assert close(loss, g["loss"]) and close(lse, g["lse"])
    assert close(dh, g["dhidden"]) and close(dw, g["dweight"])


def test_linear_ce_zero_weight_closed_form_and_all_ignored():
    rng = np.random.default_rng(8)
    n, d, v = 10, 6, 7
    h = rng.standard_normal((n, d))
    t = rng.integers(0, v, n)
    t[:3] = -100
    loss, lse = oracle.linear_ce.forward(h, np.zeros((v, d)), t)
    assert abs(loss - np.log(v)) < 1e-12
    dh, dw = oracle.linear_ce.backward(1.0, h, np.zeros((v, d)), t, lse)
    valid = t != -100
    onehot = np.zeros((n, v))
    onehot[np.nonzero(valid)[0], t[valid]] = 1
    expect = ((1.0 / v - onehot) * valid[:, None]).T @ h / valid.sum()
    assert np.all(dh == 0) and close(dw, expect)
    t[:] = -100
    loss, lse = oracle.linear_ce.forward(h, rng.standard_normal((v, d)), t)
    assert np.isnan(loss)
    dh, dw = oracle.linear_ce.backward(1.0, h, rng.standard_normal((v, d)), t, lse)
    assert np.all(dh == 0) and np.all(dw == 0)


def test_linear_ce_backward_matches_finite_differences():
    rng = np.random.default_rng(9)
    h = rng.standard_normal((6, 5))
    w = rng.standard_normal((9, 5))
    t = np.array([1, 3, -100, 8, 0, 2])
    _, lse = oracle.linear_ce.forward(h, w, t)
    dh, dw = oracle.linear_ce.backward(1.0, h, w, t, lse)
    for x, grad, f in ((h, dh, lambda hh: oracle.linear_ce.forward(hh, w, t)[0]),
                       (w, dw, lambda ww: oracle.linear_ce.forward(h, ww, t)[0])):
        fd, u = fd_grad(f, x, 1.0)
        assert abs(fd - np.sum(grad * u)) < 1e-7


# -------------------------------------------------------- planted mistakes --
def test_planted_mistakes_are_caught(monkeypatch):
    """Each pin above must reject a plausible mistake planted in the oracle."""
    g = fixture("rmsnorm")
    # rmsnorm: eps outside the square root
    def bad_rstd(x2d, eps, acc=np.float32):
        x2d = x2d.astype(acc)
        return (1.0 / (np.sqrt((x2d * x2d).mean(axis=1)) + eps)).astype(acc)
    monkeypatch.setattr(oracle.rmsnorm, "rstd_of", bad_rstd)
    y, _ = oracle.rmsnorm.forward(g["x"], g["w"], 1e-6, acc=np.float64)
    assert not close(y, g["y"], 1e-9)
    monkeypatch.undo()

    # rope: the backward uses the forward rotation (sign not flipped)
    real_apply = oracle.rope.apply

    def bad_apply(x, cos, sin, inverse=False, **kw):
        return real_apply(x, cos, sin, inverse=False, **kw)

    assert not _rope_fixture_check(bad_apply)

    # attention: scale dropped from dq
    ga = fixture("attention")
    o, lse = oracle.attention.forward(ga["q"], ga["k"], ga["v"], True)
    dq, _, _ = oracle.attention.backward(ga["do"], ga["q"], ga["k"], ga["v"], lse, True)
    assert not close(dq / 16 ** -0.5, ga["dq_1"])

    # linear-CE: mean over all rows instead of the non-ignored ones
    gl = fixture("linear_ce")
    t = gl["target"].copy()
    loss, _ = oracle.linear_ce.forward(gl["hidden"], gl["weight"], t)
    assert not close(loss * (t != -100).sum() / t.size, gl["loss"])

    # adamw: decay applied after the Adam update instead of before
    gw = fixture("adamw")
    p = gw["p0"].astype(np.float32)
    m = v = np.zeros_like(p)
    for step in (1, 2, 3):
        gr = gw["g"][step - 1].astype(np.float32)
        p2, m, v = oracle.adamw.step(p, gr, m, v, lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8,
                                     weight_decay=0.0, step=step)
        p = p2 - 3e-4 * 0.1 * p2
    assert not np.allclose(p, gw["p3"], rtol=1e-7, atol=0)


# ---------------------------------------------------- torch_ref formulas --
def test_torch_ref_formulas_agree_with_library_routines():
    """The CPU-baseline formulas (the reference's test formulas) against torch library routines."""
    g = torch.Generator().manual_seed(10)
    x = torch.randn(8, 64, generator=g, dtype=torch.float64)
    w = 1 + 0.02 * torch.randn(64, generator=g, dtype=torch.float64)
    assert torch.allclose(oracle.torch_ref.rmsnorm(x, w, 1e-6).double(),
                          torch.nn.functional.rms_norm(x.float(), (64,), w.float(), 1e-6).double(),
                          atol=1e-6)
    q = torch.randn(1, 4, 10, 16, generator=g)
    k = torch.randn(1, 2, 10, 16, generator=g)
    v = torch.randn(1, 2, 10, 16, generator=g)
    o_np, _ = oracle.attention.forward(q.numpy(), k.numpy(), v.numpy(), True)
    assert np.allclose(oracle.torch_ref.attention(q, k, v, True).numpy(), o_np, atol=1e-5)


def test_torch_ref_rmsnorm_backward_and_rope_against_golden():
    """The CPU-baseline RMSNorm backward and RoPE formulas against the golden fixtures
    (torch's F.rms_norm autograd; complex multiplication and its autograd)."""
    g = fixture("rmsnorm")
    x, w, dy = (torch.from_numpy(g[k]) for k in ("x", "w", "dy"))
    dx, dw = oracle.torch_ref.rmsnorm_backward(dy, x, w, float(g["eps"]))
    assert close(dx.numpy(), g["dx"], 1e-5) and close(dw.numpy(), g["dw"], 1e-5)
    r = fixture("rope")
    q, k, cos, sin, pos = (torch.from_numpy(r[n]) for n in ("q", "k", "cos", "sin", "pos"))
    qo, ko = oracle.torch_ref.rope(q, k, cos, sin, pos)
    assert close(qo.numpy(), r["q_out_0"], 1e-5) and close(ko.numpy(), r["k_out_0"], 1e-5)
    # the backward of a rotation is the inverse rotation
    dq, _ = oracle.torch_ref.rope(torch.from_numpy(r["dq_out"]), k, cos, sin, pos, inverse=True)
    assert close(dq.numpy(), r["dq_0"], 1e-5)
    # planted mistake: the forward rotation used as the backward
    dq_wrong, _ = oracle.torch_ref.rope(torch.from_numpy(r["dq_out"]), k, cos, sin, pos)
    assert not close(dq_wrong.numpy(), r["dq_0"], 1e-3)


# -------------------------------------------------------------- embedding --
def test_embedding_backward_against_torch_golden():
    g = fixture("embedding")
    got = oracle.embedding.backward(g["ids"], g["dx"], g["dw_head"])
    assert close(got, g["dw"], 1e-6)
    assert (np.bincount(g["ids"]) > 1).any()  # the fixture repeats ids


def test_embedding_backward_distinct_ids_closed_form():
    rng = np.random.default_rng(3)
    vocab, dim = 50, 8
    ids = rng.permutation(vocab)[:20]
    dx = rng.standard_normal((20, dim)).astype(np.float32)
    dw = rng.standard_normal((vocab, dim)).astype(np.float32)
    got = oracle.embedding.backward(ids, dx, dw)
    want = dw.astype(np.float64).copy()
    want[ids] += dx
    assert close(got, want, 1e-6)
    # out-of-range ids contribute nothing
    assert close(oracle.embedding.backward(np.array([-1, vocab]), dx[:2], dw), dw, 0)


def test_embedding_backward_planted_dropped_repeat_is_rejected():
    g = fixture("embedding")
    wrong = g["dw_head"].copy()
    wrong[g["ids"]] += g["dx"]  # fancy-index += keeps one of each repeated id
    assert not close(wrong, g["dw"], 1e-3)

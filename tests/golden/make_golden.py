"""Write the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py
[name ...]; no names = all of them).

The reference's own implementation cannot run here (it needs Triton and a
GPU), and it holds no golden vectors.  Its tests compare each kernel against
torch formulas or torch library routines at run time; these fixtures freeze
those expected values, computed in float64 by torch's *library* routines
(not by the oracle under test), on small seeded inputs:

* rmsnorm:   torch.nn.functional.rms_norm + autograd            (tests/tritium/test_rmsnorm.py:12-37)
* rope:      complex multiplication x * exp(i * pos * theta) + autograd (tests/tritium/test_rope.py:11-45)
* swiglu:    torch.nn.functional.silu(x) * gate + autograd        (tests/tritium/test_swiglu.py:9-10)
* adamw:     torch.optim.AdamW(foreach=False), 3 steps           (tests/tritium/test_adamw.py:19-27)
* attention: torch.nn.functional.scaled_dot_product_attention + autograd, GQA via
             repeat_interleave                                    (tests/tritium/test_attention.py:9-21)
* linear_ce: torch.nn.functional.cross_entropy(linear(h, W), t, ignore_index=-100) + autograd
                                                                  (tests/tritium/test_cross_entropy.py:72, 93)
* embedding: torch.nn.functional.embedding + autograd, plus the tied head's weight gradient
                                                                  (helion/nn.py:24-28)

Each fixture is an .npz of plain arrays (no pickles).
"""

from __future__ import annotations

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))
D = torch.float64


def gen(seed):
    return torch.Generator().manual_seed(seed)


def save(name, **arrays):
    path = os.path.join(HERE, f"{name}.npz")
    np.savez(path, **{k: (v.detach().numpy() if torch.is_tensor(v) else np.asarray(v))
                      for k, v in arrays.items()})
    print("wrote", path)


def rmsnorm():
    g = gen(100)
    x = torch.randn(24, 96, generator=g, dtype=D)
    w = 1 + 0.02 * torch.randn(96, generator=g, dtype=D)
    dy = torch.randn(24, 96, generator=g, dtype=D)
    xs, ws = x.clone().requires_grad_(True), w.clone().requires_grad_(True)
    y = F.rms_norm(xs, (96,), ws, eps=1e-6)
    y.backward(dy)
    save("rmsnorm", x=x, w=w, dy=dy, eps=1e-6, y=y, dx=xs.grad, dw=ws.grad)


def rope():
    g = gen(101)
    t, h, d = 20, 3, 16
    half = d // 2
    q = torch.randn(t, h, d, generator=g, dtype=D)
    k = torch.randn(t, h, d, generator=g, dtype=D)
    pos = torch.randint(0, 40, (t,), generator=g)
    inv = 1.0 / (10000.0 ** (torch.arange(half, dtype=D) / half))
    ang = torch.outer(torch.arange(40, dtype=D), inv)
    cos, sin = ang.cos(), ang.sin()
    dq = torch.randn(t, h, d, generator=g, dtype=D)

    def rot(x, interleaved):
        if interleaved:
            z = torch.view_as_complex(x.reshape(t, h, half, 2).contiguous())
        else:
            z = torch.complex(x[..., :half], x[..., half:])
        z = z * torch.polar(torch.ones_like(ang[pos]), ang[pos])[:, None, :]
        if interleaved:
            return torch.view_as_real(z).reshape(t, h, d)
        return torch.cat((z.real, z.imag), dim=-1)

    out = {}
    for il in (False, True):
        qs = q.clone().requires_grad_(True)
        yo = rot(qs, il)
        yo.backward(dq)
        out[f"q_out_{int(il)}"] = yo
        out[f"dq_{int(il)}"] = qs.grad
        out[f"k_out_{int(il)}"] = rot(k, il)
    save("rope", q=q, k=k, pos=pos, cos=cos, sin=sin, dq_out=dq, **out)


def swiglu():
    g = gen(102)
    x = torch.randn(300, generator=g, dtype=D) * 3
    gate = torch.randn(300, generator=g, dtype=D)
    dy = torch.randn(300, generator=g, dtype=D)
    xs, gs = x.clone().requires_grad_(True), gate.clone().requires_grad_(True)
    out = F.silu(xs) * gs
    out.backward(dy)
    save("swiglu", x=x, gate=gate, dy=dy, out=out, dx=xs.grad, dgate=gs.grad)


def adamw():
    g = gen(103)
    p = 0.02 * torch.randn(257, generator=g, dtype=D)
    grads = [torch.randn(257, generator=g, dtype=D) * 1e-2 for _ in range(3)]
    hp = dict(lr=3e-4, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1)
    ps = p.clone().requires_grad_(True)
    opt = torch.optim.AdamW([ps], foreach=False, **hp)
    for gr in grads:
        ps.grad = gr.clone()
        opt.step()
    st = opt.state[ps]
    save("adamw", p0=p, g=torch.stack(grads), p3=ps.detach(), m3=st["exp_avg"],
         v3=st["exp_avg_sq"], lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, wd=0.1)


def attention():
    g = gen(104)
    b, h, hkv, t, d = 2, 4, 2, 17, 16
    q = torch.randn(b, h, t, d, generator=g, dtype=D)
    k = torch.randn(b, hkv, t, d, generator=g, dtype=D)
    v = torch.randn(b, hkv, t, d, generator=g, dtype=D)
    do = torch.randn(b, h, t, d, generator=g, dtype=D)
    out = {}
    for causal in (True, False):
        qs, ks, vs = (x.clone().requires_grad_(True) for x in (q, k, v))
        o = F.scaled_dot_product_attention(qs, ks.repeat_interleave(h // hkv, 1),
                                           vs.repeat_interleave(h // hkv, 1), is_causal=causal)
        o.backward(do)
        s = (q @ k.repeat_interleave(h // hkv, 1).transpose(-1, -2)) * d ** -0.5
        if causal:
            s = s.masked_fill(~torch.ones(t, t, dtype=torch.bool).tril(), float("-inf"))
        c = int(causal)
        out.update({f"o_{c}": o, f"dq_{c}": qs.grad, f"dk_{c}": ks.grad, f"dv_{c}": vs.grad,
                    f"lse_{c}": torch.logsumexp(s, dim=-1)})
    save("attention", q=q, k=k, v=v, do=do, **out)


def linear_ce():
    g = gen(105)
    n, d, vocab = 30, 24, 50
    hdn = torch.randn(n, d, generator=g, dtype=D)
    w = 0.3 * torch.randn(vocab, d, generator=g, dtype=D)
    t = torch.randint(0, vocab, (n,), generator=g)
    t[torch.randperm(n, generator=g)[:4]] = -100
    hs, ws = hdn.clone().requires_grad_(True), w.clone().requires_grad_(True)
    logits = F.linear(hs, ws)
    loss = F.cross_entropy(logits, t, ignore_index=-100)
    loss.backward(torch.tensor(0.75, dtype=D))
    save("linear_ce", hidden=hdn, weight=w, target=t, grad_out=0.75, loss=loss,
         lse=torch.logsumexp(logits.detach(), dim=-1), dhidden=hs.grad, dweight=ws.grad)


def embedding():
    # tied embedding: the gather's scatter-add gradient plus the head's weight
    # gradient; ids repeat (rows hit several times) and leave rows untouched
    g = gen(106)
    vocab, dim, n = 40, 12, 60
    w = torch.randn(vocab, dim, generator=g, dtype=D)
    ids = torch.randint(0, vocab // 2, (n,), generator=g)
    ids[::7] = 3  # one frequent id
    dx = torch.randn(n, dim, generator=g, dtype=D)
    dw_head = torch.randn(vocab, dim, generator=g, dtype=D)
    ws = w.clone().requires_grad_(True)
    loss = (F.embedding(ids, ws) * dx).sum() + (ws * dw_head).sum()
    loss.backward()
    save("embedding", ids=ids, dx=dx, dw_head=dw_head, dw=ws.grad)


if __name__ == "__main__":
    import sys

    fns = {f.__name__: f for f in (rmsnorm, rope, swiglu, adamw, attention, linear_ce, embedding)}
    for name in (sys.argv[1:] or list(fns)):
        fns[name]()

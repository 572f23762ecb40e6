"""The reference's own PyTorch formulas for each hot-path op, run by torch on
the CPU -- TEST INFRASTRUCTURE ONLY.

These are the closed forms the reference's tests compare its kernels against
(alkinun/helion ``tests/tritium/test_*.py``), restated here so that

* ``bench.py``'s ``cpu_baseline`` leg can time "the reference PyTorch CPU path"
  on the host cores (the reference itself has no CPU path: every op rejects
  CPU tensors, ``tritium/ops/_utils.py:25-27``);
* the CPU test-suite can pin the numpy oracle against torch's library
  routines (``F.rms_norm``, ``F.scaled_dot_product_attention``,
  ``F.cross_entropy``, ``torch.optim.AdamW``) and torch autograd.

Everything computes in float32 (the references upcast with ``.float()``).
Nothing in ``helion_amd`` imports this module.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    """tests/tritium/test_rmsnorm.py:12-21 (``_rmsnorm_reference``)."""
    xf = x.float()
    rstd = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return xf * rstd * w.float()


def rmsnorm_backward(dy, x, w, eps: float):
    """tests/tritium/test_rmsnorm.py:24-37 (``_rmsnorm_backward_reference``)."""
    dyf, xf, wf = dy.float(), x.float(), w.float()
    hidden = x.shape[-1]
    rstd = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    dot = (dyf * wf * xf).sum(dim=-1, keepdim=True)
    dx = dyf * wf * rstd - xf * dot * rstd.pow(3) / hidden
    dw = (dyf * xf * rstd).sum(dim=tuple(range(x.dim() - 1)))
    return dx, dw


def rope(q, k, cos, sin, position_ids=None, inverse: bool = False):
    """tests/tritium/test_rope.py:11-35 (``_rope_reference``); ``inverse``
    flips the sign of sin (the backward, rope.py:76-85)."""
    n_tokens = q.shape[0]
    half = q.shape[-1] // 2
    pos = torch.arange(n_tokens) if position_ids is None else position_ids
    idx = pos.to(torch.long)
    c, s = cos.float()[idx], sin.float()[idx]
    if inverse:
        s = -s
    if q.dim() == 3:
        c, s = c.unsqueeze(1), s.unsqueeze(1)

    def rot(t):
        t = t.float()
        t1, t2 = t[..., :half], t[..., half:]
        return torch.cat((t1 * c - t2 * s, t2 * c + t1 * s), dim=-1)

    return rot(q), rot(k)


def make_cos_sin(max_seq_len: int, head_dim: int, theta: float = 10000.0):
    """tests/tritium/test_rope.py:38-45 (``_make_cos_sin``)."""
    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (torch.arange(0, half).float() / half))
    t = torch.arange(max_seq_len).float()
    freqs = torch.outer(t, inv_freq)
    return freqs.cos().contiguous(), freqs.sin().contiguous()


def swiglu_fwd_bwd(x, gate, dy):
    """tests/tritium/test_swiglu.py:9-10 (``F.silu(x) * gate``) and its autograd."""
    xf = x.float().requires_grad_(True)
    gf = gate.float().requires_grad_(True)
    out = F.silu(xf) * gf
    out.backward(dy.float())
    return out.detach(), xf.grad, gf.grad


def adamw(params, grads, *, lr, beta1, beta2, eps, weight_decay, steps=1):
    """tests/tritium/test_adamw.py:19-27: ``torch.optim.AdamW(foreach=False)``.

    Runs ``steps`` steps with the same grads and returns the optimizer (its
    state holds exp_avg/exp_avg_sq)."""
    ps = [p.float().clone().requires_grad_(True) for p in params]
    opt = torch.optim.AdamW(ps, lr=lr, betas=(beta1, beta2), eps=eps,
                            weight_decay=weight_decay, foreach=False)
    for _ in range(steps):
        for p, g in zip(ps, grads):
            p.grad = g.float()
        opt.step()
    return ps, opt


def attention(q, k, v, is_causal: bool = True):
    """tests/tritium/test_attention.py:9-21: SDPA with ``repeat_interleave``
    for GQA, in float32."""
    group = q.shape[1] // k.shape[1]
    kf = k.float().repeat_interleave(group, dim=1)
    vf = v.float().repeat_interleave(group, dim=1)
    return F.scaled_dot_product_attention(q.float(), kf, vf, is_causal=is_causal)


def linear_cross_entropy(hidden, weight, target, ignore_index: int = -100):
    """tests/tritium/test_cross_entropy.py:72: ``F.cross_entropy(F.linear(h, W).float(), t)``
    with torch's ``ignore_index`` and mean reduction."""
    logits = F.linear(hidden.float(), weight.float())
    return F.cross_entropy(logits, target.long(), ignore_index=ignore_index)

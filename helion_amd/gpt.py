"""GPT training step on the MI355X kernel layer, and its pure-PyTorch twin.

The model is the reference's decoder (examples/common.py:54-131:
``TransformerBlock`` = residual-RMSNorm -> attention (helion/nn.py:169-220:
q/k/v/o projections, RoPE on q and k, causal attention) -> residual-RMSNorm
-> SwiGLU MLP, final residual-RMSNorm, ``linear_cross_entropy`` against the
embedding matrix) at the 124M-class size of the benchmark: 12 layers,
d_model 768, 12 heads x 64, MLP 3072, vocab 50304, tied embeddings
(151,898,880 parameters), RoPE theta 1e4.

Precision boundary.  The optimizer owns fp32 master weights in one flat
buffer; each step runs on a bf16 working copy (one flat buffer, the model's
parameters are views into it).  The bf16 gradients come back from
``torch.autograd.grad`` (nothing accumulated, so no gradient zeroing) and
``adamw_step_mixed`` consumes them as they are: one launch updates the fp32
masters and moments and rounds each updated master into its bf16 working
weight.  Activations are bf16 throughout; every op computes in fp32
internally (the kernels' own rule), the residual stream is stored in bf16
as the reference's residual-RMSNorm does (rmsnorm.py:72-83).

Plain projections (q/k/v fused into one, o, gate/up fused into one, down)
are library GEMMs (hipBLASLt; weight gradients split over token slices by
one batched GEMM, ``_Proj``); everything on the kernel
layer's hot path is a HIP kernel: residual-RMSNorm, RoPE (k rotated once out
of the fused q/k/v output; q rotated by the attention kernels as they load it,
``_QKVRopeAttention``), causal attention, SwiGLU (on the fused gate/up
output), fused linear-cross-entropy, the tied embedding's backward and
AdamW.

``TorchTwin`` computes the same step with PyTorch only (F.rms_norm,
F.scaled_dot_product_attention, F.silu, F.cross_entropy on materialised
logits, torch.optim.AdamW) from identical initial weights and data, for the
loss-curve parity check; its attention and norms run in fp32.

Run ``python -m helion_amd.gpt --steps 200`` on a GPU for the parity report.
"""

from __future__ import annotations

import argparse
import dataclasses
import json
import math
import time

import torch
import torch.nn.functional as F

from . import _lib
from .adamw import adamw_step_mixed
from .attention import attention_rope_bwd, attention_rope_fwd
from .embedding import embedding_backward
from .linear_ce import _backward as _lce_backward
from .linear_ce import _linear_cross_entropy_forward
from .rmsnorm import residual_rmsnorm
from .rope import rope_rows
from .swiglu import swiglu_rows, swiglu_rows_backward


@dataclasses.dataclass(frozen=True)
class GPTConfig:
    vocab_size: int = 50304
    d_model: int = 768
    n_layers: int = 12
    n_heads: int = 12
    head_dim: int = 64
    d_ff: int = 3072
    max_seq_len: int = 1024
    rope_theta: float = 10000.0
    eps: float = 1e-6


@dataclasses.dataclass(frozen=True)
class TrainConfig:
    batch: int = 16
    seq_len: int = 1024
    lr: float = 6e-4
    beta1: float = 0.9
    beta2: float = 0.95
    eps: float = 1e-8
    weight_decay: float = 0.1
    seed: int = 0


def param_shapes(cfg: GPTConfig) -> list[tuple[str, tuple[int, ...]]]:
    """Parameter names and shapes in a fixed order (the flat-buffer layout)."""
    d, f = cfg.d_model, cfg.d_ff
    qd = cfg.n_heads * cfg.head_dim
    out = [("embed", (cfg.vocab_size, d))]
    for i in range(cfg.n_layers):
        p = f"blocks.{i}."
        out += [
            (p + "attn_norm", (d,)),
            (p + "wq", (qd, d)),
            (p + "wk", (qd, d)),
            (p + "wv", (qd, d)),
            (p + "wo", (d, qd)),
            (p + "ffn_norm", (d,)),
            (p + "w_gate", (f, d)),
            (p + "w_up", (f, d)),
            (p + "w_down", (d, f)),
        ]
    out.append(("final_norm", (d,)))
    return out


def init_params(cfg: GPTConfig, seed: int = 0) -> dict[str, torch.Tensor]:
    """fp32 initial weights on the CPU: N(0, 0.02) for matrices and the
    embedding (helion/nn.py:24, 48; examples/common.py:111), ones for norms."""
    g = torch.Generator().manual_seed(seed)
    params = {}
    for name, shape in param_shapes(cfg):
        if len(shape) == 1:
            params[name] = torch.ones(shape, dtype=torch.float32)
        else:
            params[name] = torch.randn(shape, generator=g, dtype=torch.float32) * 0.02
    return params


def rope_tables(cfg: GPTConfig, device) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos / sin [max_seq_len, head_dim/2] (helion/nn.py:179-184)."""
    half = cfg.head_dim // 2
    inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, half, dtype=torch.float64) / half))
    t = torch.arange(cfg.max_seq_len, dtype=torch.float64)
    freqs = torch.outer(t, inv_freq)
    return (freqs.cos().to(device=device, dtype=torch.float32),
            freqs.sin().to(device=device, dtype=torch.float32))


def lm_batch(cfg: GPTConfig, tc: TrainConfig, gen: torch.Generator, device,
             learnable: bool = False):
    """Uniform random tokens (examples/common.py:146-153), drawn on the CPU
    from ``gen`` so both models see the same batches.  ``learnable`` gives
    each row consecutive ids from a random start instead (the next token is
    predictable, so a working step lowers the loss)."""
    shape = (tc.batch, tc.seq_len + 1)
    if learnable:
        start = torch.randint(cfg.vocab_size, (tc.batch, 1), generator=gen)
        tokens = (start + torch.arange(shape[1])) % cfg.vocab_size
    else:
        tokens = torch.randint(cfg.vocab_size, shape, generator=gen)
    tokens = tokens.to(device)
    return tokens[:, :-1].contiguous(), tokens[:, 1:].contiguous()


class _Flat:
    """Views of ``param_shapes`` into one flat tensor, plus each layer's fused
    q/k/v projection ``blocks.i.wqkv`` [3 * n_heads * head_dim, d_model] and
    fused gate/up projection ``blocks.i.w_gu`` [2 * d_ff, d_model] (wq, wk, wv
    and w_gate, w_up are adjacent in the layout, so these are views too)."""

    def __init__(self, cfg: GPTConfig, flat: torch.Tensor):
        self.flat = flat
        self.views: dict[str, torch.Tensor] = {}
        offsets = {}
        off = 0
        for name, shape in param_shapes(cfg):
            n = math.prod(shape)
            self.views[name] = flat[off:off + n].view(shape)
            offsets[name] = off
            off += n
        assert off == flat.numel()
        qd = cfg.n_heads * cfg.head_dim
        for i in range(cfg.n_layers):
            o = offsets[f"blocks.{i}.wq"]
            self.views[f"blocks.{i}.wqkv"] = flat[o:o + 3 * qd * cfg.d_model].view(3 * qd, cfg.d_model)
            o = offsets[f"blocks.{i}.w_gate"]
            self.views[f"blocks.{i}.w_gu"] = flat[o:o + 2 * cfg.d_ff * cfg.d_model].view(
                2 * cfg.d_ff, cfg.d_model)

    def leaves(self) -> dict[str, torch.Tensor]:
        """The tensors the model differentiates: every parameter except the
        separate q/k/v and gate/up views, which the fused wqkv and w_gu cover."""
        return {k: v for k, v in self.views.items()
                if not k.endswith((".wq", ".wk", ".wv", ".w_gate", ".w_up"))}


def n_params(cfg: GPTConfig) -> int:
    return sum(math.prod(s) for _, s in param_shapes(cfg))


class HipGPT:
    """The model and its optimizer state on the HIP kernel layer."""

    def __init__(self, cfg: GPTConfig, tc: TrainConfig, init: dict[str, torch.Tensor], device):
        self.cfg, self.tc, self.device = cfg, tc, device
        n = n_params(cfg)
        self.master = _Flat(cfg, torch.empty(n, device=device, dtype=torch.float32))
        for name, t in init.items():
            self.master.views[name].copy_(t)
        self.work = _Flat(cfg, self.master.flat.to(torch.bfloat16))
        self.exp_avg = torch.zeros(n, device=device, dtype=torch.float32)
        self.exp_avg_sq = torch.zeros(n, device=device, dtype=torch.float32)
        leaves = self.work.leaves()
        for p in leaves.values():
            p.requires_grad_(True)
        self._params = list(leaves.values())
        m, v = _Flat(cfg, self.exp_avg), _Flat(cfg, self.exp_avg_sq)
        self._master = [self.master.views[name] for name in leaves]
        self._m = [m.views[name] for name in leaves]
        self._v = [v.views[name] for name in leaves]
        self._shadow = [p.detach() for p in self._params]
        self._last_grads: tuple[torch.Tensor, ...] = ()
        self.cos, self.sin = rope_tables(cfg, device)
        self.step_count = 0

    def _w(self, name: str) -> torch.Tensor:
        return self.work.views[name]

    def loss(self, tokens: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
        cfg = self.cfg
        b, s = tokens.shape
        nh, hd = cfg.n_heads, cfg.head_dim
        pos = torch.arange(s, device=tokens.device).repeat(b)
        cos, sin = self.cos[:s], self.sin[:s]
        tied = _TiedGrad()
        delta = _TiedEmbed.apply(self._w("embed"), tokens, tied)
        residual = torch.zeros_like(delta)
        t, d = b * s, cfg.d_model
        for i in range(cfg.n_layers):
            p = f"blocks.{i}."
            normed, residual = residual_rmsnorm(delta, residual, self._w(p + "attn_norm"), cfg.eps)
            qkv = _Proj.apply(normed.view(t, d), self._w(p + "wqkv")).view(b, s, 3, nh, hd)
            o = _QKVRopeAttention.apply(qkv, cos, sin, pos, None).reshape(t, nh * hd)
            delta = _Proj.apply(o, self._w(p + "wo")).view(b, s, d)
            normed, residual = residual_rmsnorm(delta, residual, self._w(p + "ffn_norm"), cfg.eps)
            h = _GateUpSwiGLU.apply(_Proj.apply(normed.view(t, d), self._w(p + "w_gu")))
            delta = _Proj.apply(h, self._w(p + "w_down")).view(b, s, d)
        hidden, _ = residual_rmsnorm(delta, residual, self._w("final_norm"), cfg.eps)
        return _TiedHeadCE.apply(hidden, self._w("embed"), targets, tied)

    def train_step(self, tokens: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
        """One step: forward, backward, fp32-master AdamW; returns the loss."""
        tc = self.tc
        loss = self.loss(tokens, targets)
        global _overlap_active
        overlap = OVERLAP_DW and self.device.type == "cuda"
        _overlap_active = overlap
        try:
            grads = torch.autograd.grad(loss, self._params)
        finally:
            _overlap_active = False
        if overlap:
            # the weight gradients computed on the second stream
            torch.cuda.current_stream(self.device).wait_stream(_side_stream(self.device))
        self.step_count += 1
        # fp32 masters from the bf16 gradients, and the bf16 working weights rounded
        # from the updated masters, in one pass
        adamw_step_mixed(self._master, grads, self._m, self._v, self._shadow, lr=tc.lr,
                         beta1=tc.beta1, beta2=tc.beta2, eps=tc.eps,
                         weight_decay=tc.weight_decay, step=self.step_count)
        self._last_grads = grads
        return loss.detach()

    def grad_norm(self) -> float:
        """L2 norm of the last step's gradients (fp32 accumulation)."""
        norms = torch.stack([torch.linalg.vector_norm(g.float()) for g in self._last_grads])
        return float(torch.linalg.vector_norm(norms))


class TorchTwin:
    """The same model, data and update in plain PyTorch (no kernel-layer op)."""

    def __init__(self, cfg: GPTConfig, tc: TrainConfig, init: dict[str, torch.Tensor], device):
        self.cfg, self.tc = cfg, tc
        self.master = {k: v.to(device).clone().requires_grad_(True) for k, v in init.items()}
        self.opt = torch.optim.AdamW(list(self.master.values()), lr=tc.lr,
                                     betas=(tc.beta1, tc.beta2), eps=tc.eps,
                                     weight_decay=tc.weight_decay, foreach=False)
        self.cos, self.sin = rope_tables(cfg, device)

    def _rope(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        half = x.shape[-1] // 2
        x = x.float()
        a, b = x[..., :half], x[..., half:]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], dim=-1).to(torch.bfloat16)

    def _norm(self, delta, residual, w):
        z = delta.float() + residual.float()
        out = F.rms_norm(z, (z.shape[-1],), w.float(), self.cfg.eps)
        return out.to(torch.bfloat16), z.to(torch.bfloat16)

    def loss(self, work: dict[str, torch.Tensor], tokens, targets) -> torch.Tensor:
        cfg = self.cfg
        b, s = tokens.shape
        nh, hd = cfg.n_heads, cfg.head_dim
        cos = self.cos[:s].view(1, s, 1, hd // 2)
        sin = self.sin[:s].view(1, s, 1, hd // 2)
        delta = work["embed"][tokens]
        residual = torch.zeros_like(delta)
        for i in range(cfg.n_layers):
            p = f"blocks.{i}."
            normed, residual = self._norm(delta, residual, work[p + "attn_norm"])
            q = self._rope((normed @ work[p + "wq"].t()).view(b, s, nh, hd), cos, sin)
            k = self._rope((normed @ work[p + "wk"].t()).view(b, s, nh, hd), cos, sin)
            v = (normed @ work[p + "wv"].t()).view(b, s, nh, hd)
            o = F.scaled_dot_product_attention(q.transpose(1, 2).float(), k.transpose(1, 2).float(),
                                               v.transpose(1, 2).float(), is_causal=True)
            o = o.transpose(1, 2).reshape(b, s, nh * hd).to(torch.bfloat16)
            delta = o @ work[p + "wo"].t()
            normed, residual = self._norm(delta, residual, work[p + "ffn_norm"])
            gate = (normed @ work[p + "w_gate"].t()).float()
            up = (normed @ work[p + "w_up"].t()).float()
            delta = (F.silu(gate) * up).to(torch.bfloat16) @ work[p + "w_down"].t()
        hidden, _ = self._norm(delta, residual, work["final_norm"])
        logits = hidden.reshape(-1, cfg.d_model) @ work["embed"].t()
        return F.cross_entropy(logits.float(), targets.reshape(-1))

    def train_step(self, tokens, targets) -> torch.Tensor:
        work = {k: v.detach().to(torch.bfloat16).requires_grad_(True)
                for k, v in self.master.items()}
        loss = self.loss(work, tokens, targets)
        loss.backward()
        for k, p in self.master.items():
            p.grad = work[k].grad.float()
        self.opt.step()
        self.opt.zero_grad(set_to_none=True)
        self.last_grad_norm = float(torch.norm(torch.stack([
            work[k].grad.float().norm() for k in self.master])))
        return loss.detach()


class _TiedGrad:
    """Carries the output head's weight gradient from the head's backward (which
    autograd runs first) to the embedding gather's backward (which it runs
    last), so the two gradients of the tied weight are summed in one pass."""

    def __init__(self) -> None:
        self.dw: torch.Tensor | None = None


class _TiedHeadCE(torch.autograd.Function):
    """linear_cross_entropy(hidden, weight, targets) whose weight gradient goes
    to the ``_TiedGrad`` holder instead of to autograd (the gather's backward
    returns the tied weight's whole gradient)."""

    @staticmethod
    def forward(ctx, hidden, weight, targets, holder):
        n = targets.numel()
        loss, lse = _linear_cross_entropy_forward(hidden, weight, targets)
        ctx.holder = holder
        ctx.save_for_backward(hidden.view(n, hidden.shape[-1]), weight, targets.view(n), lse)
        ctx.hidden_shape = tuple(hidden.shape)
        return loss

    @staticmethod
    def backward(ctx, g):
        hidden_2d, weight, targets, lse = ctx.saved_tensors
        dh, dw = _lce_backward(g, hidden_2d, weight, targets, lse, ctx.needs_input_grad[0], True,
                               -100)
        ctx.holder.dw = dw
        return (dh.view(ctx.hidden_shape) if dh is not None else None), None, None, None


class _TiedEmbed(torch.autograd.Function):
    """weight[tokens] (helion/nn.py:24-28); the backward adds the scatter of the
    upstream rows into the head's weight gradient from the holder, in place,
    with ``tritium_embedding_bwd`` (deterministic: token-order fp32 sums, one
    rounding), replacing torch's sort + scatter and the separate add."""

    @staticmethod
    def forward(ctx, weight, tokens, holder):
        ctx.holder = holder
        ctx.save_for_backward(tokens)
        ctx.weight_shape, ctx.dtype = tuple(weight.shape), weight.dtype
        return F.embedding(tokens, weight)

    @staticmethod
    def backward(ctx, dx):
        (tokens,) = ctx.saved_tensors
        dw, ctx.holder.dw = ctx.holder.dw, None
        if dw is None:
            dw = torch.zeros(ctx.weight_shape, device=dx.device, dtype=ctx.dtype)
        d = ctx.weight_shape[1]
        embedding_backward(tokens.reshape(-1), dx.reshape(-1, d), dw, out=dw)
        return dw, None, None


class _QKVRopeAttention(torch.autograd.Function):
    """Causal attention over the fused q/k/v projection ``[b, s, 3, heads,
    head_dim]`` with RoPE on q and k (helion/nn.py:196-220): k is rotated once
    into a contiguous copy; q and v are read in place, q unrotated and rotated
    as the attention kernels load it (``attention_rope_fwd``), so no rotated q
    is written or kept.  The output is ``[b, s, heads, head_dim]`` memory (a
    free view of the o projection's input).  The backward writes dq (the dQ
    kernel un-rotates it) and dv straight into one fused gradient and
    un-rotates dk into it.  ``pos`` holds the flattened tokens' positions for
    k's rotation; ``q_pos`` those of the attention kernels' queries, or None
    when each sequence's positions are 0..s-1 (the kernels then take a query's
    row index as its position and read no position table)."""

    @staticmethod
    def forward(ctx, qkv, cos, sin, pos, q_pos):
        b, s, _, nh, hd = qkv.shape
        flat = qkv.view(b * s, 3, nh, hd)
        k = torch.empty((b * s, nh, hd), device=qkv.device, dtype=qkv.dtype)
        rope_rows(None, flat[:, 1], cos, sin, pos, None, k, inverse=False,
                  in_token_stride=3 * nh * hd, out_token_stride=nh * hd)
        q, v = qkv[:, :, 0].transpose(1, 2), qkv[:, :, 2].transpose(1, 2)
        o, lse = attention_rope_fwd(q, k.view(b, s, nh, hd).transpose(1, 2), v, cos, sin, q_pos,
                                    True)
        ctx.save_for_backward(qkv, k, o, lse, cos, sin, pos, q_pos)
        return o.transpose(1, 2)

    @staticmethod
    def backward(ctx, do):
        qkv, k, o, lse, cos, sin, pos, q_pos = ctx.saved_tensors
        b, s, _, nh, hd = qkv.shape
        dqkv = torch.empty_like(qkv)
        dk = torch.empty((b, s, nh, hd), device=qkv.device, dtype=qkv.dtype)
        attention_rope_bwd(do.transpose(1, 2), qkv[:, :, 0].transpose(1, 2),
                           k.view(b, s, nh, hd).transpose(1, 2), qkv[:, :, 2].transpose(1, 2),
                           o, lse, cos, sin, q_pos, True, dq=dqkv[:, :, 0].transpose(1, 2),
                           dk=dk.transpose(1, 2), dv=dqkv[:, :, 2].transpose(1, 2))
        rope_rows(None, dk.view(b * s, nh, hd), cos, sin, pos, None,
                  dqkv.view(b * s, 3, nh, hd)[:, 1], inverse=True, in_token_stride=nh * hd,
                  out_token_stride=3 * nh * hd)
        return dqkv, None, None, None, None


def _split_k(n_out: int, n_in: int, k: int) -> int:
    """Number of K slices for a weight gradient dW = dY^T X [n_out, n_in] reduced
    over k tokens: the largest power of two (at most 16, slices of at least 512
    tokens) that keeps about 160 of the GPU's 256 compute units' worth of
    256 x 256 output tiles busy.  The library's own choice for these shapes
    (few output tiles, long reduction) runs at 230-590 TFLOP/s; measured at
    k = 16384: [768, 768] 90 -> 41 us with 16 slices, [2304, 768] 122 -> 95 us
    with 4, [768, 3072] 161 -> 106 us with 4, [6144, 768] unchanged."""
    tiles = -(-n_out // 256) * -(-n_in // 256)
    s = 1
    while s < 16 and 2 * s * tiles <= 160 and k % (2 * s) == 0 and k // (2 * s) >= 512:
        s *= 2
    return s


_bmm_out_dtype: bool | None = None  # torch.bmm(..., out_dtype=float32) available


def _bmm_fp32_out_supported(device) -> bool:
    """Whether this torch accepts ``torch.bmm(..., out_dtype=float32)`` for
    16-bit operands, probed once on a tiny product; a TypeError (an unknown
    keyword) or NotImplementedError (no kernel for the combination) means no,
    anything else is a real failure and propagates."""
    global _bmm_out_dtype
    if _bmm_out_dtype is None:
        a = torch.zeros((1, 2, 2), device=device, dtype=torch.bfloat16)
        try:
            torch.bmm(a, a, out_dtype=torch.float32)
            _bmm_out_dtype = True
        except (TypeError, NotImplementedError):
            _bmm_out_dtype = False
    return _bmm_out_dtype


def _sum_splits(part: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """part.sum(0) rounded once into ``dtype``, in one pass (``tritium_sum_splits``:
    fp32 sum in split order)."""
    part = part.contiguous()
    out = torch.empty(part.shape[1:], device=part.device, dtype=dtype)
    _lib.call("tritium_sum_splits", part.data_ptr(), out.data_ptr(), part.shape[0], out.numel(),
              _lib.dtype_code(dtype), _lib.stream_of(part))
    return out


# Weight gradients on a second stream: nothing in the backward reads them, so
# their GEMMs (and split sums) can run beside the rest of the backward, which
# fills the GPU around the tails of its kernels; the optimizer's stream waits
# for them once, before the update.  Only inside HipGPT.train_step, which
# makes that wait before anything reads the gradients (a plain .backward()
# through _Proj elsewhere keeps them on the calling stream).  The stream has
# the default priority.  Measured on the config-5 step: 660-663K -> 686-690K
# tokens/s, gradients and updated weights bitwise equal to the one-stream step.
OVERLAP_DW = True
_SIDE: dict[int, torch.cuda.Stream] = {}
_overlap_active = False


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    s = _SIDE.get(idx)
    if s is None:
        s = torch.cuda.Stream(device=idx)
        _SIDE[idx] = s
    return s


def _weight_grad(x: torch.Tensor, dy: torch.Tensor) -> torch.Tensor:
    k, n_out = dy.shape
    s = _split_k(n_out, x.shape[1], k)
    if s > 1 and _bmm_fp32_out_supported(dy.device):
        part = torch.bmm(dy.view(s, k // s, n_out).transpose(1, 2),
                         x.view(s, k // s, x.shape[1]), out_dtype=torch.float32)
        return _sum_splits(part, dy.dtype)
    return dy.t() @ x


class _Proj(torch.autograd.Function):
    """y = x W^T for a projection of the token rows x [tokens, in]; the weight
    gradient is reduced over token slices by one batched GEMM with fp32 outputs
    and summed in fp32 (one rounding, as a single GEMM would), which gives the
    short-and-wide weight-gradient GEMMs the parallelism they lack."""

    @staticmethod
    def forward(ctx, x, w):
        ctx.save_for_backward(x, w)
        return x @ w.t()

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dy = dy.contiguous()
        dx = dy @ w if ctx.needs_input_grad[0] else None
        dw = None
        if ctx.needs_input_grad[1]:
            if _overlap_active and not torch.cuda.is_current_stream_capturing():
                main = torch.cuda.current_stream(dy.device)
                side = _side_stream(dy.device)
                side.wait_stream(main)
                with torch.cuda.stream(side):
                    dw = _weight_grad(x, dy)
                # x and dy are freed on the main stream after this returns, dw is
                # read there after HipGPT.train_step's wait: keep each block out
                # of the other stream's reuse until both streams are past it
                x.record_stream(side)
                dy.record_stream(side)
                dw.record_stream(main)
            else:
                dw = _weight_grad(x, dy)
        return dx, dw


class _GateUpSwiGLU(torch.autograd.Function):
    """SwiGLU of a fused gate/up projection ``[tokens, 2 * d_ff]`` (gate in the
    first half of each row, up in the second): silu(gate) * up, with the
    gradients written back into one fused ``[tokens, 2 * d_ff]`` tensor.  The
    projection is then one GEMM forward and two backward instead of two and
    four plus the sum of the two input gradients."""

    @staticmethod
    def forward(ctx, gu):
        f = gu.shape[1] // 2
        out = torch.empty((gu.shape[0], f), device=gu.device, dtype=gu.dtype)
        swiglu_rows(gu[:, :f], gu[:, f:], out)
        ctx.save_for_backward(gu)
        return out

    @staticmethod
    def backward(ctx, dy):
        (gu,) = ctx.saved_tensors
        f = gu.shape[1] // 2
        dgu = torch.empty_like(gu)
        swiglu_rows_backward(dy.contiguous(), gu[:, :f], gu[:, f:], dgu[:, :f], dgu[:, f:])
        return dgu


def time_steps(model: HipGPT, cfg: GPTConfig, tc: TrainConfig, steps: int, warmup: int,
               seed: int = 0) -> dict:
    """Tokens per second of ``model.train_step`` (batches pre-generated)."""
    gen = torch.Generator().manual_seed(seed)
    batches = [lm_batch(cfg, tc, gen, model.device) for _ in range(steps + warmup)]
    for i in range(warmup):
        model.train_step(*batches[i])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup, warmup + steps):
        loss = model.train_step(*batches[i])
    torch.cuda.synchronize()
    dt = (time.perf_counter() - t0) / steps
    tokens = tc.batch * tc.seq_len
    flops = 6 * n_params(cfg) * tokens + 6 * cfg.n_layers * tc.seq_len * cfg.d_model * tokens
    return {"ms_per_step": dt * 1e3, "tokens_per_s": tokens / dt, "loss": float(loss),
            "mfu": flops / dt / 2.5e15}


def parity(steps: int, cfg: GPTConfig, tc: TrainConfig, device, learnable: bool = False) -> dict:
    """Loss curves of HipGPT and TorchTwin over ``steps`` steps from the same
    weights and batches; returns both curves and the largest relative gap."""
    init = init_params(cfg, tc.seed)
    ours = HipGPT(cfg, tc, init, device)
    twin = TorchTwin(cfg, tc, init, device)
    gen = torch.Generator().manual_seed(tc.seed + 1)
    la, lb, ga, gb = [], [], [], []
    for _ in range(steps):
        tokens, targets = lm_batch(cfg, tc, gen, device, learnable)
        la.append(float(ours.train_step(tokens, targets)))
        ga.append(ours.grad_norm())
        lb.append(float(twin.train_step(tokens, targets)))
        gb.append(twin.last_grad_norm)
    gap = max(abs(a - b) / abs(b) for a, b in zip(la, lb))
    return {"steps": steps, "loss_hip": la, "loss_torch": lb, "grad_norm_hip": ga,
            "grad_norm_torch": gb, "max_rel_loss_gap": gap}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description="config-5 GPT: loss parity and tokens/s")
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--out", default="")
    ap.add_argument("--layers", type=int, default=12)
    ap.add_argument("--batch", type=int, default=16)
    args = ap.parse_args(argv)
    cfg = GPTConfig(n_layers=args.layers)
    tc = TrainConfig(batch=args.batch)
    dev = torch.device("cuda")
    res = parity(args.steps, cfg, tc, dev)
    summary = {k: v for k, v in res.items() if not isinstance(v, list)}
    summary["loss_first_last_hip"] = [res["loss_hip"][0], res["loss_hip"][-1]]
    summary["loss_first_last_torch"] = [res["loss_torch"][0], res["loss_torch"][-1]]
    summary["grad_norm_step1"] = [res["grad_norm_hip"][0], res["grad_norm_torch"][0]]
    print(json.dumps(summary))
    if args.out:
        with open(args.out, "w") as f:
            json.dump(res, f)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())

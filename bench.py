"""Benchmark of the MI355X tritium.ops hot path (one GPU).

``python bench.py [--gpus 1] [--steps K] [--warmup W]`` prints ONE JSON line.

Headline workload (the ``value``): the bandwidth-bound config --
RMSNorm -> RoPE -> SwiGLU forward+backward in bf16 on activations
[8, 2048, 4096] (RoPE over 32 heads x 128, SwiGLU over [8, 2048, 11008]) plus
one fused multi-tensor AdamW step over the 124,439,808 fp32 parameters of the
GPT-2-small shape list (148 tensors).  A step is one pass of all four ops;
``value`` is algorithmic HBM bytes per step / step time (GB/s).  Inputs are
generated on a seeded CPU generator and are resident in HBM before timing.

Also reported in the same line (``ops``): each op's time and fraction of its
roofline, causal flash attention fwd+bwd [4, 32, 4096, 128] bf16 in TFLOP/s,
fused linear-cross-entropy fwd+bwd N=8192 D=4096 V=128256 in TFLOP/s, and the
reference PyTorch CPU path timed on this host's cores (``cpu_baseline``; the
attention, linear-CE and GPT legs carry their own).

Kernel times are measured with HIP events recorded on the stream every kernel
is launched on (torch's current stream), two per measured span: the headline
spans K whole steps, each op of the breakdown K back-to-back calls of that op
(an event recorded between two kernels leaves the GPU idle for a few
microseconds while it drains the queue for the timestamp).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16

METRIC = "per-op fwd+bwd TFLOP/s or GB/s vs roofline; 124M GPT train tokens/sec"

# config 2 shapes
ROWS_B, ROWS_T, ROWS_D = 8, 2048, 4096
ROPE_H, ROPE_HD = 32, 128
SWIGLU_F = 11008
ADAMW_HP = dict(lr=3e-4, beta1=0.9, beta2=0.95, eps=1e-8, weight_decay=0.1)


def gpt2_small_shapes() -> list[tuple[int, ...]]:
    """The 148 parameter tensors of GPT-2 small (124,439,808 params)."""
    shapes: list[tuple[int, ...]] = [(50257, 768), (1024, 768)]
    for _ in range(12):
        shapes += [(768,), (768,), (768, 2304), (2304,), (768, 768), (768,),
                   (768,), (768,), (768, 3072), (3072,), (3072, 768), (768,)]
    shapes += [(768,), (768,)]
    return shapes


# ------------------------------------------------------ algorithmic bytes --
def rmsnorm_bytes(n: int, d: int, esz: int = 2) -> tuple[int, int]:
    """fwd: read x, write y, read w, write rstd; bwd: read dy, x, w, rstd, write dx, dw (fp32)."""
    fwd = 2 * n * d * esz + esz * d + 4 * n
    bwd = 3 * n * d * esz + esz * d + 4 * n + 4 * d
    return fwd, bwd


def rope_bytes(n_tok: int, h: int, hd: int, max_pos: int, esz: int = 2) -> tuple[int, int]:
    """read q, k, write q_out, k_out, read the cos/sin rows, read position ids."""
    one = 4 * n_tok * h * hd * esz + 2 * max_pos * (hd // 2) * 4 + 8 * n_tok
    return one, one


def swiglu_bytes(n: int, esz: int = 2) -> tuple[int, int]:
    return 3 * n * esz, 5 * n * esz


def adamw_bytes(n_params: int) -> int:
    return 28 * n_params  # read p, g, m, v; write p, m, v (fp32)


def attention_flops(b, h, t, d) -> tuple[float, float]:
    """Causal FA2 convention: 4*D flops per visible pair forward, 10*D backward."""
    pairs = b * h * t * t / 2
    return 4 * d * pairs, 10 * d * pairs


def lce_flops(n, d, v) -> tuple[float, float]:
    """Algorithmic: forward GEMM 2NVD, backward dH and dW 4NVD."""
    return 2.0 * n * v * d, 4.0 * n * v * d


# ------------------------------------------------------------ GPU legs --
class Timer:
    """HIP events on torch's current stream (the stream every op launches on)."""

    def __init__(self, torch):
        self.torch = torch
        self.pairs: dict[str, list] = {}

    def start(self, name):
        ev = self.torch.cuda.Event(enable_timing=True)
        ev.record()
        self.pairs.setdefault(name, []).append([ev, None])

    def stop(self, name):
        ev = self.torch.cuda.Event(enable_timing=True)
        ev.record()
        self.pairs[name][-1][1] = ev

    def mean_ms(self, name) -> float:
        vals = [a.elapsed_time(b) for a, b in self.pairs[name]]
        return sum(vals) / len(vals)

    def reset(self):
        self.pairs = {}


def row_leg(torch, tritium, steps: int, warmup: int):
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(0)
    n_rows = ROWS_B * ROWS_T

    def rn(shape, dtype, scale=1.0, mean=0.0):
        return (torch.randn(shape, generator=g) * scale + mean).to(dtype).to(dev)

    # RMSNorm: x, w = 1 + 0.02 N, dy
    x = rn((ROWS_B, ROWS_T, ROWS_D), torch.bfloat16).requires_grad_(True)
    w = rn((ROWS_D,), torch.bfloat16, 0.02, 1.0).requires_grad_(True)
    dy = rn((ROWS_B, ROWS_T, ROWS_D), torch.bfloat16)
    # RoPE: q, k as [tokens, heads, head_dim]; fp32 cos/sin; position ids
    q = rn((n_rows, ROPE_H, ROPE_HD), torch.bfloat16).requires_grad_(True)
    k = rn((n_rows, ROPE_H, ROPE_HD), torch.bfloat16).requires_grad_(True)
    half = ROPE_HD // 2
    inv_freq = 1.0 / (10000.0 ** (torch.arange(half, dtype=torch.float32) / half))
    freqs = torch.outer(torch.arange(ROWS_T, dtype=torch.float32), inv_freq)
    cos, sin = freqs.cos().to(dev), freqs.sin().to(dev)
    pos = torch.arange(ROWS_T, dtype=torch.int64).repeat(ROWS_B).to(dev)
    dq = rn((n_rows, ROPE_H, ROPE_HD), torch.bfloat16)
    dk = rn((n_rows, ROPE_H, ROPE_HD), torch.bfloat16)
    # SwiGLU: x (gets the silu) and gate
    sx = rn((ROWS_B, ROWS_T, SWIGLU_F), torch.bfloat16).requires_grad_(True)
    sg = rn((ROWS_B, ROWS_T, SWIGLU_F), torch.bfloat16).requires_grad_(True)
    sdy = rn((ROWS_B, ROWS_T, SWIGLU_F), torch.bfloat16)
    # AdamW over the GPT-2-small shape list
    shapes = gpt2_small_shapes()
    params = [rn(s, torch.float32, 0.02) for s in shapes]
    grads = [rn(s, torch.float32, 1e-2) for s in shapes]
    ms = [torch.zeros(s, device=dev) for s in shapes]
    vs = [torch.zeros(s, device=dev) for s in shapes]
    n_params = sum(p.numel() for p in params)

    step_no = [0]

    # each op's forward+backward (AdamW: one update); the gradients are cleared
    # so that the next call does not accumulate into them
    def op_rmsnorm():
        y = tritium.rmsnorm(x, w, 1e-6)
        torch.autograd.backward(y, dy)
        x.grad = w.grad = None

    def op_rope():
        qo, ko = tritium.rope(q, k, cos, sin, position_ids=pos)
        torch.autograd.backward((qo, ko), (dq, dk))
        q.grad = k.grad = None

    def op_swiglu():
        out = tritium.swiglu(sx, sg)
        torch.autograd.backward(out, sdy)
        sx.grad = sg.grad = None

    def op_adamw():
        step_no[0] += 1
        tritium.adamw_step_multi(params, grads, ms, vs, step=step_no[0], **ADAMW_HP)

    op_fns = {"rmsnorm": op_rmsnorm, "rope": op_rope, "swiglu": op_swiglu, "adamw": op_adamw}

    def step():
        for f in op_fns.values():
            f()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    # the headline: K whole steps between two events and nothing else on the
    # stream (an event recorded between two kernels leaves the GPU idle for
    # about 5 us while it drains the queue for the timestamp)
    t0 = time.perf_counter()
    ev0 = torch.cuda.Event(enable_timing=True)
    ev1 = torch.cuda.Event(enable_timing=True)
    ev0.record()
    for _ in range(steps):
        step()
    ev1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    step_ms = ev0.elapsed_time(ev1) / steps
    # the per-op breakdown: each op K times back to back between two events
    op_ms = {}
    for name, f in op_fns.items():
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(steps):
            f()
        e1.record()
        torch.cuda.synchronize()
        op_ms[name] = e0.elapsed_time(e1) / steps

    rb = rmsnorm_bytes(n_rows, ROWS_D)
    ropeb = rope_bytes(n_rows, ROPE_H, ROPE_HD, ROWS_T)
    sb = swiglu_bytes(ROWS_B * ROWS_T * SWIGLU_F)
    ab = adamw_bytes(n_params)
    per_op_bytes = {"rmsnorm": sum(rb), "rope": sum(ropeb), "swiglu": sum(sb), "adamw": ab}
    total_bytes = sum(per_op_bytes.values())
    ops = {}
    for name, nbytes in per_op_bytes.items():
        t = op_ms[name]
        gbs = nbytes / (t * 1e-3) / 1e9
        ops[name] = {"ms": round(t, 4), "bytes": nbytes, "GB/s": round(gbs, 1),
                     "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    value = total_bytes / (step_ms * 1e-3) / 1e9
    return {
        "value": value,
        "ms_per_step": step_ms,
        "wall_s": wall,
        "total_bytes": total_bytes,
        "ops": ops,
        "n_params": n_params,
        "adamw_ms": op_ms["adamw"],
        "adamw_bytes": ab,
    }


def attention_leg(torch, tritium, iters: int = 5, warmup: int = 2,
                  b=4, h=32, t=4096, d=128):
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(0)

    def rn(shape):
        return torch.randn(shape, generator=g).to(torch.bfloat16).to(dev)

    q, k, v = (rn((b, h, t, d)).requires_grad_(True) for _ in range(3))
    do = rn((b, h, t, d))

    def fwd_bwd():
        o = tritium.attention(q, k, v, is_causal=True)
        o.backward(do)
        q.grad = k.grad = v.grad = None

    def fwd():
        tritium.attention(q, k, v, is_causal=True)

    for _ in range(warmup):
        fwd_bwd()
    # forward+backward over `iters` passes between two events (events between
    # the kernels would leave the GPU idle for their timestamps), then the
    # forward alone the same way; the backward is the difference
    spans = {}
    for name, f in (("fwd_bwd", fwd_bwd), ("fwd", fwd)):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            f()
        e1.record()
        torch.cuda.synchronize()
        spans[name] = e0.elapsed_time(e1) / iters
    ff, fb = attention_flops(b, h, t, d)
    fwd_ms = spans["fwd"]
    bwd_ms = spans["fwd_bwd"] - fwd_ms
    tot = (ff + fb) / ((fwd_ms + bwd_ms) * 1e-3) / 1e12
    return {
        "shape": [b, h, t, d],
        "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
        "fwd_TFLOP/s": round(ff / (fwd_ms * 1e-3) / 1e12, 1),
        "bwd_TFLOP/s": round(fb / (bwd_ms * 1e-3) / 1e12, 1),
        "TFLOP/s": round(tot, 1),
        "frac_mfma_peak": round(tot / MFMA_BF16_PEAK_TFLOPS, 4),
        "roofline": mfma_roofline("attn_fwd_pp + attn_bwd_delta_v + attn_bwd_dkdv_pair (storing dS) + attn_bwd_dq_ds (one fwd+bwd)",
                                  ff + fb, fwd_ms + bwd_ms, "attention_config3_counters.txt"),
    }


def attention_gpt_leg(torch, tritium, iters: int = 20, warmup: int = 3,
                      b=16, t=1024, h=12, d=64):
    """Causal attention at the config-5 GPT block's shape, timed alone (outside the
    training step, where the projection GEMMs run beside it on a second stream):
    the block's own call, RoPE on q and k over the fused q/k/v projection
    [b, t, 3, h, d] (``_QKVRopeAttention`` in helion_amd/gpt.py: k rotated once,
    q rotated as the attention kernels load it), forward and forward+backward."""
    from helion_amd.gpt import _QKVRopeAttention

    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(0)
    qkv = torch.randn((b, t, 3, h, d), generator=g).to(torch.bfloat16).to(dev)
    qkv.requires_grad_(True)
    do = torch.randn((b, t, h, d), generator=g).to(torch.bfloat16).to(dev)
    half = d // 2
    inv_freq = 1.0 / (10000.0 ** (torch.arange(half, dtype=torch.float32) / half))
    freqs = torch.outer(torch.arange(t, dtype=torch.float32), inv_freq)
    cos, sin = freqs.cos().to(dev), freqs.sin().to(dev)
    pos = torch.arange(t, dtype=torch.int64).repeat(b).to(dev)

    def fwd_bwd():
        o = _QKVRopeAttention.apply(qkv, cos, sin, pos, None)
        o.backward(do)
        qkv.grad = None

    def fwd():
        with torch.no_grad():
            _QKVRopeAttention.apply(qkv, cos, sin, pos, None)

    for _ in range(warmup):
        fwd_bwd()
    spans = {}
    for name, f in (("fwd_bwd", fwd_bwd), ("fwd", fwd)):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        for _ in range(iters):
            f()
        e1.record()
        torch.cuda.synchronize()
        spans[name] = e0.elapsed_time(e1) / iters
    ff, fb = attention_flops(b, h, t, d)
    fwd_ms = spans["fwd"]
    bwd_ms = spans["fwd_bwd"] - fwd_ms
    tot = (ff + fb) / ((fwd_ms + bwd_ms) * 1e-3) / 1e12
    return {
        "shape": [b, h, t, d], "rope": "q on load, k once", "layout": "fused qkv [b, t, 3, h, d]",
        "fwd_ms": round(fwd_ms, 4), "bwd_ms": round(bwd_ms, 4),
        "fwd_TFLOP/s": round(ff / (fwd_ms * 1e-3) / 1e12, 1),
        "bwd_TFLOP/s": round(fb / (bwd_ms * 1e-3) / 1e12, 1),
        "TFLOP/s": round(tot, 1),
        "frac_mfma_peak": round(tot / MFMA_BF16_PEAK_TFLOPS, 4),
        "flops_basis": "FA2 convention, 14*D per visible pair (T^2/2 pairs per head)",
    }


def lce_leg(torch, tritium, iters: int = 3, warmup: int = 1, n=8192, d=4096, v=128256):
    if not hasattr(tritium, "linear_cross_entropy"):
        return None
    dev = torch.device("cuda")
    g = torch.Generator().manual_seed(0)
    hidden = torch.randn((n, d), generator=g).to(torch.bfloat16).to(dev).requires_grad_(True)
    weight = (torch.randn((v, d), generator=g) * 0.02).to(torch.bfloat16).to(dev)
    weight.requires_grad_(True)
    target = torch.randint(0, v, (n,), generator=g)
    target[torch.randperm(n, generator=g)[: n // 100]] = -100
    target = target.to(dev)
    timer = Timer(torch)
    loss = None
    for i in range(warmup + iters):
        if i == warmup:
            torch.cuda.synchronize()
            timer.reset()
        timer.start("fwd")
        loss = tritium.linear_cross_entropy(hidden, weight, target)
        timer.stop("fwd")
        timer.start("bwd")
        loss.backward()
        timer.stop("bwd")
        hidden.grad = weight.grad = None
    torch.cuda.synchronize()
    ff, fb = lce_flops(n, d, v)
    fwd_ms, bwd_ms = timer.mean_ms("fwd"), timer.mean_ms("bwd")
    tot = (ff + fb) / ((fwd_ms + bwd_ms) * 1e-3) / 1e12
    return {
        "shape": {"N": n, "D": d, "V": v, "ignored": n // 100},
        "loss": round(float(loss), 4),
        "fwd_ms": round(fwd_ms, 3), "bwd_ms": round(bwd_ms, 3),
        "TFLOP/s": round(tot, 1),
        "frac_mfma_peak": round(tot / MFMA_BF16_PEAK_TFLOPS, 4),
        "flops_basis": "6NVD algorithmic",
        "roofline": mfma_roofline("lce_fwd_kernel + lce_g_kernel + gemm_store_kernel (dW, dH) "
                                  "+ sum_splits (one fwd+bwd)", ff + fb, fwd_ms + bwd_ms,
                                  "linear_ce_config4_counters.txt"),
    }


# ------------------------------------------- the reference's benchmarks --
# The reference's own published rows (benchmarks/results/rtx3090.md, RTX 3090,
# "Tritium" column): fp16 inputs, its shapes and its logical-byte formulas
# (benchmarks/bench_*.py), rerun here the same way.  Its harness times with
# triton.testing.do_bench, which zeroes a cache-sized buffer before every run;
# a 512 MiB buffer (above MI355X's 256 MiB last-level cache) is zeroed before
# each timed call here for the same reason.
REF_ROWS = [
    # name, reference value, unit (GB/s: higher is better; ms: lower), rtx3090.md line
    ("rmsnorm_fwd 4096x1024", 705.3, "GB/s", 227),
    ("rmsnorm_fwd 128x8192", 440.3, "GB/s", 230),
    ("rmsnorm_bwd 4096x1024", 525.6, "GB/s", 217),
    ("residual_rmsnorm_fwd 4096x1024", 788.4, "GB/s", 247),
    ("residual_rmsnorm_fwd_bwd 4096x1024", 378.9, "GB/s", 236),
    ("rope 2048 tok x 32 x 128", 743.2, "GB/s", 258),
    ("swiglu_fwd n=2^25", 838.3, "GB/s", 342),
    ("swiglu_bwd n=2^25", 838.7, "GB/s", 324),
    ("adamw n=2^25 fp16", 535.6, "GB/s", 21),
    ("linear_ce_fwd 512x4096x128256", 8.07, "ms", 169),
    ("linear_ce_bwd 512x4096x128256", 25.50, "ms", 160),
    ("linear_ce_fwd 1024x4096x32000", 4.05, "ms", 170),
    ("linear_ce_bwd 1024x4096x32000", 11.78, "ms", 161),
    ("cross_entropy_fwd 128x1024", 41.367951, "GB/s", 68),
    ("cross_entropy_fwd 16x32768", 112.024969, "GB/s", 70),
]


def ref_bench_leg(torch, tritium, reps: int = 20):
    """Each REF_ROWS entry measured on this GPU: median of ``reps`` event-timed
    calls, each after a cache flush; GB/s rows use the reference's byte
    formula (bench_rmsnorm.py:110, 157, 204, 290; bench_rope.py:75-77;
    bench_swiglu.py:51, 84; bench_adamw.py:84)."""
    import statistics

    dev = torch.device("cuda")
    f16 = torch.float16
    g = torch.Generator(device=dev).manual_seed(0)
    flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)

    def rnd(*shape, dtype=f16):
        return torch.randn(shape, generator=g, device=dev, dtype=torch.float32).to(dtype)

    def ms_of(fn):
        fn()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        ts = []
        for _ in range(reps):
            flush.zero_()
            s.record()
            fn()
            e.record()
            torch.cuda.synchronize()
            ts.append(s.elapsed_time(e))
        return statistics.median(ts)

    out = {}
    x, w = rnd(4096, 1024), rnd(1024)
    out["rmsnorm_fwd 4096x1024"] = ((2 * x.numel() + w.numel()) * 2, ms_of(lambda: tritium.rmsnorm(x, w, 1e-6)))
    x2, w2 = rnd(128, 8192), rnd(8192)
    out["rmsnorm_fwd 128x8192"] = ((2 * x2.numel() + w2.numel()) * 2, ms_of(lambda: tritium.rmsnorm(x2, w2, 1e-6)))
    dy = rnd(4096, 1024)
    out["rmsnorm_bwd 4096x1024"] = ((4 * x.numel() + w.numel()) * 2,
                                    ms_of(lambda: tritium.rmsnorm_backward(dy, x, w, 1e-6)))
    r = rnd(4096, 1024)
    out["residual_rmsnorm_fwd 4096x1024"] = ((4 * x.numel() + w.numel()) * 2,
                                             ms_of(lambda: tritium.residual_rmsnorm(x, r, w, 1e-6)))
    xg, rg, wg = (t.clone().requires_grad_(True) for t in (x, r, w))
    dres = rnd(4096, 1024)

    def res_fb():
        xg.grad = rg.grad = wg.grad = None
        o, ro = tritium.residual_rmsnorm(xg, rg, wg, 1e-6)
        torch.autograd.backward((o, ro), (dy, dres))

    out["residual_rmsnorm_fwd_bwd 4096x1024"] = ((7 * x.numel() + w.numel()) * 2, ms_of(res_fb))
    t_, h_, d_ = 2048, 32, 128
    q, k = rnd(t_, h_, d_), rnd(t_, h_, d_)
    inv = 1.0 / (10000.0 ** (torch.arange(0, d_ // 2, device=dev).float() / (d_ // 2)))
    fr = torch.outer(torch.arange(t_, device=dev).float(), inv)
    cos, sin = fr.cos(), fr.sin()
    out["rope 2048 tok x 32 x 128"] = ((4 * t_ * h_ * d_ + 2 * t_ * (d_ // 2)) * 2,
                                       ms_of(lambda: tritium.rope(q, k, cos, sin)))
    n = 1 << 25
    a, b, dy1 = rnd(n), rnd(n), rnd(n)
    out["swiglu_fwd n=2^25"] = (3 * n * 2, ms_of(lambda: tritium.swiglu(a, b)))
    out["swiglu_bwd n=2^25"] = (5 * n * 2, ms_of(lambda: tritium.swiglu_backward(dy1, a, b)))
    pm, gm = rnd(n), rnd(n)
    m1 = torch.zeros(n, device=dev)
    v1 = torch.zeros(n, device=dev)
    out["adamw n=2^25 fp16"] = (7 * n * 2, ms_of(lambda: tritium.adamw_step(
        pm, gm, m1, v1, lr=3e-4, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.01, step=1)))
    del a, b, dy1, pm, gm, m1, v1
    for nr, dh, vv in ((512, 4096, 128256), (1024, 4096, 32000)):
        hid, wt = rnd(nr, dh), rnd(vv, dh)
        tgt = torch.randint(vv, (nr,), generator=g, device=dev)
        out[f"linear_ce_fwd {nr}x{dh}x{vv}"] = (None, ms_of(lambda: tritium.linear_cross_entropy(hid, wt, tgt)))
        lse = torch.logsumexp(torch.nn.functional.linear(hid, wt).float(), dim=-1)
        go = torch.tensor(1.0, device=dev)
        out[f"linear_ce_bwd {nr}x{dh}x{vv}"] = (None, ms_of(
            lambda: tritium.linear_cross_entropy_backward(go, hid, wt, tgt, lse)))
        del hid, wt, lse
    # bench_cross_entropy.py:42-51: fp16 logits, effective GB/s on the logits bytes
    for nr, vv in ((128, 1024), (16, 32768)):
        lg = rnd(nr, vv)
        tg = torch.randint(vv, (nr,), generator=g, device=dev)
        out[f"cross_entropy_fwd {nr}x{vv}"] = (lg.numel() * 2, ms_of(lambda: tritium.cross_entropy(lg, tg)))
    del flush
    torch.cuda.empty_cache()
    rows = []
    for name, ref, unit, line in REF_ROWS:
        nbytes, ms = out[name]
        if unit == "GB/s":
            ours = nbytes / (ms * 1e-3) / 1e9
            rows.append({"bench": name, "unit": unit, "mi355x": round(ours, 1), "rtx3090": ref,
                         "x": round(ours / ref, 2), "source": f"benchmarks/results/rtx3090.md:{line}"})
        else:
            rows.append({"bench": name, "unit": unit, "mi355x": round(ms, 3), "rtx3090": ref,
                         "x": round(ref / ms, 2), "source": f"benchmarks/results/rtx3090.md:{line}"})
    return rows


# ------------------------------------------------------------ CPU leg --
DECODE_SHAPES = ((1, 32, 32, 4096, 128), (8, 32, 32, 4096, 128), (8, 32, 8, 8192, 128),
                 (16, 12, 12, 1024, 64))


def decode_leg(torch, tritium, calls: int = 50, rotate_bytes: int = 3 << 28):
    """KV-cache decode: ``attention`` with one query row per head against a
    bf16 cache slice (B, H, H_kv, L, D) in ``DECODE_SHAPES``.  Per shape the
    eager time per call (host path included: back-to-back calls) and the time
    per call of the same calls replayed from one captured graph (the kernels
    alone), with GB/s on the K + V bytes the call must read (HBM-bound).  The
    calls rotate over enough copies of the cache (at least ``rotate_bytes``,
    3x the 256 MB last-level cache) that each call reads its K and V from HBM,
    not from a cache the previous call left warm."""
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(0)
    out = []
    for b, h, hkv, L, d in DECODE_SHAPES:
        per_copy = 2 * b * hkv * (L + 512) * d * 2
        n_copies = max(2, -(-rotate_bytes // per_copy))
        caches = []
        for _ in range(n_copies):
            kc = torch.randn((b, hkv, L + 512, d), generator=g, device=dev).to(torch.bfloat16)
            vc = torch.randn((b, hkv, L + 512, d), generator=g, device=dev).to(torch.bfloat16)
            caches.append((kc[:, :, :L], vc[:, :, :L]))
        q = torch.randn((b, h, 1, d), generator=g, device=dev).to(torch.bfloat16)

        def fn(i):
            k, v = caches[i % n_copies]
            return tritium.attention(q, k, v, is_causal=False)

        for i in range(5):
            fn(i)
        ref = [fn(i) for i in range(n_copies)]
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(calls):
            fn(i)
        e.record()
        torch.cuda.synchronize()
        eager_us = s.elapsed_time(e) / calls * 1e3
        nbytes = 2 * b * hkv * L * d * 2
        row = {"shape": [b, h, hkv, L, d], "kv_bytes": nbytes, "cache_copies": n_copies,
               "eager_us": round(eager_us, 1)}
        try:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                for i in range(3):
                    fn(i)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                got = [fn(i) for i in range(calls)]
            for _ in range(2):
                graph.replay()
            torch.cuda.synchronize()
            row["graph_matches_eager"] = bool(all(torch.equal(got[i], ref[i % n_copies])
                                                  for i in range(calls)))
            reps = 5
            s.record()
            for _ in range(reps):
                graph.replay()
            e.record()
            torch.cuda.synchronize()
            us = s.elapsed_time(e) / (reps * calls) * 1e3
            row.update({"graph_us": round(us, 1), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                        "frac_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
            del graph, got
        except RuntimeError as exc:  # capture refused: report the eager figure only
            row["graph_error"] = str(exc)[:200]
        out.append(row)
        del caches, ref
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def gpt_leg(torch, steps: int = 10, warmup: int = 3):
    """Config 5: the 151.9M-parameter GPT (12 x 768, SwiGLU 3072, vocab 50304, tied
    embeddings) training step at B=16 x T=1024 on the kernel layer: bf16 compute,
    fp32 master weights, fused AdamW; random-init weights, uniform random tokens."""
    from helion_amd import gpt

    cfg, tc = gpt.GPTConfig(), gpt.TrainConfig()
    model = gpt.HipGPT(cfg, tc, gpt.init_params(cfg, tc.seed), torch.device("cuda"))
    res = gpt.time_steps(model, cfg, tc, steps, warmup)
    del model
    torch.cuda.empty_cache()
    return {"tokens_per_s": round(res["tokens_per_s"], 1), "ms_per_step": round(res["ms_per_step"], 3),
            "mfu_vs_2.5PF": round(res["mfu"], 4), "loss": round(res["loss"], 4),
            "params": gpt.n_params(cfg), "tokens_per_step": tc.batch * tc.seq_len}


def cpu_baseline(budget_s: float = 12.0):
    """The reference's PyTorch formulas on this host's cores, over a bounded
    sample of the headline workload (1/4 of every op), in the same unit."""
    import torch

    from oracle import torch_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    frac = 4
    n_rows = ROWS_B * ROWS_T // frac
    x = torch.randn((n_rows, ROWS_D), generator=g).bfloat16()
    w = (1 + 0.02 * torch.randn((ROWS_D,), generator=g)).bfloat16()
    dy = torch.randn((n_rows, ROWS_D), generator=g).bfloat16()
    q = torch.randn((n_rows, ROPE_H, ROPE_HD), generator=g).bfloat16()
    k = torch.randn((n_rows, ROPE_H, ROPE_HD), generator=g).bfloat16()
    cos, sin = torch_ref.make_cos_sin(ROWS_T, ROPE_HD)
    pos = torch.arange(ROWS_T).repeat(ROWS_B)[:n_rows]
    sx = torch.randn((n_rows, SWIGLU_F), generator=g).bfloat16()
    sg = torch.randn((n_rows, SWIGLU_F), generator=g).bfloat16()
    sdy = torch.randn((n_rows, SWIGLU_F), generator=g).bfloat16()
    shapes = [(max(1, math.prod(s) // frac),) for s in gpt2_small_shapes()]
    params = [0.02 * torch.randn(s, generator=g) for s in shapes]
    grads = [1e-2 * torch.randn(s, generator=g) for s in shapes]
    ps = [p.clone().requires_grad_(True) for p in params]
    opt = torch.optim.AdamW(ps, lr=ADAMW_HP["lr"], betas=(ADAMW_HP["beta1"], ADAMW_HP["beta2"]),
                            eps=ADAMW_HP["eps"], weight_decay=ADAMW_HP["weight_decay"],
                            foreach=False)
    n_params = sum(p.numel() for p in params)

    def one():
        y = torch_ref.rmsnorm(x, w, 1e-6).bfloat16()
        dx, dw = torch_ref.rmsnorm_backward(dy, x, w, 1e-6)
        qo, ko = torch_ref.rope(q, k, cos, sin, pos)
        dq_, dk_ = torch_ref.rope(qo.bfloat16(), ko.bfloat16(), cos, sin, pos, inverse=True)
        torch_ref.swiglu_fwd_bwd(sx, sg, sdy)
        for p, gr in zip(ps, grads):
            p.grad = gr
        opt.step()
        return y, dx, dw, dq_, dk_

    one()  # warmup
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or (time.perf_counter() - t_start < budget_s and len(times) < 30):
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > 3 * budget_s:
            break
    times.sort()
    med = times[len(times) // 2]
    nbytes = (sum(rmsnorm_bytes(n_rows, ROWS_D)) + sum(rope_bytes(n_rows, ROPE_H, ROPE_HD, ROWS_T))
              + sum(swiglu_bytes(n_rows * SWIGLU_F)) + adamw_bytes(n_params))
    model = _cpu_model()
    return {
        "value": round(nbytes / med / 1e9, 3),
        "unit": "GB/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"1/{frac} of the headline workload: RMSNorm+RoPE+SwiGLU fwd+bwd on "
                   f"{n_rows} of {ROWS_B * ROWS_T} rows and torch.optim.AdamW(foreach=False) "
                   f"over {n_params} params (148 tensors at 1/{frac} size); fp32 math as the "
                   f"reference's test formulas; median of {len(times)} runs ({med:.3f} s each)"),
        "cpu_model": model,
    }


def config1_cpu(torch=None, tritium=None, budget_s: float = 5.0):
    """Config 1: RMSNorm fwd+bwd on the reference's PyTorch formulas on this host's
    cores (tests/tritium/test_rmsnorm.py:12-48, restated in oracle/torch_ref.py):
    x [4096, 768] fp32 ~N(0,1), w = 1 + 0.02 N(0,1), eps 1e-6, dy ~N(0,1), drawn in
    that order from a CPU generator seeded 0.  Produces y, dx and dw; their time
    (median after a warm-up run) and checksums, and, when a GPU is given, the
    max-abs difference of this library's kernels on the same inputs."""
    import torch as _torch

    from oracle import torch_ref

    cores = len(os.sched_getaffinity(0))
    _torch.set_num_threads(cores)
    g = _torch.Generator().manual_seed(0)
    n, d, eps = 4096, 768, 1e-6
    x = _torch.randn((n, d), generator=g)
    w = 1 + 0.02 * _torch.randn((d,), generator=g)
    dy = _torch.randn((n, d), generator=g)
    out = {}

    def one():
        out["y"] = torch_ref.rmsnorm(x, w, eps)
        out["dx"], out["dw"] = torch_ref.rmsnorm_backward(dy, x, w, eps)

    med, runs = _time_cpu(one, budget_s, min_runs=3, max_runs=50)
    fwd, bwd = rmsnorm_bytes(n, d, esz=4)
    res = {
        "workload": "RMSNorm fwd+bwd, x [4096,768] fp32, w = 1+N(0,0.02), eps 1e-6, seed 0",
        "ms": round(med * 1e3, 3),
        "GB/s": round((fwd + bwd) / med / 1e9, 3),
        "runs": runs,
        "cores": cores,
        "cpu_model": _cpu_model(),
        "kind": "port",
        "checksums": {k: round(float(v.double().sum()), 6) for k, v in out.items()},
    }
    if torch is not None and tritium is not None and torch.cuda.is_available():
        xg = x.cuda().requires_grad_(True)
        wg = w.cuda().requires_grad_(True)
        yg = tritium.rmsnorm(xg, wg, eps)
        yg.backward(dy.cuda())
        res["max_abs_diff_vs_hip"] = {
            "y": float((yg.detach().cpu() - out["y"]).abs().max()),
            "dx": float((xg.grad.cpu() - out["dx"]).abs().max()),
            "dw": float((wg.grad.cpu() - out["dw"]).abs().max()),
        }
    return res


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor()


def _time_cpu(fn, budget_s: float, min_runs: int = 2, max_runs: int = 20):
    """Median wall time of ``fn`` (one untimed warm-up call first)."""
    fn()
    times = []
    t_start = time.perf_counter()
    while len(times) < min_runs or (time.perf_counter() - t_start < budget_s and len(times) < max_runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2], len(times)


def attention_cpu_baseline(budget_s: float = 10.0, t: int = 4096, d: int = 128):
    """The reference's attention formula (SDPA in float32, tests/tritium/
    test_attention.py:9-21) forward+backward on this host's cores over a
    sample of the config-3 workload: n_heads of the 4 x 32 (batch, head)
    slices at T=4096, D=128, in TFLOP/s (the same causal flop convention)."""
    import torch

    from oracle import torch_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    heads = 4
    q, k, v, do = (torch.randn((1, heads, t, d), generator=g) for _ in range(4))
    qs, ks, vs = (x.clone().requires_grad_(True) for x in (q, k, v))

    def one():
        o = torch_ref.attention(qs, ks, vs, is_causal=True)
        o.backward(do)
        qs.grad = ks.grad = vs.grad = None

    med, n = _time_cpu(one, budget_s)
    ff, fb = attention_flops(1, heads, t, d)
    return {"value": round((ff + fb) / med / 1e12, 4), "unit": "TFLOP/s", "cores": cores,
            "kind": "port", "cpu_model": _cpu_model(),
            "sample": (f"{heads} of the 128 (batch, head) slices of config 3 (T={t}, D={d}, causal), "
                       f"fp32 SDPA forward+backward through autograd; median of {n} runs "
                       f"({med:.3f} s each)")}


def lce_cpu_baseline(budget_s: float = 10.0, n_rows: int = 128, d: int = 4096, v: int = 128256):
    """The reference's linear-cross-entropy formula (F.linear then
    F.cross_entropy with ignore_index -100, float32; tests/tritium/
    test_cross_entropy.py:72) forward+backward on this host's cores over
    n_rows of the 8192 config-4 rows, full vocabulary, in TFLOP/s (6NVD)."""
    import torch

    from oracle import torch_ref

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator().manual_seed(0)
    hidden = torch.randn((n_rows, d), generator=g).requires_grad_(True)
    weight = (torch.randn((v, d), generator=g) * 0.02).requires_grad_(True)
    target = torch.randint(0, v, (n_rows,), generator=g)

    def one():
        torch_ref.linear_cross_entropy(hidden, weight, target).backward()
        hidden.grad = weight.grad = None

    med, n = _time_cpu(one, budget_s)
    ff, fb = lce_flops(n_rows, d, v)
    del weight
    return {"value": round((ff + fb) / med / 1e12, 4), "unit": "TFLOP/s", "cores": cores,
            "kind": "port", "cpu_model": _cpu_model(),
            "sample": (f"{n_rows} of the 8192 rows of config 4 (D={d}, V={v}), fp32 "
                       f"F.linear + F.cross_entropy forward+backward through autograd; "
                       f"median of {n} runs ({med:.3f} s each)")}


def gpt_cpu_baseline(budget_s: float = 10.0):
    """The config-5 training step as plain PyTorch (gpt.TorchTwin: the same
    model, bf16 matmuls, fp32 master weights and torch.optim.AdamW) on this
    host's cores, batch 1 x 1024 tokens instead of 16 x 1024, in tokens/s."""
    import dataclasses

    import torch

    from helion_amd import gpt

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    cfg = gpt.GPTConfig()
    tc = dataclasses.replace(gpt.TrainConfig(), batch=1)
    twin = gpt.TorchTwin(cfg, tc, gpt.init_params(cfg, tc.seed), torch.device("cpu"))
    gen = torch.Generator().manual_seed(1)
    tokens, targets = gpt.lm_batch(cfg, tc, gen, torch.device("cpu"))
    med, n = _time_cpu(lambda: twin.train_step(tokens, targets), budget_s, min_runs=1, max_runs=5)
    del twin
    ntok = tc.batch * tc.seq_len
    return {"value": round(ntok / med, 1), "unit": "tokens/s", "cores": cores, "kind": "port",
            "cpu_model": _cpu_model(),
            "sample": (f"1 x {tc.seq_len} tokens of the 16 x {tc.seq_len} config-5 batch, one "
                       f"TorchTwin training step (forward, backward, AdamW); median of {n} "
                       f"steps ({med:.2f} s each)")}


def _profile_figure(name: str, key: str):
    """A number recorded in profiles/NAME as a line ``KEY: value`` (None if absent)."""
    path = os.path.join(ROOT, "profiles", name)
    if not os.path.exists(path):
        return None
    with open(path) as f:
        for line in f:
            if line.startswith(key + ":"):
                return int(float(line.split(":", 1)[1].split()[0]))
    return None


def mfma_roofline(kernels: str, flops: float, ms: float, counters: str) -> dict:
    """Roofline object of an MFMA-bound leg: algorithmic flops of one pass over
    its time measured here, and the HBM bytes one pass moves as the counter
    summary in profiles/COUNTERS records them."""
    achieved = flops / (ms * 1e-3) / 1e12
    return {"kernels": kernels, "bound": "mfma", "achieved": round(achieved, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": _profile_figure(counters, "traffic_bytes_per_pass"),
            "algorithmic_flops_per_pass": flops, "counters": f"profiles/{counters}"}



def stream_probe(torch, tritium, reps: int = 10):
    """GB/s of plain HBM streaming patterns (``helion_amd/probe/stream_probe.hip``,
    its own library ``libtritium_probe.so``; nontemporal 16-byte accesses): read,
    copy and fill of 1 GiB as persistent grids of 2048-16384 workgroups (4 vectors
    per lane in flight) and as grid-covering launches (one vector per lane), two
    streams read and one written (the RMSNorm-backward shape), and the AdamW-shaped
    in-place update over 124,439,808 fp32 elements (4 streams read, 3 written).
    Median of ``reps`` event-timed launches after one warm-up."""
    import ctypes
    import statistics

    from helion_amd import _build, _lib

    _lib.lib()  # binds torch's HIP runtime first, as every library call does
    if not os.path.exists(_build.PROBE_PATH):
        raise RuntimeError(f"{_build.PROBE_PATH} is not built (python -m helion_amd._build)")
    probe = ctypes.CDLL(_build.PROBE_PATH)
    probe.tritium_stream_probe.restype = ctypes.c_int
    probe.tritium_stream_probe.argtypes = [ctypes.c_int] + [ctypes.c_void_p] * 4 + [
        ctypes.c_int64, ctypes.c_int, ctypes.c_void_p]
    probe.tritium_probe_last_error.restype = ctypes.c_char_p

    dev = torch.device("cuda")
    n = 1 << 26  # 16-byte vectors: 1 GiB
    a = torch.ones(n * 4, device=dev)
    b = torch.empty(n * 4, device=dev)
    c = torch.empty(n * 4, device=dev)
    sink = torch.zeros(256, device=dev)
    npar = 124439808 // 4 * 4
    p, g, m, v = (torch.rand(npar, device=dev) for _ in range(4))
    persistent = (2048, 4096, 8192, 16384)
    cases = [("read 1 GiB, persistent", 0, (a, sink, None, None), n, 1 << 30, persistent),
             ("copy 1 GiB, persistent", 1, (a, b, None, None), n, 2 << 30, persistent),
             ("fill 1 GiB, persistent", 2, (b, None, None, None), n, 1 << 30, persistent),
             ("adamw-shaped 4 read + 3 write, persistent", 3, (p, g, m, v), npar // 4,
              28 * npar, persistent),
             ("read 1 GiB, grid-covering", 4, (a, sink, None, None), n, 1 << 30, (0,)),
             ("copy 1 GiB, grid-covering", 5, (a, b, None, None), n, 2 << 30, (0,)),
             ("fill 1 GiB, grid-covering", 6, (b, None, None, None), n, 1 << 30, (0,)),
             ("2 read + 1 write of 1 GiB, grid-covering", 7, (a, b, c, None), n, 3 << 30, (0,)),
             ("adamw-shaped 4 read + 3 write, grid-covering (workgroup lanes)", 8, (p, g, m, v),
              npar // 4, 28 * npar, (64, 256))]
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = []
    for name, pat, bufs, nv, nbytes, grids in cases:
        row = {"pattern": name, "bytes": nbytes}
        for blocks in grids:
            ptrs = [None if x is None else x.data_ptr() for x in bufs]
            times = []
            for _ in range(reps + 1):
                s.record()
                rc = probe.tritium_stream_probe(pat, *ptrs, nv, max(blocks, 1), _lib.stream_of(a))
                if rc != 0:
                    raise RuntimeError(probe.tritium_probe_last_error().decode())
                e.record()
                torch.cuda.synchronize()
                times.append(s.elapsed_time(e))
            ms = statistics.median(times[1:])
            key = (f"GB/s {blocks} lanes" if pat == 8 else f"GB/s b{blocks}") if blocks else "GB/s"
            row[key] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        row["best_frac_of_8TB/s"] = round(max(vv for k, vv in row.items() if k.startswith("GB/s"))
                                          / HBM_PEAK_GBS, 4)
        out.append(row)
    return {"stream_probe": out}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--legs", default="rows,attention,attngpt,lce,gpt,refbench,decode",
                    help="comma list of rows,attention,attngpt,lce,gpt,refbench,decode (rows is "
                         "the headline; attngpt is attention at the GPT block's shape; refbench "
                         "reruns the reference's published benchmark rows)")
    ap.add_argument("--stream-probe", action="store_true",
                    help="only time the HBM streaming probes (read, copy, fill, AdamW-shaped "
                         "update; tritium_stream_probe) that set the row kernels' ceilings")
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device copy 5 times (calibrates the HBM "
                         "byte counters of a profiler against a kernel of known traffic)")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path "
              f"(--gpus {args.gpus} requested). Run with --gpus 1.", file=sys.stderr)
        return 2

    import torch

    import helion_amd as tritium

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    tritium._lib.lib()  # fail loudly if the HIP library is missing
    legs = set(args.legs.split(","))
    if args.copy_probe:
        src = torch.ones(1 << 28, device="cuda")  # 1 GiB fp32
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes_read": src.numel() * 4,
                          "copy_probe_bytes_written": dst.numel() * 4, "launches": 5}))
        return 0

    if args.stream_probe:
        print(json.dumps(stream_probe(torch, tritium)))
        return 0

    ops: dict = {}
    if "rows" not in legs:
        # profiling runs of a single leg: no headline line
        if "attention" in legs:
            ops["attention_fwd_bwd"] = attention_leg(torch, tritium, iters=args.steps,
                                                     warmup=args.warmup)
        if "attngpt" in legs:
            ops["attention_gpt_shape"] = attention_gpt_leg(torch, tritium, iters=args.steps,
                                                           warmup=args.warmup)
        if "lce" in legs:
            ops["linear_ce_fwd_bwd"] = lce_leg(torch, tritium, iters=args.steps,
                                               warmup=args.warmup)
        if "gpt" in legs:
            ops["gpt_train_step"] = gpt_leg(torch, steps=args.steps, warmup=args.warmup)
        if "refbench" in legs:
            ops["reference_benchmarks"] = ref_bench_leg(torch, tritium)
        if "decode" in legs:
            ops["attention_decode"] = decode_leg(torch, tritium)
        print(json.dumps({"metric": METRIC, "partial": True, "ops": ops}), flush=True)
        return 0
    rows = row_leg(torch, tritium, args.steps, args.warmup)
    print(f"[bench] rows: {rows['ms_per_step']:.3f} ms/step", file=sys.stderr, flush=True)
    ops.update(rows["ops"])
    if "attention" in legs:
        ops["attention_fwd_bwd"] = attention_leg(torch, tritium)
        print(f"[bench] attention: {ops['attention_fwd_bwd']}", file=sys.stderr, flush=True)
    if "attngpt" in legs:
        ops["attention_gpt_shape"] = attention_gpt_leg(torch, tritium)
        print(f"[bench] attention (GPT shape): {ops['attention_gpt_shape']}", file=sys.stderr,
              flush=True)
    if "lce" in legs:
        res = lce_leg(torch, tritium)
        if res is not None:
            ops["linear_ce_fwd_bwd"] = res
            print(f"[bench] linear-ce: {res}", file=sys.stderr, flush=True)
    if "gpt" in legs:
        ops["gpt_train_step"] = gpt_leg(torch)
        print(f"[bench] gpt: {ops['gpt_train_step']}", file=sys.stderr, flush=True)
    if "refbench" in legs:
        ops["reference_benchmarks"] = ref_bench_leg(torch, tritium)
        print(f"[bench] reference benchmarks: {ops['reference_benchmarks']}", file=sys.stderr,
              flush=True)
    # after the reference rows: its captured graphs' memory pools would change
    # what the allocator holds for them
    if "decode" in legs:
        ops["attention_decode"] = decode_leg(torch, tritium)
        print(f"[bench] decode: {ops['attention_decode']}", file=sys.stderr, flush=True)

    adamw_gbs = rows["adamw_bytes"] / (rows["adamw_ms"] * 1e-3) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "row_ops_config2_traffic.txt")
    if os.path.exists(tpath):
        with open(tpath) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    traffic = int(float(line.split(":", 1)[1]))
    roofline = {
        "kernel": "adamw_multi_kernel (fused AdamW, 148 tensors, one launch)",
        "bound": "hbm",
        "achieved": round(adamw_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(adamw_gbs / HBM_PEAK_GBS, 4),
        "traffic": traffic,
        "algorithmic_bytes_per_launch": rows["adamw_bytes"],
    }
    cpu = None if args.no_cpu else cpu_baseline()
    cpu_config1 = None if args.no_cpu else config1_cpu(torch, tritium)
    if not args.no_cpu:
        # the other legs' reference PyTorch paths on the same host cores
        for key, fn in (("attention_fwd_bwd", attention_cpu_baseline),
                        ("linear_ce_fwd_bwd", lce_cpu_baseline),
                        ("gpt_train_step", gpt_cpu_baseline)):
            if isinstance(ops.get(key), dict):
                ops[key]["cpu_baseline"] = fn()
                print(f"[bench] cpu {key}: {ops[key]['cpu_baseline']}", file=sys.stderr, flush=True)
    line = {
        "metric": METRIC,
        "value": round(rows["value"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(rows["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) activations; N(0,0.02) params)",
        "config": {
            "workload": ("config2 row ops: RMSNorm+RoPE+SwiGLU fwd+bwd bf16, activations "
                         "[8,2048,4096], RoPE 32x128, SwiGLU [8,2048,11008], + fused AdamW "
                         "over 124,439,808 fp32 params (148 tensors)"),
            "bytes_per_step": rows["total_bytes"],
            "parallelism": "single GPU",
        },
        "frac_hbm_peak": round(rows["value"] / HBM_PEAK_GBS, 4),
        "ops": ops,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_config1": cpu_config1,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

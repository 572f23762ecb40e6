"""``adamw_step`` (one tensor) and ``adamw_step_multi`` (one launch for a list).

``adamw_step`` is a drop-in for alkinun/helion ``tritium/ops/adamw.py:113-151``
(same keyword signature, validation 57-110 and messages, host-side float64
bias corrections 133-134).

``adamw_step_multi`` is new: it replaces the per-parameter Python loop of
``helion.AdamW.step`` (helion/optim.py:50-70) by ONE kernel launch.  The host
builds a small int64 descriptor table (pointers, sizes, dtype, chunk offsets),
copies it to the device through pinned memory without a host sync, and caches
it while the tensors' storage stays the same.

``adamw_step_mixed`` is new too: fp32 params and moments, 16-bit gradients
read as they are, and the 16-bit working weights written in the same pass.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch

from . import _lib
from ._utils import FLOAT_DTYPES, check_contiguous, check_cuda_tensor, check_supported_dtype

SUPPORTED_DTYPES = FLOAT_DTYPES
_DESC_WORDS = 7


def _check_adamw_inputs(param, grad, exp_avg, exp_avg_sq) -> None:
    """adamw.py:57-110."""
    check_cuda_tensor("param", param)
    check_cuda_tensor("grad", grad)
    check_cuda_tensor("exp_avg", exp_avg)
    check_cuda_tensor("exp_avg_sq", exp_avg_sq)
    check_supported_dtype("param", param, SUPPORTED_DTYPES)
    check_supported_dtype("grad", grad, SUPPORTED_DTYPES)
    if param.shape != grad.shape:
        raise ValueError(
            f"Shape mismatch: param has shape {tuple(param.shape)}, "
            f"grad has shape {tuple(grad.shape)}."
        )
    if exp_avg.shape != param.shape:
        raise ValueError(
            f"Shape mismatch: exp_avg has shape {tuple(exp_avg.shape)}, "
            f"expected {tuple(param.shape)}."
        )
    if exp_avg_sq.shape != param.shape:
        raise ValueError(
            f"Shape mismatch: exp_avg_sq has shape {tuple(exp_avg_sq.shape)}, "
            f"expected {tuple(param.shape)}."
        )
    if grad.dtype != param.dtype:
        raise ValueError(
            f"Dtype mismatch: grad has dtype {grad.dtype}, param has dtype {param.dtype}."
        )
    if exp_avg.dtype != torch.float32:
        raise ValueError(f"exp_avg must have dtype float32, got {exp_avg.dtype}.")
    if exp_avg_sq.dtype != torch.float32:
        raise ValueError(f"exp_avg_sq must have dtype float32, got {exp_avg_sq.dtype}.")
    for name, t in (("grad", grad), ("exp_avg", exp_avg), ("exp_avg_sq", exp_avg_sq)):
        if t.device != param.device:
            raise ValueError(
                f"Device mismatch: {name} is on {t.device}, param is on {param.device}."
            )
    check_contiguous("param", param, "for tritium.adamw_step")
    check_contiguous("grad", grad, "for tritium.adamw_step")
    check_contiguous("exp_avg", exp_avg, "for tritium.adamw_step")
    check_contiguous("exp_avg_sq", exp_avg_sq, "for tritium.adamw_step")


def _bias_corrections(beta1: float, beta2: float, step: int) -> tuple[float, float]:
    """adamw.py:133-134 (host float64)."""
    return 1.0 - beta1**step, 1.0 - beta2**step


def adamw_step(
    param: torch.Tensor,
    grad: torch.Tensor,
    exp_avg: torch.Tensor,
    exp_avg_sq: torch.Tensor,
    *,
    lr: float,
    beta1: float = 0.9,
    beta2: float = 0.999,
    eps: float = 1e-8,
    weight_decay: float = 0.01,
    step: int = 1,
) -> None:
    """Update ``param`` in-place with AdamW using fp32 moments (adamw.py:113-151)."""
    _check_adamw_inputs(param, grad, exp_avg, exp_avg_sq)
    n = param.numel()
    if n == 0:
        return
    bc1, bc2 = _bias_corrections(beta1, beta2, step)
    _lib.call(
        "tritium_adamw_step",
        param.data_ptr(),
        grad.data_ptr(),
        exp_avg.data_ptr(),
        exp_avg_sq.data_ptr(),
        n,
        float(lr),
        float(beta1),
        float(beta2),
        float(eps),
        float(weight_decay),
        bc1,
        bc2,
        _lib.dtype_code(param.dtype),
        _lib.stream_of(param),
    )


class _TableCache:
    """Device descriptor tables keyed by the storage they describe."""

    def __init__(self, capacity: int = 8) -> None:
        self.capacity = capacity
        self.entries: dict[tuple, tuple[torch.Tensor, int, int]] = {}

    def get(self, key: tuple):
        return self.entries.get(key)

    def put(self, key: tuple, value) -> None:
        if len(self.entries) >= self.capacity:
            self.entries.pop(next(iter(self.entries)))
        self.entries[key] = value


_tables = _TableCache()


def _signature(t: torch.Tensor) -> tuple:
    """Everything the checks of :func:`_check_adamw_inputs` and the kernel's
    addressing depend on (storage address, shape, dtype, contiguity; the
    device is the first parameter's, in the table key): a cache hit then means
    the same checks would pass."""
    return (t.data_ptr(), t.shape, t.dtype, t.is_contiguous())


def _table_key(params, grads, exp_avgs, exp_avg_sqs) -> tuple:
    # one flat tuple, four accessor calls per tensor: with hundreds of tensors
    # the key is host time on every step (2.4x less than per-tensor tuples of
    # (address, dtype, device, shape, strides), measured on the host)
    key = [params[0].device]
    for ts in (params, grads, exp_avgs, exp_avg_sqs):
        key.extend([(t.data_ptr(), t.shape, t.dtype, t.is_contiguous()) for t in ts])
    return tuple(key)


def _table_for(params, grads, exp_avgs, exp_avg_sqs):
    key = _table_key(params, grads, exp_avgs, exp_avg_sqs)
    hit = _tables.get(key)
    if hit is not None:
        return hit
    for p, g, m, v in zip(params, grads, exp_avgs, exp_avg_sqs):
        _check_adamw_inputs(p, g, m, v)
    device = params[0].device
    for p in params:
        if p.device != device:
            raise ValueError(
                f"Device mismatch: all params must be on {device}, got {p.device}."
            )
    chunk = int(_lib.lib().tritium_adamw_chunk_elements())
    rows = []
    first = 0
    for p, g, m, v in zip(params, grads, exp_avgs, exp_avg_sqs):
        n = p.numel()
        if n == 0:
            continue
        ptrs = (p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr())
        aligned = all(x % 16 == 0 for x in ptrs)
        rows.extend(ptrs)
        rows.extend((n, _lib.dtype_code(p.dtype) | (int(aligned) << 8), first))
        first += -(-n // chunk)
    n_tensors = len(rows) // _DESC_WORDS
    host = torch.tensor(rows if rows else [0], dtype=torch.int64).pin_memory()
    table = host.to(params[0].device, non_blocking=True)
    entry = (table, n_tensors, first)
    _tables.put(key, entry)
    return entry


def adamw_step_multi(
    params: Sequence[torch.Tensor],
    grads: Sequence[torch.Tensor],
    exp_avgs: Sequence[torch.Tensor],
    exp_avg_sqs: Sequence[torch.Tensor],
    *,
    lr: float,
    beta1: float = 0.9,
    beta2: float = 0.999,
    eps: float = 1e-8,
    weight_decay: float = 0.01,
    step: int = 1,
) -> None:
    """AdamW on every ``params[i]`` in ONE kernel launch.

    Per tensor the arithmetic and checks are those of :func:`adamw_step`;
    all tensors must be on one device.  The checks run whenever any tensor's
    storage address, dtype, device, shape or strides differ from a cached
    descriptor table's.
    """
    if not (len(params) == len(grads) == len(exp_avgs) == len(exp_avg_sqs)):
        raise ValueError(
            "params, grads, exp_avgs and exp_avg_sqs must have the same length, got "
            f"{len(params)}, {len(grads)}, {len(exp_avgs)}, {len(exp_avg_sqs)}."
        )
    if len(params) == 0:
        return
    table, n_tensors, total_chunks = _table_for(params, grads, exp_avgs, exp_avg_sqs)
    if n_tensors == 0:
        return
    bc1, bc2 = _bias_corrections(beta1, beta2, step)
    _lib.call(
        "tritium_adamw_step_multi",
        table.data_ptr(),
        n_tensors,
        total_chunks,
        float(lr),
        float(beta1),
        float(beta2),
        float(eps),
        float(weight_decay),
        bc1,
        bc2,
        _lib.stream_of(params[0]),
    )


def adamw_step_mixed(
    params: Sequence[torch.Tensor],
    grads: Sequence[torch.Tensor],
    exp_avgs: Sequence[torch.Tensor],
    exp_avg_sqs: Sequence[torch.Tensor],
    shadows: Sequence[torch.Tensor] | None = None,
    *,
    lr: float,
    beta1: float = 0.9,
    beta2: float = 0.999,
    eps: float = 1e-8,
    weight_decay: float = 0.01,
    step: int = 1,
) -> None:
    """Mixed-precision AdamW over a parameter list in one launch
    (``tritium_adamw_step_mixed``): fp32 ``params`` and moments updated from
    16-bit ``grads`` read as they are, and, when ``shadows`` is given, each
    updated parameter rounded into the matching 16-bit tensor in the same
    pass.  The arithmetic is :func:`adamw_step`'s on the widened gradient.
    Not part of the reference's surface (its ``adamw_step`` wants grad and
    param of one dtype, adamw.py:86-90): a training step with 16-bit working
    weights over fp32 masters uses it instead of widening every gradient and
    re-rounding every weight in two extra passes."""
    n = len(params)
    lists = [grads, exp_avgs, exp_avg_sqs] + ([shadows] if shadows is not None else [])
    if any(len(x) != n for x in lists):
        raise ValueError("params, grads, exp_avgs, exp_avg_sqs (and shadows) must have the same length.")
    if n == 0:
        return
    gdt = grads[0].dtype
    if gdt not in (torch.float16, torch.bfloat16):
        raise ValueError(f"grads must be float16 or bfloat16, got {gdt}.")
    device = params[0].device
    check_cuda_tensor("param", params[0])
    dev_index = params[0].get_device()
    chunk = int(_lib.lib().tritium_adamw_mixed_chunk_elements())
    f32 = torch.float32
    sh_list = shadows if shadows is not None else [None] * n
    # every tensor of a model passes through here once per step, and this
    # host time sits between the backward's last kernel and the update: the
    # common case is checked in bulk, the per-tensor loop below only runs to
    # name the first bad tensor
    def good(ts, dt):
        return all(t.is_cuda and t.dtype is dt and t.get_device() == dev_index and t.is_contiguous()
                   for t in ts)

    fast = (good(params, f32) and good(exp_avgs, f32) and good(exp_avg_sqs, f32) and good(grads, gdt)
            and (shadows is None or good(shadows, gdt))
            and all(p.shape == g.shape == m.shape == v.shape
                    for p, g, m, v in zip(params, grads, exp_avgs, exp_avg_sqs))
            and (shadows is None or all(p.shape == s.shape for p, s in zip(params, shadows))))
    if not fast:
        for i in range(n):
            p, sh = params[i], sh_list[i]
            for name, t, dt in (("param", p, f32), ("grad", grads[i], gdt), ("exp_avg", exp_avgs[i], f32),
                                ("exp_avg_sq", exp_avg_sqs[i], f32)) + ((("shadow", sh, gdt),) if sh is not None else ()):
                check_cuda_tensor(name, t)
                if t.dtype != dt:
                    raise ValueError(f"{name} must have dtype {dt}, got {t.dtype}.")
                if t.shape != p.shape:
                    raise ValueError(f"Shape mismatch: {name} has shape {tuple(t.shape)}, "
                                     f"param has shape {tuple(p.shape)}.")
                if t.device != device:
                    raise ValueError(f"Device mismatch: {name} is on {t.device}, expected {device}.")
                check_contiguous(name, t, "for tritium.adamw_step_mixed")
    rows: list[int] = []
    first = 0
    for p, g, m, v, sh in zip(params, grads, exp_avgs, exp_avg_sqs, sh_list):
        numel = p.numel()
        if numel == 0:
            continue
        pp, gp, mp, vp = p.data_ptr(), g.data_ptr(), m.data_ptr(), v.data_ptr()
        sp = sh.data_ptr() if sh is not None else 0
        aligned = ((pp | gp | mp | vp | sp) & 15) == 0
        rows += (pp, gp, mp, vp, numel, int(aligned), first, sp)
        first += -(-numel // chunk)
    if not rows:
        return
    host = torch.tensor(rows, dtype=torch.int64).pin_memory()
    table = host.to(device, non_blocking=True)
    bc1, bc2 = _bias_corrections(beta1, beta2, step)
    _lib.call(
        "tritium_adamw_step_mixed", table.data_ptr(), len(rows) // 8, first, float(lr),
        float(beta1), float(beta2), float(eps), float(weight_decay), bc1, bc2,
        _lib.dtype_code(gdt), _lib.stream_of(params[0]),
    )

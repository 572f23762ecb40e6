"""The no-allocation decode entry (``tritium_attention_decode_noalloc``) against
the allocating one (``tritium_attention_decode``), both called through the C
ABI: two calls in a row, the second smaller, each bitwise equal to the
allocating entry's o and lse (same kernels, same key chunks), and the first
call's larger partials in the shared scratch do not leak into the second.
An oversized request is rejected before any device work."""

from __future__ import annotations

import ctypes

import pytest
import torch

import helion_amd._lib as L
from _helpers import randn
from helion_amd.attention import _strides


def _decode_both(dtype, b, h, hkv, kv_len, d, seed):
    print(f"[no-alloc decode] {dtype} b={b} h={h} hkv={hkv} L={kv_len} d={d}", flush=True)
    cache_k = randn((b, hkv, kv_len + 24, d), dtype, seed)
    cache_v = randn((b, hkv, kv_len + 24, d), dtype, seed + 1)
    k, v = cache_k[:, :, :kv_len], cache_v[:, :, :kv_len]
    q = randn((b, 1, h, d), dtype, seed + 2).transpose(1, 2)  # the module's layout
    outs = []
    for noalloc in (False, True):
        o = torch.full((b, h, 1, d), float("nan"), device="cuda", dtype=dtype)
        lse = torch.full((b, h, 1), float("nan"), device="cuda", dtype=torch.float32)
        strides = _strides(q, k, v, o)
        stream = L.stream_of(q)
        if noalloc:
            L.call("tritium_attention_decode_noalloc", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                   o.data_ptr(), lse.data_ptr(), b, h, hkv, kv_len, d, strides,
                   L.dtype_code(dtype), stream)
        else:
            ws_bytes = L.lib().tritium_attention_decode_workspace_size(b, h, hkv, kv_len, d)
            ws = torch.empty((max(ws_bytes, 4) // 4,), device="cuda", dtype=torch.float32)
            L.call("tritium_attention_decode", q.data_ptr(), k.data_ptr(), v.data_ptr(),
                   o.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws_bytes, b, h, hkv, kv_len, d,
                   strides, L.dtype_code(dtype), stream)
        torch.cuda.synchronize()
        outs.append((o, lse))
    (o_ref, lse_ref), (o_new, lse_new) = outs
    assert torch.isfinite(o_ref).all() and torch.isfinite(lse_ref).all()
    assert torch.equal(o_new, o_ref), "o differs from tritium_attention_decode"
    assert torch.equal(lse_new, lse_ref), "lse differs from tritium_attention_decode"


@pytest.mark.gpu
def test_noalloc_decode_matches_allocating_entry_on_two_calls():
    # first call: GQA group 4, many key chunks (large partials); second: smaller,
    # another dtype and head_dim, fewer chunks, so stale rows of the first call
    # sit in the scratch beyond what the second one writes
    _decode_both(torch.bfloat16, 4, 32, 8, 3000, 128, seed=11)
    _decode_both(torch.float16, 2, 8, 8, 700, 64, seed=21)


def test_noalloc_decode_rejects_beyond_its_scratch():
    # 65536 (batch, head) rows of one chunk each: 65536 * (128 + 2) * 4 bytes
    # of partials > 32 MiB; rejected before any pointer is used
    handle = L.lib()
    cap = handle.tritium_attention_decode_noalloc_max_bytes()
    assert cap == 32 << 20
    need = handle.tritium_attention_decode_workspace_size(512, 128, 128, 1, 128)
    assert need > cap
    strides = (ctypes.c_int64 * 12)(*([0] * 12))
    rc = handle.tritium_attention_decode_noalloc(None, None, None, None, None, 512, 128, 128, 1,
                                                 128, strides, 2, None)
    assert rc == 1
    assert b"scratch" in handle.tritium_last_error()

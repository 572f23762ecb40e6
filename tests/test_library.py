"""CPU checks of the C-ABI library: it loads, binds to torch's HIP runtime and
exports every entry point declared in include/tritium_hip.h (no kernel runs)."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

import helion_amd._lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tritium_hip.h")


def _declared_symbols() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tritium_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_what_the_loader_binds():
    assert _declared_symbols() == sorted(L.SIGNATURES)


@pytest.mark.skipif(not os.path.exists(L.LIB_PATH), reason="library not built")
def test_library_exports_every_declared_symbol():
    raw = ctypes.CDLL(L.LIB_PATH)
    for name in _declared_symbols():
        assert hasattr(raw, name), name
    handle = L.lib()
    assert handle.tritium_abi_version() == L.ABI_VERSION
    assert len(L.hip_runtime_paths()) == 1


@pytest.mark.skipif(not os.path.exists(L.LIB_PATH), reason="library not built")
def test_argument_errors_come_back_as_messages():
    handle = L.lib()
    # rejected before any device work: odd head_dim
    rc = handle.tritium_rope(None, None, None, None, None, 0, None, None, 4, 1, 3, 8, 0, 0, 0,
                             0, 0, None)
    assert rc == 1
    assert b"head_dim" in handle.tritium_last_error()
    with pytest.raises(RuntimeError, match="unsupported dtype"):
        L.call("tritium_swiglu_fwd", None, None, None, 16, 7, None)


@pytest.mark.skipif(not os.path.exists(L.LIB_PATH), reason="library not built")
def test_attention_bwd_workspace_size_and_rejection():
    handle = L.lib()
    size = handle.tritium_attention_bwd_workspace_size
    # causal: query tile i sees min(i + 1, n_kv) 64 x 64 chunks of 2-byte dS
    bf16, f16, f32 = 2, 1, 0
    assert size(4, 32, 4096, 4096, 128, 1, bf16) == 4 * 32 * (64 * 65 // 2) * 8192
    assert size(1, 2, 200, 50, 128, 1, bf16) == 2 * (1 + 1 + 1 + 1) * 8192
    assert size(1, 2, 50, 200, 128, 1, bf16) == 2 * 1 * 8192
    assert size(1, 2, 129, 127, 128, 0, f16) == 2 * 3 * 2 * 8192
    assert size(1, 2, 128, 128, 64, 1, bf16) == 0   # head_dim 64: no stored dS
    assert size(1, 2, 128, 128, 128, 1, f32) == 0
    # an undersized workspace is rejected before any device work
    strides = (ctypes.c_int64 * 24)(*([128] * 24))
    p = ctypes.c_void_p(1 << 20)
    rc = handle.tritium_attention_bwd_ws(p, p, p, p, p, p, p, p, p, p, p, 8192, 1, 2, 2, 128, 128,
                                         128, strides, 1, bf16, None)
    assert rc == 1
    assert b"dS workspace" in handle.tritium_last_error()


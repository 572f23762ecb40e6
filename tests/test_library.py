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

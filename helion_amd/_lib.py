"""Loader for ``libtritium_hip.so`` (the gfx950 kernel library, C ABI).

Replaces the reference's import-time Triton shim (alkinun/helion
``tritium/_compat.py:1-34``): instead of patching a JIT compiler, importing an
op binds the prebuilt HIP library once, under a lock, and checks that

* its ABI version matches ``include/tritium_hip.h``;
* it shares torch's HIP runtime (torch ships its own ``libamdhip64.so`` with
  the same soname as ROCm's; loading this library after torch makes the
  dynamic linker reuse torch's copy, so streams and device pointers are
  interchangeable).  Two runtimes in one process is a hard error.

There is no fallback: if the library is missing the first kernel call raises
``RuntimeError`` telling how to build it.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_NAME = "libtritium_hip.so"
# TRITIUM_HIP_LIB selects another build of the same library (e.g. a variant
# tile configuration built with `python -m helion_amd._build --out ... -D ...`).
LIB_PATH = os.environ.get("TRITIUM_HIP_LIB") or os.path.join(
    os.path.dirname(os.path.abspath(__file__)), LIB_NAME
)
ABI_VERSION = 1

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_F64 = ctypes.c_double
_SZ = ctypes.c_size_t

# symbol -> (restype, argtypes); every symbol declared in include/tritium_hip.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "tritium_last_error": (ctypes.c_char_p, []),
    "tritium_abi_version": (_I32, []),
    "tritium_runtime_version": (_I32, []),
    "tritium_rmsnorm_fwd": (_I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _F32, _I32, _P]),
    "tritium_rmsnorm_bwd_workspace_size": (_SZ, [_I64, _I64]),
    "tritium_rmsnorm_bwd": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _F32, _I32, _P],
    ),
    "tritium_rope": (
        _I32,
        [_P, _P, _P, _P, _P, _I32, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I32,
         _I32, _P],
    ),
    "tritium_rope_strided": (
        _I32,
        [_P, _P, _P, _P, _P, _I32, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, _I64, _I64,
         _I32, _I32, _P],
    ),
    "tritium_swiglu_fwd": (_I32, [_P, _P, _P, _I64, _I32, _P]),
    "tritium_swiglu_bwd": (_I32, [_P, _P, _P, _P, _P, _I64, _I32, _P]),
    "tritium_swiglu_rows_fwd": (_I32, [_P, _P, _P, _I64, _I64, _I64, _I64, _I32, _P]),
    "tritium_swiglu_rows_bwd": (
        _I32, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I32, _P],
    ),
    "tritium_adamw_step": (
        _I32,
        [_P, _P, _P, _P, _I64, _F32, _F32, _F32, _F32, _F32, _F64, _F64, _I32, _P],
    ),
    "tritium_adamw_chunk_elements": (_I64, []),
    "tritium_adamw_mixed_chunk_elements": (_I64, []),
    "tritium_attention_fwd": (
        _I32,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I32, _I32, _P],
    ),
    "tritium_attention_bwd": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P,
         _I32, _I32, _P],
    ),
    "tritium_attention_bwd_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _I64, _I32, _I32]),
    "tritium_attention_bwd_ws": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64, _I64, _P,
         _I32, _I32, _P],
    ),
    "tritium_attention_fwd_rope": (
        _I32,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P, _I32, _I32,
         _P, _P, _P, _I32, _I64, _P],
    ),
    "tritium_attention_bwd_rope": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _P,
         _I32, _I32, _P, _P, _P, _I32, _I64, _P],
    ),
    "tritium_attention_bwd_rope_ws": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64, _I64,
         _P, _I32, _I32, _P, _P, _P, _I32, _I64, _P],
    ),
    "tritium_attention_decode_workspace_size": (_SZ, [_I64, _I64, _I64, _I64, _I64]),
    "tritium_attention_decode": (
        _I32,
        [_P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I64, _P, _I32, _P],
    ),
    "tritium_attention_decode_noalloc_max_bytes": (_SZ, []),
    "tritium_attention_decode_noalloc": (
        _I32,
        [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _I32, _P],
    ),
    "tritium_embedding_bwd_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "tritium_embedding_bwd": (
        _I32, [_P, _I32, _I64, _P, _I64, _P, _P, _I64, _I64, _P, _SZ, _I32, _P],
    ),
    "tritium_linear_ce_fwd_workspace_size": (_SZ, [_I64, _I64, _I32]),
    "tritium_linear_ce_fwd": (
        _I32,
        [_P, _P, _P, _I32, _I64, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I32, _P],
    ),
    "tritium_linear_ce_bwd_workspace_size": (_SZ, [_I64, _I64, _I64, _I32, _I32, _I32, _I64]),
    "tritium_linear_ce_bwd": (
        _I32,
        [_P, _P, _P, _P, _I32, _I64, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _I64, _I32, _P],
    ),
    "tritium_adamw_step_multi": (
        _I32,
        [_P, _I32, _I64, _F32, _F32, _F32, _F32, _F32, _F64, _F64, _P],
    ),
    "tritium_cross_entropy_fwd_ws": (_I32, [_P, _P, _I32, _P, _P, _P, _SZ, _I64, _I64, _I32, _P]),
    "tritium_cross_entropy_fwd_workspace_size": (_SZ, [_I64, _I64, _I32]),
    "tritium_cross_entropy_bwd": (
        _I32, [_P, _P, _P, _I32, _P, _P, _I64, _I64, _F64, _I32, _P],
    ),
    "tritium_adamw_step_mixed": (
        _I32,
        [_P, _I32, _I64, _F32, _F32, _F32, _F32, _F32, _F64, _F64, _I32, _P],
    ),
    "tritium_sum_splits": (_I32, [_P, _P, _I64, _I64, _I32, _P]),
    "tritium_linear_ce_grad_logits": (
        _I32,
        [_P, _P, _P, _P, _P, _I32, _I64, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P],
    ),
}

_lock = threading.Lock()
_handle: ctypes.CDLL | None = None


class LibraryNotBuilt(RuntimeError):
    pass


def hip_runtime_paths() -> list[str]:
    """Distinct ``libamdhip64`` files mapped into this process."""
    paths = set()
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                parts = line.split()
                if len(parts) >= 6 and "libamdhip64" in parts[-1]:
                    paths.add(os.path.realpath(parts[-1]))
    except OSError:
        pass
    return sorted(paths)


def _bind(path: str) -> ctypes.CDLL:
    handle = ctypes.CDLL(path, mode=ctypes.RTLD_LOCAL)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = handle.tritium_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(
            f"{path} has ABI version {version}, expected {ABI_VERSION}; rebuild it "
            "with `python -m helion_amd._build`."
        )
    runtimes = hip_runtime_paths()
    if len(runtimes) > 1:
        raise RuntimeError(
            "two HIP runtimes are loaded in this process "
            f"({', '.join(runtimes)}); {LIB_NAME} must bind to torch's."
        )
    return handle


def lib() -> ctypes.CDLL:
    """The bound library (loaded on first use)."""
    global _handle
    if _handle is None:
        with _lock:
            if _handle is None:
                if not os.path.exists(LIB_PATH):
                    raise LibraryNotBuilt(
                        f"{LIB_PATH} is missing: build the HIP kernels with "
                        "`python -m helion_amd._build` (hipcc, gfx950)."
                    )
                _handle = _bind(LIB_PATH)
    return _handle


def call(name: str, *args) -> None:
    """Call an entry point; a nonzero return becomes ``RuntimeError``."""
    handle = lib()
    rc = getattr(handle, name)(*args)
    if rc != 0:
        msg = handle.tritium_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    return DTYPE_CODES[dtype]


# torch's raw current-stream query (what its own C++ extensions use) returns
# the handle without building a Stream object: 0.1 us per call against about
# 2 us for torch.cuda.current_stream(...).cuda_stream
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t: torch.Tensor) -> int:
    """Handle of torch's current stream on ``t``'s device."""
    if _raw_stream is not None and t.is_cuda:
        return _raw_stream(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()

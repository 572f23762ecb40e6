"""Host-side boundary checks that need no GPU: the public names, and the
reference's error contract (tritium/ops/_utils.py:25-78 and each op's own
checks; the reference's rejection tests, e.g. tests/tritium/test_attention.py:110-133,
test_adamw.py:45-58, test_rmsnorm.py and test_cross_entropy.py:112-123).

CPU tensors exercise the "must be a CUDA tensor" path directly.  The later
checks run on shape-only "meta" tensors with the device check patched to
accept them, so every message is reached without touching a GPU.
"""

from __future__ import annotations

import importlib

import pytest
import torch

import helion_amd as tritium
from helion_amd import _utils

# the package re-exports functions named like their modules (rope, swiglu, ...)
adamw_mod = importlib.import_module("helion_amd.adamw")
attn_mod = importlib.import_module("helion_amd.attention")
lce_mod = importlib.import_module("helion_amd.linear_ce")
rms_mod = importlib.import_module("helion_amd.rmsnorm")
rope_mod = importlib.import_module("helion_amd.rope")
swiglu_mod = importlib.import_module("helion_amd.swiglu")

HOT_PATH_NAMES = {
    "adamw_step", "attention", "linear_cross_entropy", "linear_cross_entropy_backward",
    "residual_rmsnorm", "rmsnorm", "rmsnorm_backward", "rope", "rope_", "swiglu",
    "swiglu_backward",
}


def test_public_names_cover_the_hot_path():
    assert HOT_PATH_NAMES <= set(tritium.__all__)
    for name in HOT_PATH_NAMES | {"adamw_step_multi", "matmul", "matmul_vec"}:
        assert callable(getattr(tritium, name))


@pytest.mark.parametrize(
    "call",
    [
        lambda: tritium.rmsnorm(torch.randn(4, 8), torch.ones(8)),
        lambda: tritium.rmsnorm_backward(torch.randn(4, 8), torch.randn(4, 8), torch.ones(8)),
        lambda: tritium.residual_rmsnorm(torch.randn(4, 8), torch.randn(4, 8), torch.ones(8)),
        lambda: tritium.rope(torch.randn(4, 8), torch.randn(4, 8), torch.randn(4, 4), torch.randn(4, 4)),
        lambda: tritium.swiglu(torch.randn(8), torch.randn(8)),
        lambda: tritium.swiglu_backward(torch.randn(8), torch.randn(8), torch.randn(8)),
        lambda: tritium.adamw_step(torch.randn(8), torch.randn(8), torch.zeros(8), torch.zeros(8), lr=1e-3),
        lambda: tritium.attention(*(torch.randn(1, 2, 4, 16) for _ in range(3))),
        lambda: tritium.linear_cross_entropy(torch.randn(4, 8), torch.randn(10, 8), torch.zeros(4, dtype=torch.long)),
        lambda: tritium.matmul(torch.randn(4, 4), torch.randn(4, 4)),
        lambda: tritium.matmul_vec(torch.randn(4), torch.randn(4, 4)),
    ],
)
def test_cpu_tensors_are_rejected(call):
    with pytest.raises(ValueError, match="must be a CUDA tensor"):
        call()


@pytest.fixture
def meta_ok(monkeypatch):
    """Treat meta tensors as device tensors so the later checks are reachable."""

    def check(name, tensor):
        if tensor.device.type not in ("cuda", "meta"):
            raise ValueError(f"{name} must be a CUDA tensor.")

    for mod in (_utils, rms_mod, rope_mod, swiglu_mod, adamw_mod, attn_mod, lce_mod):
        if hasattr(mod, "check_cuda_tensor"):
            monkeypatch.setattr(mod, "check_cuda_tensor", check)
    monkeypatch.setattr(_utils, "check_cuda_tensor", check)


def meta(*shape, dtype=torch.float32):
    return torch.empty(shape, device="meta", dtype=dtype)


def test_rmsnorm_messages(meta_ok):
    with pytest.raises(ValueError, match="Dtype mismatch"):
        rms_mod._check_rmsnorm_inputs(meta(4, 8), meta(8, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="Shape mismatch"):
        rms_mod._check_rmsnorm_inputs(meta(4, 8), meta(9))
    with pytest.raises(ValueError, match="Unsupported hidden size"):
        rms_mod._check_rmsnorm_inputs(meta(2, 70000), meta(70000))
    with pytest.raises(ValueError, match="x must be contiguous"):
        rms_mod._check_rmsnorm_inputs(meta(8, 4).t(), meta(8))
    with pytest.raises(ValueError, match="must have one of these dtypes"):
        rms_mod._check_rmsnorm_inputs(meta(4, 8, dtype=torch.int32), meta(8, dtype=torch.int32))


def test_attention_messages(meta_ok):
    with pytest.raises(ValueError, match="power of 2"):
        attn_mod._check_attention_inputs(meta(1, 2, 4, 24), meta(1, 2, 4, 24), meta(1, 2, 4, 24))
    with pytest.raises(ValueError, match="divisible"):
        attn_mod._check_attention_inputs(meta(1, 3, 4, 16), meta(1, 2, 4, 16), meta(1, 2, 4, 16))
    with pytest.raises(ValueError, match="Dtype mismatch"):
        attn_mod._check_attention_inputs(meta(1, 2, 4, 16), meta(1, 2, 4, 16, dtype=torch.float16),
                                         meta(1, 2, 4, 16))
    with pytest.raises(ValueError, match="Shape mismatch"):
        attn_mod._check_attention_inputs(meta(1, 2, 4, 16), meta(1, 2, 5, 16), meta(1, 2, 4, 16))
    # valid: GQA, q_len != kv_len
    assert attn_mod._check_attention_inputs(meta(2, 8, 3, 64), meta(2, 2, 7, 64), meta(2, 2, 7, 64)) == (
        2, 8, 2, 3, 7, 64)


def test_rope_messages(meta_ok):
    with pytest.raises(ValueError, match="head_dim must be even"):
        rope_mod._check_rope_inputs(meta(4, 7), meta(4, 7), meta(8, 3), meta(8, 3), None)
    with pytest.raises(ValueError, match="Shape mismatch"):
        rope_mod._check_rope_inputs(meta(4, 8), meta(4, 8), meta(8, 3), meta(8, 3), None)
    with pytest.raises(ValueError, match="Shape mismatch"):
        rope_mod._check_rope_inputs(meta(4, 8), meta(4, 8), meta(8, 4), meta(8, 4),
                                    meta(5, dtype=torch.int64))
    with pytest.raises(ValueError, match="must have one of these dtypes"):
        rope_mod._check_rope_inputs(meta(4, 8), meta(4, 8), meta(8, 4), meta(8, 4),
                                    meta(4, dtype=torch.float32))


def test_swiglu_and_adamw_messages(meta_ok):
    with pytest.raises(ValueError, match="Shape mismatch"):
        _utils.check_same_shape_dtype_device("x", meta(8), "gate", meta(9))
    with pytest.raises(ValueError, match="Dtype mismatch"):
        _utils.check_same_shape_dtype_device("x", meta(8), "gate", meta(8, dtype=torch.float16))
    with pytest.raises(ValueError, match="exp_avg must have dtype float32"):
        adamw_mod._check_adamw_inputs(meta(8), meta(8), meta(8, dtype=torch.bfloat16), meta(8))
    with pytest.raises(ValueError, match="Dtype mismatch"):
        adamw_mod._check_adamw_inputs(meta(8), meta(8, dtype=torch.float16), meta(8), meta(8))
    with pytest.raises(ValueError, match="same length"):
        tritium.adamw_step_multi([meta(8)], [], [], [], lr=1e-3)


def test_adamw_table_cache_revalidates_changed_tensors(meta_ok, monkeypatch):
    """A cached descriptor table is reused only for tensors with the same
    address, dtype, shape and contiguity on the same device; a wrong-dtype
    grad, a 16-bit moment, a reshaped or a non-contiguous view at a cached
    address is checked again and rejected (meta tensors all share address 0,
    the worst case)."""
    cache = adamw_mod._TableCache()
    monkeypatch.setattr(adamw_mod, "_tables", cache)
    p, g, m, v = meta(8, 4), meta(8, 4), meta(8, 4), meta(8, 4)
    key = adamw_mod._table_key([p], [g], [m], [v])
    assert key == (p.device,) + tuple(adamw_mod._signature(t) for t in (p, g, m, v))
    sentinel = ("table", 1, 1)
    cache.put(key, sentinel)
    assert adamw_mod._table_for([p], [g], [m], [v]) is sentinel
    with pytest.raises(ValueError, match="Dtype mismatch"):
        adamw_mod._table_for([p], [meta(8, 4, dtype=torch.float16)], [m], [v])
    with pytest.raises(ValueError, match="exp_avg must have dtype float32"):
        adamw_mod._table_for([p], [g], [meta(8, 4, dtype=torch.bfloat16)], [v])
    with pytest.raises(ValueError, match="must be contiguous"):
        adamw_mod._table_for([p], [g], [m], [meta(4, 8).t()])
    with pytest.raises(ValueError, match="Shape mismatch"):
        adamw_mod._table_for([p], [meta(4, 8)], [m], [v])


def test_linear_ce_messages(meta_ok):
    lt = torch.int64
    with pytest.raises(ValueError, match="at least 2 dimensions"):
        lce_mod._check_linear_cross_entropy_inputs(meta(8), meta(10, 8), meta(8, dtype=lt))
    with pytest.raises(ValueError, match="Shape mismatch"):
        lce_mod._check_linear_cross_entropy_inputs(meta(4, 8), meta(10, 9), meta(4, dtype=lt))
    with pytest.raises(ValueError, match="Shape mismatch"):
        lce_mod._check_linear_cross_entropy_inputs(meta(4, 8), meta(10, 8), meta(5, dtype=lt))
    with pytest.raises(ValueError, match="Dtype mismatch"):
        lce_mod._check_linear_cross_entropy_inputs(meta(4, 8), meta(10, 8, dtype=torch.bfloat16),
                                                   meta(4, dtype=lt))
    with pytest.raises(ValueError, match="must have one of these dtypes"):
        lce_mod._check_linear_cross_entropy_inputs(meta(4, 8), meta(10, 8), meta(4))
    assert lce_mod._check_linear_cross_entropy_inputs(meta(2, 3, 8), meta(10, 8),
                                                      meta(2, 3, dtype=lt)) == (6, 8, 10)
    with pytest.raises(ValueError, match="expected \\(\\)"):
        tritium.linear_cross_entropy_backward(meta(1), meta(4, 8), meta(10, 8), meta(4, dtype=lt), meta(4))


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import helion_amd._lib as L

    monkeypatch.setattr(L, "_handle", None)
    monkeypatch.setattr(L, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(L.LibraryNotBuilt, match="missing"):
        L.lib()

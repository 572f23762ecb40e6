"""The whole public surface of ``tritium`` (tritium/__init__.py:40-70) on the
CPU: every name exists, every op rejects CPU tensors as the reference does
(tests/tritium/test_{add,relu,add_relu,gelu,dropout,softmax,layernorm,sgd,
cross_entropy}.py, the ``*_rejects_*`` tests), and the later checks of the ops
off the hot path raise the reference's messages.  Those checks run on
shape-only "meta" tensors with the device check patched to accept them, so
no GPU is touched.
"""

from __future__ import annotations

import importlib

import pytest
import torch

import helion_amd as tritium
from helion_amd import _utils

ce_mod = importlib.import_module("helion_amd.cross_entropy")
ew_mod = importlib.import_module("helion_amd.elementwise")
nx_mod = importlib.import_module("helion_amd.norms_extra")

# tritium/__init__.py:40-70
REFERENCE_ALL = [
    "__version__", "add", "add_gelu", "add_relu", "adamw_step", "attention", "cross_entropy",
    "cross_entropy_backward", "dropout", "dropout_backward", "gelu", "gelu_backward",
    "layernorm", "layernorm_backward", "linear_cross_entropy", "linear_cross_entropy_backward",
    "matmul", "matmul_vec", "relu", "rope", "rope_", "residual_rmsnorm", "rmsnorm",
    "rmsnorm_backward", "sgd_step", "softmax", "softmax_backward", "swiglu", "swiglu_backward",
]


def test_every_reference_name_is_exported():
    assert set(REFERENCE_ALL) <= set(tritium.__all__)
    for name in REFERENCE_ALL[1:]:
        assert callable(getattr(tritium, name)), name


def _cpu(*shape, dtype=torch.float32):
    return torch.randn(*shape).to(dtype)


@pytest.mark.parametrize(
    "call",
    [
        lambda: tritium.add(_cpu(4), _cpu(4)),
        lambda: tritium.relu(_cpu(4)),
        lambda: tritium.add_relu(_cpu(4), _cpu(4)),
        lambda: tritium.gelu(_cpu(4)),
        lambda: tritium.add_gelu(_cpu(4), _cpu(4)),
        lambda: tritium.gelu_backward(_cpu(4), _cpu(4)),
        lambda: tritium.dropout(_cpu(8), 0.5, seed=0),
        lambda: tritium.dropout_backward(_cpu(8), 0.5, 0),
        lambda: tritium.sgd_step(_cpu(4), _cpu(4), 1e-2),
        lambda: tritium.softmax(_cpu(4, 8)),
        lambda: tritium.softmax_backward(_cpu(4, 8), _cpu(4, 8)),
        lambda: tritium.layernorm(_cpu(4, 8), _cpu(8), _cpu(8)),
        lambda: tritium.layernorm_backward(_cpu(4, 8), _cpu(4, 8), _cpu(8)),
        lambda: tritium.cross_entropy(_cpu(4, 10), torch.zeros(4, dtype=torch.long)),
        lambda: tritium.cross_entropy_backward(torch.tensor(1.0), _cpu(4, 10),
                                               torch.zeros(4, dtype=torch.long), _cpu(4)),
    ],
)
def test_cpu_tensors_are_rejected(call):
    with pytest.raises(ValueError, match="must be a CUDA tensor"):
        call()


def test_dropout_p_zero_returns_input_even_on_cpu():
    # dropout.py:152-153: p == 0 returns x before any check
    x = _cpu(8)
    assert tritium.dropout(x, 0.0) is x


@pytest.fixture
def meta_ok(monkeypatch):
    """Treat meta tensors as device tensors so the later checks are reachable."""

    def check(name, tensor):
        if tensor.device.type not in ("cuda", "meta"):
            raise ValueError(f"{name} must be a CUDA tensor.")

    for mod in (_utils, ce_mod, ew_mod, nx_mod):
        if hasattr(mod, "check_cuda_tensor"):
            monkeypatch.setattr(mod, "check_cuda_tensor", check)


def meta(*shape, dtype=torch.float32):
    return torch.empty(shape, device="meta", dtype=dtype)


def test_elementwise_messages(meta_ok):
    with pytest.raises(ValueError, match="Shape mismatch"):
        tritium.add(meta(4), meta(5))
    with pytest.raises(ValueError, match="Dtype mismatch"):
        tritium.add_relu(meta(4), meta(4, dtype=torch.float16))
    with pytest.raises(ValueError, match="must have one of these dtypes"):
        tritium.gelu(meta(4, dtype=torch.int32))
    with pytest.raises(ValueError, match="Shape mismatch: dy"):
        tritium.gelu_backward(meta(5), meta(4))
    with pytest.raises(ValueError, match="Shape mismatch"):
        tritium.add_gelu(meta(4), meta(2, 2))


@pytest.mark.parametrize("bad_p", [-0.1, 1.0, 1.5])
def test_dropout_rejects_invalid_p(meta_ok, bad_p):
    # tests/tritium/test_dropout.py:166-170
    with pytest.raises(ValueError, match="0 <= p < 1"):
        tritium.dropout(meta(16), bad_p, seed=0)
    with pytest.raises(ValueError, match="0 <= p < 1"):
        tritium.dropout_backward(meta(16), bad_p, 0)


def test_sgd_messages(meta_ok):
    with pytest.raises(ValueError, match="must be contiguous for tritium.sgd_step"):
        tritium.sgd_step(meta(4, 4).t(), meta(4, 4), 1e-2)
    with pytest.raises(ValueError, match="Dtype mismatch"):
        tritium.sgd_step(meta(4), meta(4, dtype=torch.bfloat16), 1e-2)


def test_softmax_messages(meta_ok):
    # tests/tritium/test_softmax.py:169-195
    with pytest.raises(ValueError, match="x must be contiguous"):
        tritium.softmax(meta(8, 4).t())
    with pytest.raises(ValueError, match="Unsupported hidden size"):
        tritium.softmax(meta(1, 65537))
    with pytest.raises(ValueError, match="at least 1 dimension"):
        tritium.softmax(torch.empty((), device="meta"))
    with pytest.raises(ValueError, match="Shape mismatch: dy"):
        tritium.softmax_backward(meta(2, 8), meta(2, 4))
    with pytest.raises(ValueError, match="Dtype mismatch: dy"):
        tritium.softmax_backward(meta(2, 4, dtype=torch.float16), meta(2, 4))


def test_layernorm_messages(meta_ok):
    # tests/tritium/test_layernorm.py:260-311
    with pytest.raises(ValueError, match="x must be contiguous"):
        tritium.layernorm(meta(8, 4).t(), meta(8), meta(8))
    with pytest.raises(ValueError, match="Shape mismatch"):
        tritium.layernorm(meta(2, 8), meta(4), meta(8))
    with pytest.raises(ValueError, match="Dtype mismatch: bias"):
        tritium.layernorm(meta(2, 8), meta(8), meta(8, dtype=torch.float16))
    with pytest.raises(ValueError, match="Unsupported hidden size"):
        tritium.layernorm(meta(1, 65537), meta(65537), meta(65537))
    with pytest.raises(ValueError, match="Shape mismatch: dy"):
        tritium.layernorm_backward(meta(2, 4), meta(2, 8), meta(8))


def test_cross_entropy_messages(meta_ok):
    # cross_entropy.py:385-428, 728-789; tests/tritium/test_cross_entropy.py:112-123
    tgt = meta(4, dtype=torch.long)
    with pytest.raises(ValueError, match="contiguous"):
        tritium.cross_entropy(meta(10, 4).t(), tgt)
    with pytest.raises(ValueError, match="logits must be a 2D tensor"):
        tritium.cross_entropy(meta(4), tgt)
    with pytest.raises(ValueError, match="target must be a 1D tensor"):
        tritium.cross_entropy(meta(4, 10), meta(4, 1, dtype=torch.long))
    with pytest.raises(ValueError, match="must have one of these dtypes"):
        tritium.cross_entropy(meta(4, 10), meta(4))
    with pytest.raises(ValueError, match="Shape mismatch: target"):
        tritium.cross_entropy(meta(4, 10), meta(3, dtype=torch.long))
    with pytest.raises(ValueError, match="Unsupported vocab size"):
        tritium.cross_entropy(meta(4, 131073), tgt)
    with pytest.raises(ValueError, match="Dtype mismatch: logsumexp"):
        tritium.cross_entropy_backward(meta(), meta(4, 10), tgt, meta(4, dtype=torch.float16))
    with pytest.raises(ValueError, match="Shape mismatch: grad_out"):
        tritium.cross_entropy_backward(meta(1), meta(4, 10), tgt, meta(4))
    with pytest.raises(ValueError, match="Shape mismatch: logsumexp"):
        tritium.cross_entropy_backward(meta(), meta(4, 10), tgt, meta(5))

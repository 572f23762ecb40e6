"""CPU oracle for the tritium.ops hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy on the CPU, the arithmetic of the reference's
``tritium.ops`` kernels (alkinun/helion, ``tritium/ops/*.py``).  It is the
checker the HIP kernels are compared against; it is never part of the product:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  ``helion_amd`` never imports it and has no CPU
fallback.

Conventions shared by every function here:

* Inputs are float32 numpy arrays whose values are exactly representable in the
  storage dtype of the op under test (``"f32"``, ``"f16"`` or ``"bf16"``);
  :func:`oracle.numerics.quantize` produces such arrays.
* Arithmetic is float32, as in the reference kernels (every kernel upcasts with
  ``.to(tl.float32)`` before computing); outputs are rounded to the storage
  dtype with round-to-nearest-even, as the kernels' ``tl.store`` does.
* Each function cites the reference ``file:line`` whose arithmetic it follows.

Pinning status (what independent check fixes each function) is written in the
docstring of every module; the CPU test-suite (``tests/test_oracle.py``)
runs those checks.
"""

from . import adamw, attention, embedding, linear_ce, numerics, rmsnorm, rope, swiglu, torch_ref

__all__ = [
    "adamw",
    "attention",
    "embedding",
    "linear_ce",
    "numerics",
    "rmsnorm",
    "rope",
    "swiglu",
    "torch_ref",
]

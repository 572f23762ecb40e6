"""Embedding backward with a tied output head (test infrastructure).

Follows alkinun/helion ``helion/nn.py:24-28`` (``Embedding.forward`` is the
gather ``weight[ids]``; its gradient is torch's scatter-add of the upstream
rows into the rows the ids name) and the tied head of ``examples/common.py``
(the same weight is the output projection, so its gradient is the head's
weight gradient plus that scatter-add).

Pinned by (tests/test_oracle.py, test_embedding_*): the golden fixture of
torch's own ``F.embedding`` autograd (float64, repeated ids included), the
closed form for ids that are all distinct (each row gets exactly its one
upstream row), and a planted mistake (a dropped repeat) that the fixture
rejects.
"""

from __future__ import annotations

import numpy as np

from .numerics import quantize


def backward(ids: np.ndarray, dx: np.ndarray, dw_in: np.ndarray, dtype: str = "f32",
             acc=np.float64) -> np.ndarray:
    """``dw_in + scatter_add(ids, dx)`` rounded once into ``dtype``; ids outside
    ``[0, vocab)`` add nothing."""
    vocab = dw_in.shape[0]
    out = dw_in.astype(acc).copy()
    ids = np.asarray(ids).reshape(-1).astype(np.int64)
    rows = dx.reshape(ids.shape[0], -1).astype(acc)
    keep = (ids >= 0) & (ids < vocab)
    np.add.at(out, ids[keep], rows[keep])
    return quantize(out.astype(np.float32), dtype)

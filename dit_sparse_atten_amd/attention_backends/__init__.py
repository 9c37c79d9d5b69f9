"""Attention backends with the reference's selection names and call signature.

``dense`` -> DenseBackend, ``flex_reuse`` -> FlexReuseBackend and ``sparse`` ->
MatrixSparseBackend, mirroring attention_backends/__init__.py and
infer.py:180-223 of the reference.
"""

from .dense import DenseBackend
from .flex import FlexReuseBackend, FlexReuseConfig
from .sparse import MatrixSparseBackend, SparseConfig

BACKENDS = {
    "dense": DenseBackend,
    "flex_reuse": FlexReuseBackend,
    "sparse": MatrixSparseBackend,
}

__all__ = ["BACKENDS", "DenseBackend", "FlexReuseBackend", "FlexReuseConfig",
           "MatrixSparseBackend", "SparseConfig"]

"""Attention backends with the reference's selection names and call signature.

``dense`` -> DenseBackend, ``flex_reuse`` -> FlexReuseBackend (and, once its
GPU path lands, ``sparse`` -> MatrixSparseBackend), mirroring
attention_backends/__init__.py and infer.py:180-223 of the reference.
"""

from .dense import DenseBackend
from .flex import FlexReuseBackend, FlexReuseConfig

__all__ = ["DenseBackend", "FlexReuseBackend", "FlexReuseConfig"]

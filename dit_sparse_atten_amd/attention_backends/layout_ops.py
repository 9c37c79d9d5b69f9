"""Data-movement operations shared by the sparse backends.

Mirrors attention_backends/layout_ops.py of the reference: ``reorder_qkv``
(layout_ops.py:86-125) gathers Q/K/V through one permutation in one launch and
``pack_boolean_rows`` (layout_ops.py:128-151) stable-partitions boolean route
rows.  Both run libdsa HIP kernels for every input layout (strided views
included); there is no index_select or argsort fallback.
"""

from __future__ import annotations

import torch

from .. import ops


def reorder_qkv(q, k, v, permutation, head_major=True):
    """Return Q/K/V reordered on the token axis: X'[b, t] = X[b, permutation[t]].

    Outputs keep the logical [B, T, H, D] shape; with ``head_major`` their
    storage is head-major (each head's tokens contiguous), the layout the
    attention kernel streams fastest.
    """
    if not (q.ndim == k.ndim == v.ndim == 4 and q.shape == k.shape == v.shape):
        raise ValueError("q, k and v must share one [batch, tokens, heads, dim] shape")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k and v must share one dtype")
    if permutation.ndim != 1 or permutation.numel() != q.shape[1]:
        raise ValueError("permutation must contain one index per token")
    return tuple(ops.permute_tokens((q, k, v), permutation, head_major=head_major))


def reorder(tensor, permutation, head_major=False):
    """Single-tensor gather along the token axis (restore uses the inverse)."""
    if permutation.ndim != 1 or permutation.numel() != tensor.shape[1]:
        raise ValueError("permutation must contain one index per token")
    return ops.permute_tokens((tensor,), permutation, head_major=head_major)[0]


def pack_boolean_rows(route):
    """Pack selected column IDs first in every row, preserving ID order."""
    if not isinstance(route, torch.Tensor) or route.dtype != torch.bool or route.ndim < 2:
        raise ValueError("route must be a boolean tensor with at least two axes")
    return ops.pack_rows(route)

"""CPU restatement of block-sparse attention (test infrastructure only).

The reference computes block-sparse attention with FlexAttention over a
BlockMask (attention_backends/flex.py:379-399) and, in its matrix-tile path,
by gathering the selected key tiles and applying a ``finfo.min`` masked
softmax (attention_backends/sparse.py:670-751).  Both equal the closed form

    O[b,t,h] = softmax_k( scale * q[b,t,h] . k[b,k,h] + mask(-inf) ) @ v[b,k,h]

with mask = route[h, t // block, k // block] (the pattern of the reference's
tests/test_flex_backend.py:138-144).  This module evaluates that closed form
in float64 with numpy.  It is never imported by the product path.
"""

from __future__ import annotations

import numpy as np


def _as_route(route, batch):
    """Return the route as [R, H, QB, KB] with R in {1, batch}."""
    route = np.asarray(route, dtype=bool)
    if route.ndim == 3:
        route = route[None]
    if route.shape[0] not in (1, batch):
        raise ValueError("route batch must be 1 or the attention batch")
    return route


def block_sparse_attention(q, k, v, route, block_size, scale=None, rows=None, causal=False):
    """Masked-softmax attention in float64.

    q: [B,Tq,H,D]; k, v: [B,Tk,H,D] (any float dtype); route: boolean
    [H,QB,KB] / [R,H,QB,KB] or None for dense.  ``rows`` optionally restricts
    the evaluation to a list of (b, h, query_block) triples; the result then
    holds only those query blocks (others are NaN).  Query rows whose route row
    is empty produce zeros (the convention of an attention kernel without the
    ROWS_GUARANTEED_SAFE guarantee, flex.py:360-364).  ``causal`` (dense only)
    additionally masks keys k > t for query t, as SDPA's is_causal does
    (dense.py:40-47 passes it through).
    Returns (O [B,Tq,H,D] float64, LSE [B,H,Tq] float64 natural log).
    """
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    batch, q_tokens, heads, head_dim = q.shape
    kv_tokens = k.shape[1]
    if scale is None:
        scale = head_dim ** -0.5
    if route is not None:
        route = _as_route(route, batch)
    q_blocks = -(-q_tokens // block_size)
    if rows is None:
        rows = [(b, h, qb) for b in range(batch) for h in range(heads)
                for qb in range(q_blocks)]
    out = np.full(q.shape, np.nan)
    lse = np.full((batch, heads, q_tokens), np.nan)
    key_block = np.arange(kv_tokens) // block_size
    for b, h, qb in rows:
        t0, t1 = qb * block_size, min((qb + 1) * block_size, q_tokens)
        scores = (q[b, t0:t1, h] @ k[b, :, h].T) * scale
        if route is not None:
            allowed = route[0 if route.shape[0] == 1 else b, h, qb][key_block]
            scores = np.where(allowed[None, :], scores, -np.inf)
        if causal:
            later = np.arange(kv_tokens)[None, :] > np.arange(t0, t1)[:, None]
            scores = np.where(later, -np.inf, scores)
        row_max = scores.max(-1, keepdims=True)
        empty = ~np.isfinite(row_max[:, 0])
        row_max = np.where(np.isfinite(row_max), row_max, 0.0)
        weights = np.exp(scores - row_max)
        total = weights.sum(-1, keepdims=True)
        safe = np.where(total > 0, total, 1.0)
        out[b, t0:t1, h] = np.where(empty[:, None], 0.0, (weights @ v[b, :, h]) / safe)
        lse[b, h, t0:t1] = np.where(empty, -np.inf, row_max[:, 0] + np.log(safe[:, 0]))
    return out, lse


def summarize(actual, reference):
    """rel-L2, max-abs and cosine, as defined by profiles/backend/metrics.py:8-30."""
    actual = np.asarray(actual, dtype=np.float64).ravel()
    reference = np.asarray(reference, dtype=np.float64).ravel()
    difference = np.linalg.norm(actual - reference)
    denominator = max(np.linalg.norm(reference), 1e-12)
    norms = np.linalg.norm(actual) * np.linalg.norm(reference)
    cosine = float(actual @ reference / norms) if norms > 0 else 0.0
    return {
        "relative_l2": float(difference / denominator),
        "max_absolute_error": float(np.abs(actual - reference).max()) if actual.size else 0.0,
        "cosine_similarity": cosine,
    }

"""CPU restatement of the exact (dense + LSE) route estimator (test infrastructure only).

Follows attention_backends/flex.py:
  dense_lse          the per-query log-sum-exp that flex_attention(...,
                     return_lse=True) returns (flex.py:254-265, 779-783)
  exact_block_mass   _reference_block_mass / _block_attention_mass
                     (flex.py:96-106, 158-202)
  exact_route        _dense_bootstrap's route + _add_first_frame_sink
                     (flex.py:254-272, 708-716)

Everything is float64 on the given (already bf16-rounded, if the device path
computes in bf16) inputs.  Pinned by tests/test_oracle_exact.py: the
reference's own identities (full sampling S = block equals exact / block,
test_flex_backend.py:43-53; explicit softmax over the padded matrix,
test_flex_backend.py:62-76), rows summing to the valid query count, and
planted mistakes.
"""

from __future__ import annotations

import math

import numpy as np

from . import route as route_oracle


def _heads_first(x):
    """[1, T, H, D] or [T, H, D] -> float64 [H, T, D]."""
    x = np.asarray(x, dtype=np.float64)
    if x.ndim == 4:
        if x.shape[0] != 1:
            raise ValueError("exact route estimation supports batch-1 self-attention")
        x = x[0]
    return np.ascontiguousarray(x.transpose(1, 0, 2))


def scores(q, k, scale=None):
    """scale * q k^T per head: float64 [H, T, T]."""
    qh, kh = _heads_first(q), _heads_first(k)
    if scale is None:
        scale = qh.shape[-1] ** -0.5
    return np.einsum("hqd,hkd->hqk", qh, kh) * scale


def dense_lse(q, k, scale=None):
    """Natural-log normaliser of every query row: float64 [H, T]."""
    s = scores(q, k, scale)
    peak = s.max(-1, keepdims=True)
    return (peak + np.log(np.exp(s - peak).sum(-1, keepdims=True)))[..., 0]


def exact_block_mass(q, k, lse, block_size, scale=None):
    """mass[h, qb, kb] = sum over the tokens of both blocks of exp(s - lse)
    (flex.py:96-106): probabilities padded to whole blocks with zeros."""
    s = scores(q, k, scale)
    heads, tokens, _ = s.shape
    lse = np.asarray(lse, dtype=np.float64).reshape(heads, tokens)
    probabilities = np.exp(s - lse[..., None])
    blocks = math.ceil(tokens / block_size)
    padded = np.zeros((heads, blocks * block_size, blocks * block_size))
    padded[:, :tokens, :tokens] = probabilities
    return padded.reshape(heads, blocks, block_size, blocks, block_size).sum((2, 4))


def exact_block_mass_rows(q, k, lse, block_size, rows, scale=None):
    """Rows (h, qb) of exact_block_mass only, for full-size inputs: float64
    [len(rows), blocks].  Each row costs one [block, T] score tile."""
    qh, kh = _heads_first(q), _heads_first(k)
    heads, tokens, dim = qh.shape
    if scale is None:
        scale = dim ** -0.5
    lse = np.asarray(lse, dtype=np.float64).reshape(heads, tokens)
    blocks = math.ceil(tokens / block_size)
    out = np.zeros((len(rows), blocks))
    for i, (h, qb) in enumerate(rows):
        t0, t1 = qb * block_size, min(tokens, (qb + 1) * block_size)
        p = np.exp(qh[h, t0:t1] @ kh[h].T * scale - lse[h, t0:t1, None])
        padded = np.zeros((t1 - t0, blocks * block_size))
        padded[:, :tokens] = p
        out[i] = padded.reshape(t1 - t0, blocks, block_size).sum((0, 2))
    return out


def exact_route(mass, target, keep, grid=None, block_size=128, first_frame_sink=True):
    """Top-mass route of the exact mass, then the first-frame sink columns
    (flex.py:254-272 then 550-566), with the shared selection arithmetic."""
    route = route_oracle.top_mass_route(np.asarray(mass, dtype=np.float32), target, keep)
    if first_frame_sink and grid is not None:
        route = route_oracle.first_frame_sink(route, grid, block_size)
    return route

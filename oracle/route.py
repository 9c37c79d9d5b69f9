"""CPU restatement of the sampled route update (test infrastructure only).

Follows attention_backends/flex.py:
  sampled_block_mass   flex.py:205-251  (_sampled_block_mass)
  persistence_prior    flex.py:535-541  (prior inside _sampled_route)
  top_mass_route       flex.py:83-94    (_top_mass_route; == sparse.py:171-181 _row_mask)
  first_frame_sink     flex.py:550-566  (_add_first_frame_sink)
  pack_rows            layout_ops.py:128-151 (pack_boolean_rows), flex.py:275-281
  route_keep / dense   flex.py:473-493  (_update_dispatch)

Route-selection arithmetic (the one documented arithmetic shared with the HIP
kernel, so that routes are bit-exact given the same fp32 mass):
  * a row value m >= 0 is represented exactly as the integer
    floor(m * 2^(52 + s)), with the row exponent s the largest integer for
    which K * max(row) * 2^s < 2^10 (s = 0 for an all-zero row), so no sum of
    the row reaches 2^62 whatever the mass's magnitude;
  * every row sum and prefix sum is the exact integer sum, rounded once to
    fp32 (round-to-nearest-even) and scaled by 2^-(52 + s) (a power of two:
    the fp32 arithmetic below does not depend on s);
  * threshold = fp32(fp32(row sum) * fp32(target)); mean = fp32(row sum / K);
  * prior: m' = fp32(m + fp32(fp32(rho) * mean) * prev);
  * the row is ordered by value descending, ties by key index ascending;
  * count = #{i : prefix_i < threshold} + 1, clamped to the cap.
The reference's torch reductions round partial sums in an order that differs
between CPU and GPU builds; they agree with this arithmetic except in rows
whose deciding prefix lies within a few fp32 ulp of the threshold.
"""

from __future__ import annotations

import math

import numpy as np

FIXED_SHIFT = 52
_FIXED_SCALE = float(2 ** FIXED_SHIFT)
_INV_SCALE = np.float32(2.0 ** -FIXED_SHIFT)


def to_bf16(values):
    """Round float32 values to bfloat16 (round-to-nearest-even), kept as float32."""
    values = np.ascontiguousarray(values, dtype=np.float32)
    bits = values.view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return rounded.astype(np.uint32).view(np.float32)


def to_fp16(values):
    """Round float32 values to float16 (round-to-nearest-even, overflow to
    inf), kept as float32."""
    return np.asarray(values, dtype=np.float32).astype(np.float16).astype(np.float32)


def sample_indices(tokens, block_size, samples):
    """Token indices sampled per block: [blocks, samples] (flex.py:221-231)."""
    blocks = -(-tokens // block_size)
    block_ids = np.arange(blocks)
    sizes = np.minimum(tokens - block_ids * block_size, block_size)
    sample_ids = np.arange(samples)
    local = ((2 * sample_ids + 1)[None] * sizes[:, None]) // (2 * samples)
    local = np.minimum(local, sizes[:, None] - 1)
    return block_ids[:, None] * block_size + local, sizes


def sampled_block_mass(q, k, block_size, samples, scale=None, bf16_scores=True,
                       query_blocks=None, score_dtype=None):
    """Sampled estimate of per-(head, q-block, k-block) attention mass.

    q, k: [1, T, H, D] arrays (values already representable in the input
    dtype).  The scores are rounded to the input dtype after the dot product
    and again after the scale multiply, as a matmul and a multiply in that
    dtype do (flex.py:245): ``score_dtype`` "bf16" or "fp16", or None for
    float32 inputs (no rounding); without ``score_dtype``, ``bf16_scores``
    selects "bf16" or None.  The softmax runs on float64 here (float32 in the
    reference).  Returns mass [H, blocks, blocks] float64, or,
    with ``query_blocks`` (a list of query-block ids), only those rows:
    [H, len(query_blocks), blocks].  Every row is a softmax over all sampled
    keys, so a row does not depend on which other rows are evaluated.
    """
    if q.shape[0] != 1 or q.shape[1] != k.shape[1]:
        raise ValueError("sampled route update supports batch-1 self-attention")
    if samples <= 0 or samples > block_size:
        raise ValueError("route_samples must be in [1, block_size]")
    tokens, heads, head_dim = q.shape[1:]
    indices, sizes = sample_indices(tokens, block_size, samples)
    blocks = indices.shape[0]
    q_indices = indices if query_blocks is None else indices[np.asarray(query_blocks)]
    # Only the sampled tokens are converted to float64.
    sampled_q = np.asarray(q[0, q_indices.reshape(-1)], dtype=np.float64).transpose(1, 0, 2)
    sampled_k = np.asarray(k[0, indices.reshape(-1)], dtype=np.float64).transpose(1, 0, 2)
    log_weights = np.log(
        (sizes.astype(np.float32) / np.float32(samples)).astype(np.float32)).astype(np.float32)
    log_weights = np.repeat(log_weights, samples).astype(np.float64)
    if scale is None:
        scale = head_dim ** -0.5
    scores = np.einsum("hqd,hkd->hqk", sampled_q, sampled_k)
    rounding = score_dtype if score_dtype is not None else ("bf16" if bf16_scores else None)
    if rounding is not None:
        rounder = {"bf16": to_bf16, "fp16": to_fp16}[rounding]
        scores = rounder(scores.astype(np.float32))
        scores = rounder((scores * np.float32(scale)).astype(np.float32)).astype(np.float64)
    else:
        scores = (scores.astype(np.float32) * np.float32(scale)).astype(np.float64)
    logits = scores + log_weights[None, None]
    logits -= logits.max(-1, keepdims=True)
    weights = np.exp(logits)
    probabilities = weights / weights.sum(-1, keepdims=True)
    rows = q_indices.shape[0]
    return probabilities.reshape(heads, rows, samples, blocks, samples).sum(-1).mean(2)


def row_shift(mass):
    """Row exponent s of every row of a non-negative fp32 [..., K] tensor: the
    largest integer with K * max(row) * 2^s < 2^10, 0 for an all-zero row."""
    mass = np.asarray(mass, dtype=np.float32)
    top = mass.max(-1).astype(np.float64)
    _, exponent = np.frexp(mass.shape[-1] * top)  # K * max = f * 2^e, f in [0.5, 1)
    return np.where(top > 0, 10 - exponent, 0).astype(np.int64)


def _fixed(row, shift=None):
    """Exact integer image floor(m * 2^(52 + s)) of non-negative fp32 values
    (s per row, [..., 1]; None: s = 0)."""
    row = np.asarray(row, dtype=np.float32).astype(np.float64)
    if shift is None:
        return np.floor(row * _FIXED_SCALE).astype(np.int64)
    return np.floor(np.ldexp(row, (FIXED_SHIFT + shift).astype(np.int32))).astype(np.int64)


def _fixed_to_f32(total, shift=None):
    """Round exact fixed-point sums to fp32 (RNE) and rescale by 2^-(52 + s)."""
    total = np.asarray(total, dtype=np.int64).astype(np.float32)
    if shift is None:
        return total * _INV_SCALE
    return np.ldexp(total, (-(FIXED_SHIFT + shift)).astype(np.int32)).astype(np.float32)


def row_sums_f32(mass, scaled=True):
    """Exact row sums of a non-negative fp32 [..., K] tensor, rounded to fp32:
    in the scaled fixed point of the route arithmetic, or (scaled=False) at
    the fixed scale 2^52, as the matrix-sparse head sums accumulate across
    workgroups."""
    if not scaled:
        return _fixed_to_f32(_fixed(mass).sum(-1))
    shift = row_shift(mass)
    return _fixed_to_f32(_fixed(mass, shift[..., None]).sum(-1), shift)


def persistence_prior(mass, previous, rho):
    """m' = m + rho * mean_k(m) * previous, in the documented fp32 arithmetic."""
    mass = np.asarray(mass, dtype=np.float32)
    keys = mass.shape[-1]
    mean = (row_sums_f32(mass) / np.float32(keys)).astype(np.float32)
    prior = (np.float32(rho) * mean).astype(np.float32)
    term = prior[..., None] * np.asarray(previous, dtype=np.float32)
    return (mass + term.astype(np.float32)).astype(np.float32)


def route_cap(keys, keep):
    """Per-row block cap max(1, ceil(K * keep)) (flex.py:89)."""
    return max(1, math.ceil(keys * keep))


def top_mass_route(mass, target, keep, return_margins=False):
    """Select, per row, the fewest top blocks whose mass reaches the target.

    mass: fp32 [..., K] with non-negative entries.  Returns a bool route of the
    same shape.  With ``return_margins`` it also returns, per row, the distance
    in fp32 ulps between the threshold and the nearest prefix sum, which tells
    how sensitive the row's decision is to reduction order.
    """
    mass = np.asarray(mass, dtype=np.float32)
    shape = mass.shape
    keys = shape[-1]
    rows = mass.reshape(-1, keys)
    cap = route_cap(keys, keep)
    target32 = np.float32(target)
    order = np.argsort(-rows, axis=-1, kind="stable")
    shift = row_shift(rows)
    fixed = _fixed(rows, shift[:, None])
    totals = _fixed_to_f32(fixed.sum(-1), shift)
    thresholds = (totals * target32).astype(np.float32)
    prefix = _fixed_to_f32(np.cumsum(np.take_along_axis(fixed, order, -1), axis=-1),
                           shift[:, None])
    below = prefix < thresholds[:, None]
    counts = np.minimum(below.sum(-1) + 1, cap)
    ranks = np.empty_like(order)
    np.put_along_axis(ranks, order, np.arange(keys)[None].repeat(rows.shape[0], 0), -1)
    route = ranks < counts[:, None]
    if not return_margins:
        return route.reshape(shape)
    spacing = np.spacing(np.abs(thresholds)).astype(np.float64)
    spacing[spacing == 0] = np.finfo(np.float32).tiny
    gaps = np.abs(prefix.astype(np.float64) - thresholds[:, None].astype(np.float64))
    margins = gaps.min(-1) / spacing
    return route.reshape(shape), margins.reshape(shape[:-1])


def first_frame_sink(route, grid, block_size):
    """route[..., :ceil(H*W / block)] = True (flex.py:550-566)."""
    route = np.array(route, dtype=bool, copy=True)
    if grid is None:
        return route
    sink = math.ceil(grid[1] * grid[2] / block_size)
    route[..., :sink] = True
    return route


def sampled_route(q, k, block_size, samples, target, keep, previous=None, rho=0.5,
                  grid=None, scale=None, mass=None):
    """Mass -> prior -> top-mass -> sink, as flex.py:508-548 (no directional update)."""
    if mass is None:
        mass = sampled_block_mass(q, k, block_size, samples, scale).astype(np.float32)
    mass = np.asarray(mass, dtype=np.float32)
    if rho and previous is not None:
        mass = persistence_prior(mass, previous, rho)
    route = top_mass_route(mass, target, keep)
    return first_frame_sink(route, grid, block_size)


def pack_rows(route):
    """Stable partition of each boolean row: selected IDs ascending, then
    unselected IDs ascending (layout_ops.py:128-151).  Returns (counts int32,
    indices int32) with the route's leading shape."""
    route = np.asarray(route, dtype=bool)
    counts = route.sum(-1).astype(np.int32)
    indices = np.argsort(~route, axis=-1, kind="stable").astype(np.int32)
    return counts, indices


def to_csr(route):
    """CSR (row_ptr, col_idx, counts) of a boolean route over its last axis."""
    route = np.asarray(route, dtype=bool)
    flat = route.reshape(-1, route.shape[-1])
    counts = flat.sum(-1).astype(np.int32)
    row_ptr = np.zeros(flat.shape[0] + 1, dtype=np.int64)
    row_ptr[1:] = np.cumsum(counts)
    col_idx = np.nonzero(flat)[1].astype(np.int32)
    return row_ptr.astype(np.int32), col_idx, counts.reshape(route.shape[:-1])


def route_keep(route):
    """Keep fraction as torch computes route.float().mean() (fp32)."""
    route = np.asarray(route, dtype=bool)
    return float(np.float32(np.float32(route.sum()) / np.float32(route.size)))


def dense_dispatch(route, threshold):
    """keep >= threshold (flex.py:482-486)."""
    return threshold is not None and route_keep(route) >= threshold

"""CPU restatement of the frontier-aware directional route update (test
infrastructure only).

Follows attention_backends/routing.py:
  frontier_mask              routing.py:10-41
  best_targets               routing.py:53-80  (_sparse_best_targets)
  select_fixed_budget        routing.py:83-89  (_select_fixed_budget)
  directional_budget_update  routing.py:92-168
  budget_select              its row-local half, routing.py:139-160

Arithmetic shared bit-for-bit with the HIP kernels (the reference's torch
reductions and unstable argsorts leave these open):
  * row mean = fp32(exact row sum / K) (fixed point, as oracle.route);
  * score = fp32(fp32(mass + fp32(fp32(fp32(persistence) * mean) * prev))
                 + fp32(fp32(fp32(bonus) * mean) * candidate));
  * budget = clamp(ceil(fp32(fp32(|previous row|) * fp32(budget_scale))), 1, cap);
  * every ordering is value descending, then key index ascending; the best
    neighbour of a cell is the first direction (0..3) holding the maximum.
Pinned by tests/test_oracle_routing.py: the reference's known answers
(test_directional_routing.py), golden vectors written by the reference's own
functions, brute force and planted mistakes.
"""

from __future__ import annotations

import math

import numpy as np

from . import route as route_oracle


def _check(route, neighbors):
    route = np.asarray(route, dtype=bool)
    neighbors = np.asarray(neighbors, dtype=np.int64)
    if route.ndim != 3 or route.shape[1] != route.shape[2]:
        raise ValueError("route must have shape [heads, blocks, blocks]")
    if neighbors.shape != (route.shape[-1], 4):
        raise ValueError("neighbors must have shape [blocks, 4]")
    return route, neighbors


def frontier_mask(route, neighbors):
    """Selected cells with an unselected valid 4-neighbour along the query
    axis (rows) or the key axis (columns)."""
    route, neighbors = _check(route, neighbors)
    open_any = np.zeros_like(route)
    for direction in range(4):
        target = neighbors[:, direction]
        valid = target >= 0
        safe = np.maximum(target, 0)
        open_any |= valid[None, :, None] & ~route[:, safe, :]
        open_any |= valid[None, None, :] & ~route[:, :, safe]
    return route & open_any


def best_targets(mass, previous, neighbors, frontier, axis, min_ratio):
    """For every frontier cell (h, q, k), in lexicographic order: the
    unselected neighbour (of q for axis 1, of k for axis 2) with the largest
    mass, and whether it passes min_ratio.  Returns (cells [n, 3], targets
    [n], eligible [n], candidates bool like previous)."""
    mass = np.asarray(mass, dtype=np.float32)
    cells = np.argwhere(frontier)
    candidates = np.zeros(previous.shape, dtype=bool)
    if cells.size == 0:
        return cells, np.zeros(0, np.int64), np.zeros(0, bool), candidates
    h, q, k = cells.T
    source = q if axis == 1 else k
    targets = neighbors[source]                       # [n, 4]
    valid = targets >= 0
    safe = np.maximum(targets, 0)
    if axis == 1:
        selected = previous[h[:, None], safe, k[:, None]]
        values = mass[h[:, None], safe, k[:, None]]
    else:
        selected = previous[h[:, None], q[:, None], safe]
        values = mass[h[:, None], q[:, None], safe]
    values = np.where(~valid | selected, -np.inf, values.astype(np.float64))
    direction = values.argmax(-1)                     # first maximum
    best = values[np.arange(len(cells)), direction]
    target = safe[np.arange(len(cells)), direction]
    floor_value = (mass[h, q, k] * np.float32(min_ratio)).astype(np.float32)
    eligible = np.isfinite(best) & (best >= floor_value.astype(np.float64))
    if axis == 1:
        candidates[h[eligible], target[eligible], k[eligible]] = True
    else:
        candidates[h[eligible], q[eligible], target[eligible]] = True
    return cells, target, eligible, candidates


def _order(values):
    """Per-row order: value descending, then index ascending."""
    keys = np.arange(values.shape[-1])
    return np.lexsort((np.broadcast_to(keys, values.shape), -values), axis=-1)


def _rank(values):
    order = _order(values)
    ranks = np.empty_like(order)
    np.put_along_axis(ranks, order, np.broadcast_to(np.arange(values.shape[-1]), order.shape),
                      axis=-1)
    return ranks


def select_fixed_budget(score, pool, counts):
    """The top min(count, |pool|) (at least 1) pool entries of every row by score."""
    values = np.where(pool, score.astype(np.float64), -np.inf)
    ranks = _rank(values)
    counts = np.maximum(np.minimum(counts, pool.sum(-1)), 1)
    return (ranks < counts[..., None]) & pool


def row_mean_f32(mass):
    """fp32(exact row sum / K), the shared row-scale arithmetic."""
    mass = np.asarray(mass, dtype=np.float32)
    sums = route_oracle.row_sums_f32(mass)
    return (sums / np.float32(mass.shape[-1])).astype(np.float32)


def directional_budget_update(mass, previous, neighbors, *, keep, persistence=0.5,
                              min_ratio=0.0, candidate_bonus=0.0, budget_scale=1.0,
                              exploration_fraction=0.0, expand_q=True, expand_k=True,
                              expand_joint=True, previous_frontier=None):
    """Expand only route frontiers, then prune back to a per-row budget."""
    mass = np.asarray(mass, dtype=np.float32)
    previous, neighbors = _check(previous, neighbors)
    if previous.shape != mass.shape:
        raise ValueError("previous route and mass must have identical shapes")
    if budget_scale <= 0:
        raise ValueError("budget_scale must be positive")
    if not 0 <= exploration_fraction <= 1:
        raise ValueError("exploration_fraction must be in [0, 1]")
    source = (np.asarray(previous_frontier, dtype=bool) if previous_frontier is not None
              else frontier_mask(previous, neighbors))
    cells, q_targets, q_eligible, q_candidates = best_targets(
        mass, previous, neighbors, source, 1, min_ratio)
    _, k_targets, k_eligible, k_candidates = best_targets(
        mass, previous, neighbors, source, 2, min_ratio)
    candidates = np.zeros_like(previous)
    if expand_q:
        candidates |= q_candidates
    if expand_k:
        candidates |= k_candidates
    if expand_joint and cells.size:
        joint = q_eligible & k_eligible
        candidates[cells[joint, 0], q_targets[joint], k_targets[joint]] = True
    candidates &= ~previous
    route, exploration = budget_select(
        mass, previous, candidates, keep=keep, persistence=persistence,
        candidate_bonus=candidate_bonus, budget_scale=budget_scale,
        exploration_fraction=exploration_fraction)
    return {
        "route": route,
        "frontier": frontier_mask(route, neighbors),
        "candidates": candidates,
        "exploration": exploration,
        "dropped": previous & ~route,
        "added": route & ~previous,
    }


def budget_select(mass, previous, candidates, *, keep, persistence=0.5, candidate_bonus=0.0,
                  budget_scale=1.0, exploration_fraction=0.0):
    """The row-local half of directional_budget_update (routing.py:139-160):
    exploration, scores and the fixed-budget selection of every row of
    [..., K] inputs, given the row's candidates (disjoint from previous).
    Each row's result depends only on that row and K.  Returns (route,
    exploration)."""
    mass = np.asarray(mass, dtype=np.float32)
    previous = np.asarray(previous, dtype=bool)
    candidates = np.asarray(candidates, dtype=bool)
    blocks = mass.shape[-1]
    pool = previous | candidates
    exploration = np.zeros_like(pool)
    if exploration_fraction:
        explore = max(1, math.ceil(blocks * exploration_fraction))
        ranks = _rank(np.where(pool, -np.inf, mass.astype(np.float64)))
        exploration = ranks < explore
        pool = pool | exploration
    mean = row_mean_f32(mass)[..., None]
    prior = (np.float32(persistence) * mean).astype(np.float32)
    score = (mass + (prior * previous.astype(np.float32)).astype(np.float32)).astype(np.float32)
    if candidate_bonus:
        bonus = (np.float32(candidate_bonus) * mean).astype(np.float32)
        score = (score + (bonus * candidates.astype(np.float32)).astype(np.float32)).astype(
            np.float32)
    cap = max(1, math.ceil(blocks * keep))
    budget = np.ceil((previous.sum(-1).astype(np.float32) * np.float32(budget_scale)).astype(
        np.float32)).astype(np.int64)
    budget = np.clip(budget, 1, cap)
    return select_fixed_budget(score, pool, budget), exploration

"""Frontier-aware directional updates for spatial routes, on the GPU.

Mirrors attention_backends/routing.py of the reference:
  frontier_mask              routing.py:35-41    -> dsa_frontier_mask
  directional_budget_update  routing.py:92-168   -> dsa_directional_update
Same arguments, validation errors and result keys.  Orderings that the
reference leaves to torch's unstable argsort are value descending, then key
index ascending; row means are exact row sums rounded once to fp32.
"""

from __future__ import annotations

from .. import ops


def frontier_mask(route, neighbors):
    """Return selected route cells adjacent to an unselected spatial cell."""
    return ops.frontier_mask(route, neighbors)


def directional_budget_update(
    mass,
    previous,
    neighbors,
    *,
    keep,
    persistence=0.5,
    min_ratio=0.0,
    candidate_bonus=0.0,
    budget_scale=1.0,
    exploration_fraction=0.0,
    expand_q=True,
    expand_k=True,
    expand_joint=True,
    previous_frontier=None,
    sink_blocks=0,
):
    """Expand only route frontiers, then prune back to a per-row budget.

    ``sink_blocks`` (not in the reference's signature; 0 there) also sets the
    first key-block columns, as the backend's first-frame sink does next
    (flex.py:544-546); ``frontier`` is then that of the final route.
    """
    if previous.shape != mass.shape:
        raise ValueError("previous route and mass must have identical shapes")
    if tuple(neighbors.shape) != (mass.shape[-1], 4):
        raise ValueError("neighbors must have shape [blocks, 4]")
    if budget_scale <= 0:
        raise ValueError("budget_scale must be positive")
    if not 0 <= exploration_fraction <= 1:
        raise ValueError("exploration_fraction must be in [0, 1]")
    result = ops.directional_update(
        mass, previous, neighbors, keep=keep, persistence=persistence, min_ratio=min_ratio,
        candidate_bonus=candidate_bonus, budget_scale=budget_scale,
        exploration_fraction=exploration_fraction, expand_q=expand_q, expand_k=expand_k,
        expand_joint=expand_joint, previous_frontier=previous_frontier,
        sink_blocks=sink_blocks)
    result["frontier"] = ops.frontier_mask(result["route"], neighbors)
    return result

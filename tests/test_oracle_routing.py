"""Pins of the frontier / directional-update oracle (CPU): the reference's
known answers (tests/test_directional_routing.py), golden vectors its own
routing functions wrote on the 720p neighbour table, and planted mistakes."""

from pathlib import Path

import numpy as np
import pytest

from oracle import routing as G
from tests.golden.inputs import random_route, route_mass

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = {
    # Must match tests/golden/make_golden.py ROUTING_CASES.
    "default": (11, 12, 0.625, False, dict(keep=0.625)),
    "tuned": (13, 14, 0.55, True, dict(
        keep=0.625, persistence=0.5, min_ratio=0.5, candidate_bonus=0.25, budget_scale=0.8,
        exploration_fraction=0.02, expand_joint=False)),
    "q_only": (15, 16, 0.4, False, dict(
        keep=0.5, persistence=0.0, budget_scale=1.3, expand_k=False, expand_joint=False)),
}


def _golden():
    return np.load(GOLDEN / "routing.npz", allow_pickle=False)


def _unpack(bits, shape):
    return np.unpackbits(bits, count=int(np.prod(shape))).reshape(shape).astype(bool)


def line_neighbors(blocks):
    """tests/test_directional_routing.py:9-16."""
    neighbors = np.full((blocks, 4), -1, dtype=np.int32)
    for block in range(blocks):
        if block:
            neighbors[block, 2] = block - 1
        if block + 1 < blocks:
            neighbors[block, 3] = block + 1
    return neighbors


def case_inputs(name):
    mass_seed, prev_seed, prev_keep, explicit, kwargs = CASES[name]
    data = _golden()
    neighbors = data["neighbors"]
    mass = route_mass(1, 450, mass_seed).numpy()
    previous = random_route(1, 450, prev_seed, prev_keep).numpy()
    frontier = G.frontier_mask(previous, neighbors) if explicit else None
    return mass, previous, neighbors, frontier, kwargs


def test_known_answer_frontier():
    """test_directional_routing.py:19-24."""
    route = np.zeros((1, 4, 4), dtype=bool)
    route[:, :, 1:3] = True
    frontier = G.frontier_mask(route, line_neighbors(4))
    assert frontier[:, :, 1:3].all()
    assert not frontier[:, :, [0, 3]].any()


def test_known_answer_directional_update():
    """test_directional_routing.py:27-44."""
    blocks = 4
    route = np.eye(blocks, dtype=bool)[None]
    mass = route.astype(np.float32)
    for row in range(blocks - 1):
        mass[0, row, row + 1] = 2.0
    result = G.directional_budget_update(
        mass, route, line_neighbors(blocks), keep=.5, persistence=0, expand_q=False,
        expand_k=True, expand_joint=False)
    updated = result["route"]
    assert (updated.sum(-1) == 1).all()
    assert updated[0, 0, 1] and updated[0, 1, 2] and updated[0, 2, 3] and updated[0, 3, 3]
    assert result["added"].sum() == 3
    assert result["dropped"].sum() == 3


@pytest.mark.parametrize("name", ["frontier_p625", "frontier_p90"])
def test_frontier_matches_reference_golden(name):
    data = _golden()
    seed, keep = data[f"{name}__params"]
    route = random_route(1, 450, int(seed), float(keep)).numpy()
    expected = _unpack(data[f"{name}__frontier"], route.shape)
    np.testing.assert_array_equal(G.frontier_mask(route, data["neighbors"]), expected)


@pytest.mark.parametrize("name", sorted(CASES))
def test_directional_update_matches_reference_golden(name):
    data = _golden()
    mass, previous, neighbors, frontier, kwargs = case_inputs(name)
    checksum = data[f"{name}__checksum"]
    assert abs(mass.astype(np.float64).sum() - checksum[0]) < 1e-6 * abs(checksum[0])
    assert previous.sum() == checksum[1]
    result = G.directional_budget_update(mass, previous, neighbors,
                                         previous_frontier=frontier, **kwargs)
    for key in ("route", "frontier", "candidates", "exploration"):
        expected = _unpack(data[f"{name}__{key}"], mass.shape)
        np.testing.assert_array_equal(result[key], expected, err_msg=key)


def test_frontier_invariants():
    route = random_route(2, 64, 3).numpy()
    nb = line_neighbors(64)
    frontier = G.frontier_mask(route, nb)
    assert not (frontier & ~route).any()
    full = np.ones_like(route)
    assert not G.frontier_mask(full, nb).any()
    none = np.full_like(nb, -1)
    assert not G.frontier_mask(route, none).any()


def test_budget_and_pool_invariants():
    mass, previous, neighbors, _, kwargs = case_inputs("tuned")
    result = G.directional_budget_update(mass, previous, neighbors, **kwargs)
    route = result["route"]
    pool = previous | result["candidates"] | result["exploration"]
    assert not (route & ~pool).any()
    cap = int(np.ceil(450 * kwargs["keep"]))
    budget = np.clip(np.ceil(previous.sum(-1).astype(np.float32)
                             * np.float32(kwargs["budget_scale"])), 1, cap)
    np.testing.assert_array_equal(route.sum(-1), np.minimum(budget, pool.sum(-1)))
    assert not (result["candidates"] & previous).any()


def test_planted_mistakes_fail():
    """Swapping the neighbour axis, dropping the validity test, or selecting
    the lowest-scoring entries each change the golden results."""
    data = _golden()
    route = random_route(1, 450, 21, 0.625).numpy()
    expected = _unpack(data["frontier_p625__frontier"], route.shape)
    nb = data["neighbors"]
    # Query-axis only (forgetting the key axis).
    q_only = np.zeros_like(route)
    for d in range(4):
        t = nb[:, d]
        q_only |= (t >= 0)[None, :, None] & ~route[:, np.maximum(t, 0), :]
    assert not np.array_equal(route & q_only, expected)
    # Treating -1 (no neighbour) as block 0.
    no_valid = np.zeros_like(route)
    for d in range(4):
        t = np.maximum(nb[:, d], 0)
        no_valid |= ~route[:, t, :] | ~route[:, :, t]
    assert not np.array_equal(route & no_valid, expected)
    # Ascending instead of descending selection.
    mass, previous, neighbors, frontier, kwargs = case_inputs("default")
    flipped = G.directional_budget_update(-mass + 2.0, previous, neighbors,
                                          previous_frontier=frontier, **kwargs)
    golden_route = _unpack(data["default__route"], mass.shape)
    assert not np.array_equal(flipped["route"], golden_route)


def test_budget_select_is_row_local():
    """Without neighbours there are no candidates, so the full update's rows
    equal budget_select applied to any subset of rows on its own."""
    rng = np.random.default_rng(5)
    heads, blocks = 2, 40
    mass = (rng.random((heads, blocks, blocks)) ** 4).astype(np.float32)
    previous = rng.random((heads, blocks, blocks)) < 0.3
    neighbors = np.full((blocks, 4), -1)
    kwargs = dict(keep=0.4, persistence=0.5, candidate_bonus=0.5, budget_scale=1.1,
                  exploration_fraction=0.05)
    full = G.directional_budget_update(mass, previous, neighbors, **kwargs)
    assert not full["candidates"].any()
    rows = [0, 7, 39]
    route, exploration = G.budget_select(mass[1, rows], previous[1, rows],
                                         np.zeros((3, blocks), bool), **kwargs)
    np.testing.assert_array_equal(route, full["route"][1, rows])
    np.testing.assert_array_equal(exploration, full["exploration"][1, rows])

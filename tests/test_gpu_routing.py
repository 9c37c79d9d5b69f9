"""GPU parity of the frontier and directional-update kernels against the
oracle (oracle/routing.py, itself equal to the reference's routing.py on the
golden cases): every output is bit-exact."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import routing as G
from tests.golden.inputs import random_route, route_mass
from tests.test_oracle_routing import CASES, case_inputs, line_neighbors

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _dev(x, device):
    return torch.as_tensor(np.ascontiguousarray(x)).to(device)


def test_frontier_known_answer(ops, cuda_device):
    """tests/test_directional_routing.py:19-24."""
    route = torch.zeros(1, 4, 4, dtype=torch.bool)
    route[:, :, 1:3] = True
    frontier, count = ops.frontier_mask(route.to(cuda_device),
                                        _dev(line_neighbors(4), cuda_device), return_count=True)
    torch.cuda.synchronize()
    frontier = frontier.cpu()
    assert frontier[:, :, 1:3].all() and not frontier[:, :, [0, 3]].any()
    assert count.item() == 8


@pytest.mark.parametrize("keep", [0.3, 0.625, 0.9])
def test_frontier_matches_oracle_on_720p_table(ops, cuda_device, keep):
    nb = np.load(GOLDEN / "routing.npz", allow_pickle=False)["neighbors"]
    route = random_route(6, 450, seed=int(keep * 100), keep=keep).numpy()
    frontier, count = ops.frontier_mask(_dev(route, cuda_device), _dev(nb, cuda_device),
                                        return_count=True)
    torch.cuda.synchronize()
    expected = G.frontier_mask(route, nb)
    np.testing.assert_array_equal(frontier.cpu().numpy(), expected)
    assert count.item() == expected.sum()


def test_directional_known_answer(ops, cuda_device):
    """tests/test_directional_routing.py:27-44."""
    blocks = 4
    route = torch.eye(blocks, dtype=torch.bool).unsqueeze(0)
    mass = route.float()
    for row in range(blocks - 1):
        mass[0, row, row + 1] = 2.0
    result = ops.directional_update(
        mass.to(cuda_device), route.to(cuda_device), _dev(line_neighbors(blocks), cuda_device),
        keep=.5, persistence=0, expand_q=False, expand_k=True, expand_joint=False)
    torch.cuda.synchronize()
    updated = result["route"].cpu()
    assert (updated.sum(-1) == 1).all()
    assert updated[0, 0, 1] and updated[0, 1, 2] and updated[0, 2, 3] and updated[0, 3, 3]
    assert result["added"].sum().item() == 3
    assert result["dropped"].sum().item() == 3


@pytest.mark.parametrize("name", sorted(CASES))
def test_directional_matches_oracle_golden_cases(ops, cuda_device, name):
    mass, previous, neighbors, frontier, kwargs = case_inputs(name)
    result = ops.directional_update(
        _dev(mass, cuda_device), _dev(previous, cuda_device), _dev(neighbors, cuda_device),
        previous_frontier=_dev(frontier, cuda_device) if frontier is not None else None,
        **kwargs)
    torch.cuda.synchronize()
    expected = G.directional_budget_update(mass, previous, neighbors,
                                           previous_frontier=frontier, **kwargs)
    for key in ("route", "candidates", "exploration", "dropped", "added"):
        np.testing.assert_array_equal(result[key].cpu().numpy(), expected[key], err_msg=key)
    np.testing.assert_array_equal(result["counts"].cpu().numpy(), expected["route"].sum(-1))


@pytest.mark.parametrize("heads,seed", [(8, 3), (40, 4)])
def test_directional_full_shape_with_sink(ops, cuda_device, heads, seed):
    """40 heads x 450 blocks, exploration, bonus and the 29-column sink."""
    nb = np.load(GOLDEN / "routing.npz", allow_pickle=False)["neighbors"]
    mass = route_mass(heads, 450, seed).numpy()
    previous = random_route(heads, 450, seed + 100, 0.6).numpy()
    kwargs = dict(keep=0.625, persistence=0.5, min_ratio=0.25, candidate_bonus=0.5,
                  budget_scale=1.1, exploration_fraction=0.01)
    result = ops.directional_update(_dev(mass, cuda_device), _dev(previous, cuda_device),
                                    _dev(nb, cuda_device), sink_blocks=29, **kwargs)
    torch.cuda.synchronize()
    expected = G.directional_budget_update(mass, previous, nb, **kwargs)
    route = expected["route"].copy()
    route[..., :29] = True
    np.testing.assert_array_equal(result["route"].cpu().numpy(), route)
    np.testing.assert_array_equal(result["counts"].cpu().numpy(), route.sum(-1))
    for key in ("candidates", "exploration", "dropped", "added"):
        np.testing.assert_array_equal(result[key].cpu().numpy(), expected[key], err_msg=key)


def test_backend_directional_update_uses_frontier(cuda_device):
    """flex_reuse with spatial_reorder + directional_update: the sampled update
    equals the oracle's directional update of the same sampled mass, with the
    state's frontier as the source, then the sink; frontier_fraction is
    reported."""
    from dit_sparse_atten_amd.attention_backends import context, flex
    from tests.golden.inputs import clustered_qkv
    context.reset_runtime_state()
    try:
        grid = (4, 16, 32)
        tokens, heads = 2048, 4
        config = flex.FlexReuseConfig(
            bootstrap_mode="sampled", prefetch_sampled_bootstrap=False,
            sampled_update_interval=1, prefetch_sampled_update=False, route_samples=16,
            mass_target=0.95, keep=0.625, spatial_reorder=True, directional_update=True,
            direction_min_ratio=0.1, total_steps=4)
        backend = flex.FlexReuseBackend(config)
        q, k, v = clustered_qkv(tokens, heads, 128, group=64, seed=5, dtype=torch.bfloat16)
        qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
        context.set_routing_context(attention_id=1, step=0, branch=0, grid=grid)
        backend(qd, kd, vd)
        state = next(iter(backend.state.values()))
        previous = state["route"].clone()
        previous_frontier = state["frontier"].clone()
        assert state["frontier_fraction"] == pytest.approx(
            previous_frontier.float().mean().item(), abs=0)
        layout = state["layout"]
        q2, k2, v2 = clustered_qkv(tokens, heads, 128, group=64, seed=6, dtype=torch.bfloat16)
        q2d, k2d, v2d = (x.to(cuda_device) for x in (q2, k2, v2))
        context.set_routing_context(attention_id=1, step=1, branch=0, grid=grid)
        backend(q2d, k2d, v2d)
        torch.cuda.synchronize()
        assert backend.phase_counts["sampled_update"] == 1
        rq, rk, _ = layout.reorder_qkv(q2d, k2d, v2d)
        mass = flex._sampled_block_mass(rq, rk, 128, samples=16).cpu().numpy()
        nb = layout.neighbors(cuda_device).cpu().numpy()
        expected = G.directional_budget_update(
            mass, previous.cpu().numpy(), nb, keep=0.625, persistence=0.5, min_ratio=0.1,
            previous_frontier=previous_frontier.cpu().numpy())
        route = expected["route"].copy()
        route[..., :4] = True  # ceil(16 * 32 / 128) first-frame blocks
        np.testing.assert_array_equal(state["route"].cpu().numpy(), route)
        np.testing.assert_array_equal(state["frontier"].cpu().numpy(),
                                      G.frontier_mask(route, nb))
    finally:
        context.reset_runtime_state()


@pytest.mark.parametrize("grid,heads", [((21, 45, 80), 2), ((62, 45, 80), 2),
                                        ((84, 45, 80), 1)])
def test_frontier_and_directional_beyond_512_blocks(ops, cuda_device, grid, heads):
    """81 frames at 720p (591 blocks), 244 frames (1,744 blocks) and 333
    frames (2,363 blocks: a workgroup per row): the spatial layout's neighbour
    table, bit-exact against the oracle."""
    from dit_sparse_atten_amd.attention_backends.spatial import build_spatial_layout
    layout = build_spatial_layout(grid, 128, 32)
    nb = layout.neighbors_cpu.numpy()
    blocks = nb.shape[0]
    mass = route_mass(heads, blocks, seed=blocks).numpy()
    previous = random_route(heads, blocks, seed=blocks + 1, keep=0.5).numpy()
    frontier = ops.frontier_mask(_dev(previous, cuda_device), _dev(nb, cuda_device))
    kwargs = dict(keep=0.625, persistence=0.5, min_ratio=0.25, candidate_bonus=0.5,
                  budget_scale=1.1, exploration_fraction=0.01)
    result = ops.directional_update(_dev(mass, cuda_device), _dev(previous, cuda_device),
                                    _dev(nb, cuda_device), sink_blocks=29, **kwargs)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(frontier.cpu().numpy(), G.frontier_mask(previous, nb))
    expected = G.directional_budget_update(mass, previous, nb, **kwargs)
    route = expected["route"].copy()
    route[..., :29] = True
    np.testing.assert_array_equal(result["route"].cpu().numpy(), route)
    np.testing.assert_array_equal(result["counts"].cpu().numpy(), route.sum(-1))


@pytest.mark.parametrize("blocks", [4219, 16384])
def test_directional_rows_up_to_16384_blocks(ops, cuda_device, blocks):
    """Rows of 4,219 and 16,384 (the maximum) blocks.  Without neighbours
    there are no candidates and every row is independent, so sampled rows are
    checked bit-exact against the oracle's row-local selection, which the
    oracle tests show equal to the full update's rows."""
    generator = torch.Generator(device=cuda_device).manual_seed(blocks)
    mass = torch.rand(1, blocks, blocks, device=cuda_device, generator=generator) ** 4
    previous = torch.rand(1, blocks, blocks, device=cuda_device, generator=generator) < 0.3
    nb = torch.full((blocks, 4), -1, dtype=torch.int32, device=cuda_device)
    # A budget below the pool, and a prior small enough that explored blocks
    # compete with previous ones.
    kwargs = dict(keep=0.4, persistence=0.05, candidate_bonus=0.5, budget_scale=0.9,
                  exploration_fraction=0.01)
    result = ops.directional_update(mass, previous, nb, sink_blocks=29, **kwargs)
    torch.cuda.synchronize()
    rows = torch.tensor(sorted({0, 1, blocks // 2, blocks - 1,
                                *torch.randint(0, blocks, (28,), generator=torch.Generator()
                                               .manual_seed(1)).tolist()}))
    m = mass[0, rows.to(cuda_device)].cpu().numpy()
    prev = previous[0, rows.to(cuda_device)].cpu().numpy()
    route, exploration = G.budget_select(m, prev, np.zeros_like(prev), **kwargs)
    sunk = route.copy()
    sunk[:, :29] = True
    got = {name: result[name][0, rows.to(cuda_device)].cpu().numpy()
           for name in ("route", "exploration", "candidates", "dropped", "added")}
    np.testing.assert_array_equal(got["route"], sunk)
    np.testing.assert_array_equal(got["exploration"], exploration)
    assert not got["candidates"].any()
    np.testing.assert_array_equal(got["dropped"], prev & ~route)
    np.testing.assert_array_equal(got["added"], route & ~prev)
    np.testing.assert_array_equal(result["counts"][0, rows.to(cuda_device)].cpu().numpy(),
                                  sunk.sum(-1))

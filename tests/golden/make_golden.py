"""Write the golden fixtures of tests/golden/ by running the reference's own
CPU functions (yangshuo1230/DiT_Sparse_Atten, read-only at /root/reference).

Only functions whose exact output no reference test or closed form pins are
run here:
  * flex._top_mass_route        tie order / fp32 rounding of sum and cumsum
  * flex._sampled_block_mass    sample-index choice and log-weights
  * FlexReuseBackend._sampled_route   persistence prior + selection, also at
    config-3 scale on a reproducible mass (route_config3.npz)
  * spatial.build_spatial_layout      Morton order and majority-vote neighbours
  * sparse.MatrixSparseBackend  config-0 bootstrap route, mass and outputs
  * sparse.MatrixSparseBackend  four steps per policy (reuse / all / directional):
    masks, fp16 mass and centroids, outputs (drop, expansion and statistics)
  * routing.frontier_mask / directional_budget_update   on the 720p block
    neighbour table (the known answers of test_directional_routing.py cover
    one line-shaped case only)
This script runs in the build container only (it reads /root/reference);
tests, smoke() and bench.py read the .npz files it writes and never the
reference.  Regenerate with:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
REFERENCE = Path(os.environ.get("DSA_REFERENCE", "/root/reference"))

from tests.golden.inputs import (  # noqa: E402
    block_mass_like, clustered_qkv, random_route, route_mass)


def _reference_modules():
    if not REFERENCE.exists():
        raise SystemExit(f"reference not found at {REFERENCE}")
    sys.path.insert(0, str(REFERENCE))
    from attention_backends import context, flex, routing, sparse, spatial  # noqa: PLC0415
    return context, flex, routing, sparse, spatial


def _save(name, **arrays):
    path = HERE / f"{name}.npz"
    np.savez_compressed(path, **arrays)
    print(f"wrote {path.name}: {sorted(arrays)} ({path.stat().st_size} bytes)")


def top_mass_fixture(flex):
    rng = np.random.default_rng(20261201)
    cases = {}
    # Softmax-like rows with a heavy head, as block mass looks in practice.
    cases["dirichlet"] = (rng.dirichlet(np.full(450, 0.3), size=(2, 48)).astype(np.float32),
                          0.95, 0.625)
    cases["dirichlet_t90_k50"] = (rng.dirichlet(np.full(450, 0.5), size=(1, 48)).astype(
        np.float32), 0.90, 0.5)
    # Many exact ties, including ties that straddle the selection boundary.
    ties = rng.integers(0, 4, size=(1, 32, 64)).astype(np.float32) / np.float32(64.0)
    ties[0, 0] = 1.0 / 64
    cases["ties"] = (ties, 0.95, 0.625)
    # Rows where the cap, not the target, decides.
    flat = np.full((1, 8, 16), 1.0 / 16, dtype=np.float32)
    cases["flat_cap"] = (flat, 0.95, 0.625)
    cases["known_answer"] = (np.array([[[0.50, 0.30, 0.15, 0.05]]], np.float32), 0.90, 0.50)
    arrays = {}
    for name, (mass, target, keep) in cases.items():
        route = flex._top_mass_route(torch.from_numpy(mass), target, keep).numpy()
        arrays[f"{name}__mass"] = mass
        arrays[f"{name}__route"] = route
        arrays[f"{name}__params"] = np.array([target, keep], dtype=np.float64)
    _save("top_mass_route", **arrays)


def sampled_mass_fixture(flex):
    arrays = {}
    specs = {
        # name: (tokens, heads, head_dim, block, samples, dtype)
        "fp32_partial_s2": (1000, 3, 64, 128, 2, torch.float32),
        "fp32_partial_s16": (1000, 3, 64, 128, 16, torch.float32),
        "bf16_s16": (1024, 2, 128, 128, 16, torch.bfloat16),
        "bf16_partial_s16": (300, 2, 128, 128, 16, torch.bfloat16),
        "f16_partial_s16": (1000, 3, 128, 128, 16, torch.float16),
        "bf16_partial_s12": (1000, 3, 128, 128, 12, torch.bfloat16),
        "bf16_partial_s48": (1000, 2, 128, 128, 48, torch.bfloat16),
    }
    codes = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
    # params: tokens, heads, head_dim, block, samples, dtype (0 fp32, 1 bf16,
    # 2 fp16), seed.
    for index, (name, (tokens, heads, dim, block, samples, dtype)) in enumerate(specs.items()):
        q, k, _ = clustered_qkv(tokens, heads, dim, group=block, seed=100 + index, dtype=dtype)
        mass = flex._sampled_block_mass(q, k, block, samples=samples)
        arrays[f"{name}__checksum"] = np.array([q.double().sum().item(),
                                                k.double().sum().item()])
        arrays[f"{name}__mass"] = mass.numpy()
        arrays[f"{name}__params"] = np.array(
            [tokens, heads, dim, block, samples, codes[dtype], 100 + index])
    _save("sampled_mass", **arrays)


def sampled_route_fixture(flex):
    """Sampled update with a previous route (prior 0.5), no grid: 32 blocks."""
    tokens, heads = 4096, 4
    q, k, _ = clustered_qkv(tokens, heads, 128, group=128, seed=7, dtype=torch.bfloat16)
    generator = torch.Generator().manual_seed(8)
    previous = torch.rand(heads, 32, 32, generator=generator) < 0.625
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        route_samples=16, mass_target=0.95, keep=0.625, route_persistence=0.5))
    state = {"route": previous, "grid": None, "layout": None}
    result = backend._sampled_route(state, q, k, None)
    mass = flex._sampled_block_mass(q, k, 128, samples=16)
    _save("sampled_route", seed=np.array([7, 8]), previous=previous.numpy(),
          mass=mass.numpy(), route=result["route"].numpy())


def route_summary(route):
    """Per-row (count, sum of selected indices, sum of their squares) of a
    boolean route [..., K]: a compact fingerprint of every row's selection."""
    route = np.asarray(route, dtype=bool)
    index = np.arange(route.shape[-1], dtype=np.int64)
    return (route.sum(-1).astype(np.int16), (route * index).sum(-1).astype(np.int32),
            (route * index * index).sum(-1).astype(np.int64))


def route_config3_fixture(flex):
    """The reference's sampled-route selection at config-3 scale (40 heads x
    450 x 450, target .95, keep .625, 29-block first-frame sink of the
    16x45x80 grid): FlexReuseBackend._sampled_route on a reproducible
    softmax-shaped mass (inputs.block_mass_like), without a previous route
    (bootstrap) and with one (persistence prior 0.5).  The mass is injected in
    place of _sampled_block_mass; everything after it (prior, _top_mass_route,
    sink) is the reference's own code.  Stored as per-row fingerprints."""
    heads, blocks, seed, sharpness, previous_seed = 40, 450, 31, 4.0, 32
    mass = block_mass_like(heads, blocks, seed, sharpness=sharpness)
    previous = random_route(heads, blocks, previous_seed)
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        route_samples=16, mass_target=0.95, keep=0.625, route_persistence=0.5))
    original_mass, original_top = flex._sampled_block_mass, flex._top_mass_route
    selected_from = []

    def recording_top_mass_route(primed, target, keep):
        selected_from.append(primed.clone())  # the mass the reference selects from
        return original_top(primed, target, keep)

    flex._sampled_block_mass = lambda *args, **kwargs: mass.clone()
    flex._top_mass_route = recording_top_mass_route
    try:
        arrays = {"params": np.array([heads, blocks, seed, sharpness, previous_seed])}
        dummy = torch.zeros(1, blocks * 128, heads, 1)
        for name, prev in (("bootstrap", None), ("prior", previous)):
            selected_from.clear()
            state = {"route": prev, "grid": (16, 45, 80), "layout": None}
            route = backend._sampled_route(state, dummy, dummy, None)["route"].numpy()
            count, index_sum, square_sum = route_summary(route)
            arrays[f"{name}__count"] = count
            arrays[f"{name}__index_sum"] = index_sum
            arrays[f"{name}__square_sum"] = square_sum
            # Sum of the selected values (sink columns included) in float64: a
            # selection that differs only in which of several equal values it
            # took at the boundary (torch's unstable argsort) has the same sum.
            primed = selected_from[-1].double().numpy()
            arrays[f"{name}__value_sum"] = (primed * route).sum(-1)
    finally:
        flex._sampled_block_mass, flex._top_mass_route = original_mass, original_top
    _save("route_config3", **arrays)


def spatial_fixture(spatial):
    grids = {
        "g2x4x8_b8_m8": ((2, 4, 8), 8, 8),
        "g1x4x64": ((1, 4, 64), 128, 32),
        "g16x45x80": ((16, 45, 80), 128, 32),
        "g21x30x52": ((21, 30, 52), 128, 32),
        "g4x16x16": ((4, 16, 16), 128, 32),
    }
    arrays = {}
    for name, (grid, block, max_tokens) in grids.items():
        layout = spatial.build_spatial_layout(grid, block, max_tokens)
        arrays[f"{name}__params"] = np.array([*grid, block, max_tokens])
        arrays[f"{name}__microtile"] = np.array(layout.microtile_shape)
        arrays[f"{name}__permutation"] = layout.permutation_cpu.numpy()
        arrays[f"{name}__neighbors"] = layout.neighbors_cpu.numpy()
        arrays[f"{name}__block_frames"] = layout.block_frames_cpu.numpy()
    _save("spatial_layout", **arrays)


def sparse_config0_fixture(context, sparse):
    """BASELINE config 0 through MatrixSparseBackend: step 0 then step 1."""
    grid, tile = (4, 16, 16), 64
    tokens, heads = 1024, 12
    layout = sparse._spatial_layout(grid, tile, tokens)
    order = layout.to_tile_major(torch.arange(tokens).view(1, tokens, 1, 1)).flatten()
    q, k, v = clustered_qkv(tokens, heads, 128, group=tile, seed=0, permutation=order)
    backend = sparse.MatrixSparseBackend(sparse.SparseConfig(
        tile=tile, keep=0.625, mass_target=0.95, prefetch_route=False))
    context.reset_runtime_state()
    context._STATE.attention_id = 1
    context._STATE.cfg_branch = 0
    context._STATE.grid_size = grid
    context._STATE.denoising_step = 0
    with torch.no_grad():
        out0 = backend(q, k, v, dtype=torch.float32)
        state = next(iter(backend.state.values()))
        route, mass = state["mask"].clone(), state["mass"].clone()
        context._STATE.denoising_step = 1
        out1 = backend(q, k, v, dtype=torch.float32)
    heads_kept = [0, 7]
    _save("sparse_config0",
          tile_shape=np.array([layout.tile_h, layout.tile_w]),
          order=order.numpy().astype(np.int32),
          route=route.numpy(), mass=mass.float().numpy(),
          checksum=np.array([q.double().sum().item(), k.double().sum().item(),
                             v.double().sum().item()]),
          heads=np.array(heads_kept),
          out0=out0[0, :256, heads_kept].numpy(), out1=out1[0, :256, heads_kept].numpy())


ROUTING_CASES = {
    # name: (mass seed, previous seed, previous keep, explicit previous frontier, kwargs)
    "default": (11, 12, 0.625, False, dict(keep=0.625)),
    "tuned": (13, 14, 0.55, True, dict(
        keep=0.625, persistence=0.5, min_ratio=0.5, candidate_bonus=0.25, budget_scale=0.8,
        exploration_fraction=0.02, expand_joint=False)),
    "q_only": (15, 16, 0.4, False, dict(
        keep=0.5, persistence=0.0, budget_scale=1.3, expand_k=False, expand_joint=False)),
}


def routing_fixture(routing, spatial):
    """frontier_mask and directional_budget_update on the 16x45x80 layout's
    450-block neighbour table (one head; inputs regenerated from seeds)."""
    layout = spatial.build_spatial_layout((16, 45, 80), 128, 32)
    neighbors = layout.neighbors_cpu
    arrays = {"neighbors": neighbors.numpy()}
    for name, seed, keep in (("frontier_p625", 21, 0.625), ("frontier_p90", 22, 0.9)):
        route = random_route(1, 450, seed, keep)
        arrays[f"{name}__params"] = np.array([seed, keep])
        arrays[f"{name}__frontier"] = np.packbits(routing.frontier_mask(route, neighbors).numpy())
    for name, (mass_seed, prev_seed, prev_keep, explicit, kwargs) in ROUTING_CASES.items():
        mass = route_mass(1, 450, mass_seed)
        previous = random_route(1, 450, prev_seed, prev_keep)
        frontier = routing.frontier_mask(previous, neighbors) if explicit else None
        result = routing.directional_budget_update(
            mass, previous, neighbors, previous_frontier=frontier, **kwargs)
        arrays[f"{name}__checksum"] = np.array([mass.double().sum().item(),
                                                float(previous.sum().item())])
        for key in ("route", "frontier", "candidates", "exploration"):
            arrays[f"{name}__{key}"] = np.packbits(result[key].numpy())
    _save("routing", **arrays)


MATRIX_SPARSE_CASES = {
    # name: (grid, heads, policy)
    "g4x16x16_reuse": ((4, 16, 16), 4, "reuse"),
    "g4x16x16_all": ((4, 16, 16), 4, "all"),
    "g4x16x16_directional": ((4, 16, 16), 4, "directional"),
    "g2x24x32_directional": ((2, 24, 32), 3, "directional"),
    "g2x24x32_all": ((2, 24, 32), 3, "all"),
}


def matrix_sparse_fixture(context, sparse):
    """MatrixSparseBackend through steps 0..3 (fresh clustered inputs per
    step): the route state after every step and an output sample."""
    arrays = {}
    for name, (grid, heads, policy) in MATRIX_SPARSE_CASES.items():
        tokens = grid[0] * grid[1] * grid[2]
        backend = sparse.MatrixSparseBackend(sparse.SparseConfig(
            tile=64, keep=0.625, mass_target=0.95, policy=policy, prefetch_route=False))
        layout = sparse._spatial_layout(grid, 64, tokens)
        order = layout.to_tile_major(torch.arange(tokens).view(1, tokens, 1, 1)).flatten()
        arrays[f"{name}__params"] = np.array([*grid, heads, layout.tile_h, layout.tile_w])
        context.reset_runtime_state()
        context._STATE.attention_id = 1
        context._STATE.cfg_branch = 0
        context._STATE.grid_size = grid
        for step in range(4):
            q, k, v = clustered_qkv(tokens, heads, 128, group=64, seed=40 + step,
                                    permutation=order)
            context._STATE.denoising_step = step
            with torch.no_grad():
                out = backend(q, k, v, dtype=torch.float32)
            state = next(iter(backend.state.values()))
            arrays[f"{name}__step{step}_mask"] = np.packbits(state["mask"].numpy())
            arrays[f"{name}__step{step}_mass"] = state["mass"].numpy()
            for key in ("centroid_q_y", "centroid_q_x", "centroid_k_y", "centroid_k_x"):
                arrays[f"{name}__step{step}_{key}"] = state[key].numpy()
            # Output sample: the first 32 tokens (original order), heads 0-1, fp16.
            arrays[f"{name}__step{step}_out"] = out[0, :32, :2].to(torch.float16).numpy()
    _save("matrix_sparse", **arrays)


def main():
    torch.set_num_threads(4)
    context, flex, routing, sparse, spatial = _reference_modules()
    top_mass_fixture(flex)
    sampled_mass_fixture(flex)
    sampled_route_fixture(flex)
    route_config3_fixture(flex)
    spatial_fixture(spatial)
    sparse_config0_fixture(context, sparse)
    routing_fixture(routing, spatial)
    matrix_sparse_fixture(context, sparse)


if __name__ == "__main__":
    main()

"""Pins of the matrix-sparse oracle (CPU) against golden vectors written by
the reference's own MatrixSparseBackend (sparse.py) through four steps of each
next-route policy, plus known answers and planted mistakes of the route ops."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import sparse_path as S
from tests.golden.inputs import clustered_qkv

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = ["g4x16x16_reuse", "g4x16x16_all", "g4x16x16_directional",
         "g2x24x32_directional", "g2x24x32_all"]


def _golden():
    return np.load(GOLDEN / "matrix_sparse.npz", allow_pickle=False)


def run_case(name, steps=4):
    """Yields (step, oracle state, oracle output, golden arrays) per step."""
    data = _golden()
    frames, height, width, heads, tile_h, tile_w = (int(x) for x in data[f"{name}__params"])
    policy = name.split("_", 1)[1]
    case = S.MatrixSparseCase((frames, height, width), tile=64, keep=0.625, mass_target=0.95,
                              policy=policy)
    assert case.case.tile_shape == (tile_h, tile_w)
    tokens = frames * height * width
    order = case.case.permutation
    for step in range(steps):
        q, k, v = clustered_qkv(tokens, heads, 128, group=64, seed=40 + step,
                                permutation=torch.as_tensor(order, dtype=torch.long))
        out = case.step(step, q.numpy(), k.numpy(), v.numpy())
        yield step, case.state, out, data, (heads, case.state["mask"].shape[-1])


@pytest.mark.parametrize("name", CASES)
def test_matches_reference_backend(name):
    for step, state, out, data, (heads, tiles) in run_case(name):
        key = f"{name}__step{step}"
        mask = np.unpackbits(data[f"{key}_mask"], count=heads * tiles * tiles).reshape(
            heads, tiles, tiles).astype(bool)
        np.testing.assert_array_equal(state["mask"], mask, err_msg=f"{key} mask")
        np.testing.assert_allclose(state["mass"].astype(np.float32), data[f"{key}_mass"],
                                   rtol=2e-3, atol=1e-7, err_msg=f"{key} mass")
        for c in ("q_y", "q_x", "k_y", "k_x"):
            np.testing.assert_allclose(state[f"centroid_{c}"].astype(np.float32),
                                       data[f"{key}_centroid_{c}"], atol=2e-3,
                                       err_msg=f"{key} centroid {c}")
        np.testing.assert_allclose(out[0, :32, :2], data[f"{key}_out"].astype(np.float32),
                                   atol=2e-3, rtol=2e-3, err_msg=f"{key} output")


def test_drop_known_answers():
    # One head, 2 x 3 tiles: mean selected mass .25 -> drop below .025 (factor .1).
    mask = np.array([[[1, 1, 0], [1, 0, 0]]], bool)
    mass = np.array([[[0.7, 0.02, 0.9], [0.03, 0.5, 0.4]]], np.float32)
    kept = S.drop_low_mass(mask, mass, 0.1)
    assert kept.tolist() == [[[True, False, False], [True, False, False]]]
    # A row the drop empties keeps its highest-mass original tile.
    mass2 = np.array([[[0.7, 0.02, 0.9], [0.001, 0.5, 0.4]]], np.float32)
    mask2 = np.array([[[1, 1, 0], [1, 0, 0]]], bool)
    kept2 = S.drop_low_mass(mask2, mass2, 0.5)
    assert kept2.tolist() == [[[True, False, False], [True, False, False]]]
    # drop_factor <= 0 keeps the mask.
    assert (S.drop_low_mass(mask, mass, 0.0) == mask).all()


def test_fp16_drop_uses_fp16_threshold():
    """A ratio of exactly fp16(0.1) = 0.0999755859375 is kept: torch compares
    fp16 tensors with fp16(drop_factor).  mean = fp16(2.0 / 2) = 1.0."""
    mask = np.ones((1, 1, 2), bool)
    mass = np.array([[[0.0999755859375, 1.9000244140625]]], np.float16)
    assert S.drop_low_mass(mask, mass, 0.1).tolist() == [[[True, True]]]
    # The same values in fp32 are compared with fp32(0.1) and dropped.
    assert S.drop_low_mass(mask, mass.astype(np.float32), 0.1).tolist() == [[[False, True]]]


def test_spatial_neighbors_known_answer():
    """One routed tile in the middle of a 3x3 grid gains its eight coupled
    neighbours (same shift on the query and key tile), nothing else."""
    grid = np.zeros((1, 1, 3, 3, 1, 3, 3), bool)
    grid[0, 0, 1, 1, 0, 1, 1] = True
    out = S.spatial_neighbors(grid)
    assert out.sum() == 9
    for dy in (-1, 0, 1):
        for dx in (-1, 0, 1):
            assert out[0, 0, 1 + dy, 1 + dx, 0, 1 + dy, 1 + dx]
    corner = np.zeros_like(grid)
    corner[0, 0, 0, 0, 0, 2, 2] = True
    # Shifts that leave either tile's grid are dropped, never wrapped.
    assert S.spatial_neighbors(corner).sum() == 1


def test_directional_steps_known_answer():
    """A non-huge routed tile with centroid directions q=(+1, 0), k=(0, -1)
    adds the Q-only, K-only and joint moves."""
    mask = np.zeros((1, 9, 9), bool)
    mask[0, 4, 4] = True  # tile (1, 1) attends tile (1, 1) on a 3x3 grid
    state = {"mask": mask, "mass": np.full((1, 9, 9), 0.01, np.float16)}
    zeros = np.zeros((1, 9, 9), np.float16)
    state.update({f"centroid_{n}": zeros.copy() for n in ("q_y", "q_x", "k_y", "k_x")})
    state["centroid_q_y"][0, 4, 4] = 0.5
    state["centroid_k_x"][0, 4, 4] = -0.2
    state["mass"][0, 4, 4] = 0.01
    # Huge needs mass >= 2x the mean of the selected (itself): never, so directional.
    out = S.expand(state, "directional", (1, 3, 3), huge_factor=2.0)
    expected = {(4, 4), (7, 4), (4, 3), (7, 3)}  # (q tile, k tile) ids
    assert {tuple(x) for x in np.argwhere(out[0])} == expected
    # Below the threshold: no move.
    state["centroid_q_y"][0, 4, 4] = 0.1
    state["centroid_k_x"][0, 4, 4] = -0.1
    assert np.argwhere(S.expand(state, "directional", (1, 3, 3))[0]).tolist() == [[4, 4]]


def test_planted_mistakes_fail(monkeypatch):
    """Neighbour shifts that wrap around the tile grid, or a drop that ignores
    the one-per-row fallback, disagree with the reference's vectors."""
    name = "g2x24x32_all"
    data = _golden()

    def mask_at(step, heads, tiles):
        return np.unpackbits(data[f"{name}__step{step}_mask"],
                             count=heads * tiles * tiles).reshape(heads, tiles, tiles).astype(bool)

    def wrapped(grid_mask):
        out = grid_mask.copy()
        for dy in (-1, 0, 1):
            for dx in (-1, 0, 1):
                if dy or dx:
                    out |= np.roll(grid_mask, (dy, dx, dy, dx), axis=(2, 3, 5, 6))
        return out

    monkeypatch.setattr(S, "spatial_neighbors", wrapped)
    mismatched = [not (state["mask"] == mask_at(step, heads, tiles)).all()
                  for step, state, _, _, (heads, tiles) in run_case(name, steps=3) if step]
    assert any(mismatched)
    monkeypatch.undo()
    monkeypatch.setattr(S, "preserve_one_per_row", lambda kept, original, mass: kept)
    mass = np.array([[[0.9, 0.9], [0.001, 0.0]]], np.float32)
    mask = np.array([[[1, 1], [1, 0]]], bool)
    assert not S.drop_low_mass(mask, mass, 0.5)[0, 1].any()

"""Pins of the layout and sparse.py-path oracles (CPU): the reference's golden
outputs, its known answers and closed-form invariants."""

from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import route as R
from oracle import sparse_path as SP
from oracle import spatial as S
from tests.golden.inputs import clustered_qkv

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    return np.load(GOLDEN / f"{name}.npz", allow_pickle=False)


@pytest.mark.parametrize("grid,block,max_tokens,shape", [
    ((2, 4, 8), 8, 8, (2, 4)),        # tests/test_spatial_layout.py:6-8
    ((16, 45, 80), 128, 32, (1, 16)),  # tests/test_spatial_layout.py:23-29
    ((1, 4, 64), 128, 32, (4, 8)),     # tests/test_flex_route_update.py:102
])
def test_microtile_known_answers(grid, block, max_tokens, shape):
    assert S.choose_microtile(grid[1], grid[2], block, max_tokens) == shape


def test_morton_code_closed_form():
    for y in range(16):
        for x in range(16):
            expected = sum(((x >> b) & 1) << (2 * b) | ((y >> b) & 1) << (2 * b + 1)
                           for b in range(4))
            assert S.morton_code(y, x) == expected


@pytest.mark.parametrize("name", sorted({k.split("__")[0] for k in _load("spatial_layout").files}))
def test_spatial_layout_matches_reference_golden(name):
    data = _load("spatial_layout")
    grid_h_w = tuple(int(x) for x in data[f"{name}__params"])
    grid, block, max_tokens = grid_h_w[:3], grid_h_w[3], grid_h_w[4]
    layout = S.spatial_layout(grid, block, max_tokens)
    assert layout["microtile"] == tuple(data[f"{name}__microtile"].tolist())
    np.testing.assert_array_equal(layout["permutation"], data[f"{name}__permutation"])
    np.testing.assert_array_equal(layout["neighbors"], data[f"{name}__neighbors"])
    np.testing.assert_array_equal(layout["block_frames"], data[f"{name}__block_frames"])
    # Invariants: bijection, inverse, micro-tiles never straddle blocks.
    tokens = int(np.prod(grid))
    assert sorted(layout["permutation"].tolist()) == list(range(tokens))
    assert (layout["permutation"][layout["inverse"]] == np.arange(tokens)).all()
    area = layout["microtile"][0] * layout["microtile"][1]
    for offset in range(0, tokens, area):
        assert offset // block == (offset + area - 1) // block


def test_720p_layout_counts():
    """tests/test_spatial_layout.py:23-29."""
    layout = S.spatial_layout((16, 45, 80), 128)
    assert layout["permutation"].size == 57600
    assert layout["neighbors"].shape == (450, 4)
    assert (layout["neighbors"] >= 0).any()


def test_sparse_tile_known_answers():
    """sparse.py:113-138 scoring: (4,16,16) tile 64 -> 8x8; (1,60,60) -> 6x10."""
    assert S.sparse_tile_shape((4, 16, 16), 64, 1024) == (8, 8)
    assert S.sparse_tile_shape((1, 60, 60), 64, 3600) == (6, 10)
    assert S.sparse_tile_shape((4, 16, 16), 64, 1000) is None


def test_tile_major_matches_reshape_permute():
    """to_tile_major is reshape(F, bh, th, bw, tw) -> permute(0,1,3,2,4)."""
    grid, tile = (3, 12, 20), (4, 5)
    perm = S.tile_major_permutation(grid, tile)
    ids = np.arange(np.prod(grid)).reshape(3, 3, 4, 4, 5).transpose(0, 1, 3, 2, 4).reshape(-1)
    np.testing.assert_array_equal(perm, ids)


@pytest.fixture(scope="module")
def config0():
    data = _load("sparse_config0")
    order = data["order"]
    q, k, v = clustered_qkv(1024, 12, 128, group=64, seed=0, permutation=order)
    np.testing.assert_allclose(
        [q.double().sum().item(), k.double().sum().item(), v.double().sum().item()],
        data["checksum"])
    return data, q.numpy(), k.numpy(), v.numpy()


def test_config0_layout_matches_reference(config0):
    data, *_ = config0
    case = SP.SparsePathCase((4, 16, 16), tile=64, keep=0.625, mass_target=0.95)
    assert case.tile_shape == tuple(data["tile_shape"].tolist())
    np.testing.assert_array_equal(case.permutation, data["order"])


def test_config0_bootstrap_route_and_outputs_match_reference(config0):
    data, q, k, v = config0
    case = SP.SparsePathCase((4, 16, 16), tile=64, keep=0.625, mass_target=0.95)
    out0 = case.bootstrap(q, k, v)
    heads = data["heads"]
    np.testing.assert_allclose(out0[0, :256][:, heads], data["out0"], atol=2e-5, rtol=1e-4)
    # Route: bit-exact on rows whose decision is not a near tie.
    qt, kt, vt = (case.to_tile_major(x) for x in (q, k, v))
    _, normalized, _ = SP.dense_route(qt, kt, vt, 64, 256, 0.95, 0.625)
    np.testing.assert_allclose(normalized, data["mass"], atol=1e-3, rtol=2e-3)
    _, margins = R.top_mass_route(normalized, 0.95, 0.625, return_margins=True)
    differs = (case.route != data["route"]).any(-1)
    assert not (differs & (margins > 4)).any()
    assert case.route[..., :4].all()  # 2x2 frame-0 tiles form the key sink


def test_config0_sparse_step_matches_reference(config0):
    data, q, k, v = config0
    case = SP.SparsePathCase((4, 16, 16), tile=64, keep=0.625, mass_target=0.95)
    case.route = data["route"]
    out1 = case.step(q, k, v)
    heads = data["heads"]
    np.testing.assert_allclose(out1[0, :256][:, heads], data["out1"], atol=2e-5, rtol=1e-4)
    # sparse_chunk's finfo.min masking equals the closed-form masked softmax.
    tiled = [case.to_tile_major(x) for x in (q, k, v)]
    closed, _ = A.block_sparse_attention(*tiled, data["route"], 64)
    np.testing.assert_allclose(case.to_tile_major(out1), closed, atol=2e-5, rtol=1e-4)


def test_sparse_chunk_stats_rows_sum_to_query_count():
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 256, 2, 16)).astype(np.float32) for _ in range(3))
    route = rng.random((2, 4, 4)) < 0.6
    route[:, np.arange(4), np.arange(4)] = True
    stats = SP.empty_stats(2, 4)
    SP.sparse_chunk(q, k, v, route, 64, 0, 256, 0.25, stats)
    # Each query row's probabilities sum to 1, so a query tile's mass is 64.
    np.testing.assert_allclose(stats["mass"].sum(-1), 64.0, rtol=1e-5)
    assert (stats["mass"][~route] == 0).all()


def test_metrics_known_answers():
    """tests/test_sparse_profile_tools.py:6-20."""
    metrics = A.summarize(np.array([1.0, 2.0]), np.array([1.0, 3.0]))
    assert abs(metrics["relative_l2"] - 0.3162277638912201) < 1e-7
    assert metrics["max_absolute_error"] == 1.0
    assert abs(metrics["cosine_similarity"] - 0.9899494647979736) < 1e-7
    zero = A.summarize(np.zeros(4), np.zeros(4))
    assert zero["relative_l2"] == 0.0 and zero["max_absolute_error"] == 0.0


def test_attention_oracle_full_route_equals_sdpa():
    """Full route == SDPA (tests/test_flex_route_update.py:67-71), torch CPU fp32."""
    torch.manual_seed(0)
    q, k, v = (torch.randn(1, 200, 2, 32) for _ in range(3))
    expected = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)).transpose(1, 2)
    out, _ = A.block_sparse_attention(q.numpy(), k.numpy(), v.numpy(), None, 128)
    ones, _ = A.block_sparse_attention(q.numpy(), k.numpy(), v.numpy(),
                                       np.ones((2, 2, 2), bool), 128)
    np.testing.assert_allclose(out, expected.numpy(), atol=2e-6)
    np.testing.assert_allclose(ones, out, atol=0)


@pytest.mark.parametrize("q_tokens,kv_tokens", [(200, 200), (150, 230), (230, 150)])
def test_attention_oracle_causal_equals_sdpa_is_causal(q_tokens, kv_tokens):
    """causal=True == SDPA(is_causal=True), including SDPA's top-left alignment
    when the query and key lengths differ (torch CPU fp64)."""
    generator = torch.Generator().manual_seed(q_tokens + kv_tokens)
    q = torch.randn(1, q_tokens, 2, 16, generator=generator, dtype=torch.float64)
    k, v = (torch.randn(1, kv_tokens, 2, 16, generator=generator, dtype=torch.float64)
            for _ in range(2))
    expected = torch.nn.functional.scaled_dot_product_attention(
        q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), is_causal=True).transpose(1, 2)
    out, _ = A.block_sparse_attention(q.numpy(), k.numpy(), v.numpy(), None, 64, causal=True)
    np.testing.assert_allclose(out, expected.numpy(), atol=1e-12)
    # A planted mistake (keys k < t instead of k <= t: the diagonal dropped)
    # must not pass the same check.
    scores = np.einsum("bqhd,bkhd->bhqk", q.numpy(), k.numpy()) / 4.0
    strict = np.arange(kv_tokens)[None, :] >= np.arange(q_tokens)[:, None]
    scores = np.where(strict, -np.inf, scores)[:, :, 1:]
    weights = np.exp(scores - scores.max(-1, keepdims=True))
    wrong = np.einsum("bhqk,bkhd->bqhd", weights / weights.sum(-1, keepdims=True), v.numpy())
    assert not np.allclose(wrong, expected.numpy()[:, 1:], atol=1e-3)

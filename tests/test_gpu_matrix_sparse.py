"""GPU parity of the matrix-sparse (``sparse``) backend pieces against the oracle
(oracle/sparse_path.py, itself equal to the reference's sparse.py on the
golden cases): tile statistics within fp32 tolerance of its numpy restatement
on the same bf16 inputs, routes bit-exact given the same mass,
outputs within max-abs 2e-2 / cosine 0.9995."""

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import route as R
from oracle import sparse_path as S
from tests.golden.inputs import clustered_qkv, random_route, route_mass

pytestmark = pytest.mark.gpu

STAT_ATOL = 2e-5     # normalised mass (values ~ 1 / tiles^2 .. 1 / tiles)
CENTROID_ATOL = 2e-3  # fp16 centroids in [-1, 1]


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _tile_major_inputs(grid, heads, seed, tile=64, head_dim=128):
    case = S.SparsePathCase(grid, tile=tile)
    tokens = grid[0] * grid[1] * grid[2]
    q, k, v = clustered_qkv(tokens, heads, head_dim, group=case.tile, seed=seed,
                            permutation=torch.as_tensor(case.permutation, dtype=torch.long),
                            dtype=torch.bfloat16)
    # Tile-major order on both sides.
    perm = torch.as_tensor(case.permutation, dtype=torch.long)
    return case, q[:, perm], k[:, perm], v[:, perm]


def _oracle_stats(case, q, k, v, route=None, scale=None):
    """Oracle statistics (fp32 numpy) of tile-major bf16 inputs; the softmax
    scale defaults to head_dim ** -0.5, as the kernels' does."""
    qf, kf, vf = (x.float().numpy() for x in (q, k, v))
    tokens, heads = qf.shape[1:3]
    tiles = tokens // case.tile
    stats = S.empty_stats(heads, tiles)
    offsets = S.spatial_offsets(case.tile_shape, tiles)
    if scale is None:
        scale = qf.shape[-1] ** -0.5
    if route is None:
        _, _, out = S.dense_route(qf, kf, vf, case.tile, 256, 0.95, 0.625, scale, stats, offsets)
    else:
        out = np.empty_like(qf)
        for start in range(0, tokens, case.tile * 4):
            end = min(start + case.tile * 4, tokens)
            out[:, start:end] = S.sparse_chunk(qf, kf, vf, route, case.tile, start, end, scale,
                                               stats, offsets)
    den = np.maximum(stats["mass"], np.float32(1e-12))
    expected = {"mass": (stats["mass"] / np.float32(tokens)).astype(np.float32)}
    for name in ("q_y", "q_x", "k_y", "k_x"):
        expected[f"centroid_{name}"] = (stats[name] / den).astype(np.float32)
    return expected, out


def _compare_stats(got, expected, rtol=2e-3):
    np.testing.assert_allclose(got["mass"].cpu().numpy(), expected["mass"], atol=STAT_ATOL,
                               rtol=rtol)
    np.testing.assert_allclose(got["mass_f16"].float().cpu().numpy(), expected["mass"],
                               atol=STAT_ATOL, rtol=rtol)
    for name in ("q_y", "q_x", "k_y", "k_x"):
        key = f"centroid_{name}"
        np.testing.assert_allclose(got[key].float().cpu().numpy(), expected[key],
                                   atol=CENTROID_ATOL, err_msg=key)


@pytest.mark.parametrize("grid,tile", [((4, 16, 16), 64), ((2, 18, 32), 64), ((2, 24, 32), 64),
                                       ((1, 44, 100), 4), ((2, 15, 26), 64), ((1, 20, 30), 100)])
def test_dense_tile_stats_match_oracle(ops, cuda_device, grid, tile):
    """Tiles of 8x8 (64 tokens), 9x8 (72 tokens, gathered key stream, 3 waves),
    2x2 (1,100 tiles: more than 1,024 per row), 5x13 (65 tokens padded to 72)
    and 10x10 (100 tokens padded to 104, 4 waves)."""
    case, q, k, v = _tile_major_inputs(grid, 3, seed=sum(grid), tile=tile)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    got = ops.tile_stats(qd, kd, lse, case.tile_shape)
    torch.cuda.synchronize()
    expected, _ = _oracle_stats(case, q, k, v)
    _compare_stats(got, expected)
    # Every query row of the dense softmax sums to one: rows of mass sum to tile / tokens.
    np.testing.assert_allclose(got["mass"].sum(-1).cpu().numpy(),
                               case.tile / q.shape[1], rtol=1e-4)


@pytest.mark.parametrize("grid,tile", [((4, 16, 16), 64), ((2, 18, 32), 64), ((2, 15, 26), 64),
                                       ((1, 20, 30), 100)])
def test_routed_tile_attention_and_stats_match_oracle(ops, cuda_device, grid, tile):
    case, q, k, v = _tile_major_inputs(grid, 2, seed=7, tile=tile)
    tiles = q.shape[1] // case.tile
    route = random_route(2, tiles, seed=3, keep=0.5).numpy()
    route[..., 0] = True
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=case.tile)
    out, lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=case.tile)
    got = ops.tile_stats(qd, kd, lse, case.tile_shape, csr=csr)
    torch.cuda.synchronize()
    expected, expected_out = _oracle_stats(case, q, k, v, route)
    _compare_stats(got, expected)
    metrics = A.summarize(out.float().cpu().numpy(), expected_out)
    assert metrics["max_absolute_error"] <= 2e-2 and metrics["cosine_similarity"] >= 0.9995
    assert (got["mass"].cpu().numpy()[~route] == 0).all()


@pytest.mark.parametrize("routed", [True, False])
def test_tile_stats_every_tile_size(ops, cuda_device, routed):
    """Tiles of 1..128 tokens (as 1 x t rows, 5 tiles per head) through every
    statistics variant they select (2, 3 or 4 waves; one or two half-tiles;
    the gathered stream for 65..88 and 97..120) against the oracle."""
    import types
    failures = []
    for t in range(1, 129):
        tiles = 5
        tokens = tiles * t
        q, k, v = clustered_qkv(tokens, 2, 128, group=t, seed=t, dtype=torch.bfloat16)
        case = types.SimpleNamespace(tile=t, tile_shape=(1, t))
        qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
        if routed:
            route = random_route(2, tiles, seed=t, keep=0.6).numpy()
            route[..., tiles - 1] = True
            csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=t)
            _, lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=t)
            got = ops.tile_stats(qd, kd, lse, (1, t), csr=csr)
            expected, _ = _oracle_stats(case, q, k, v, route)
        else:
            _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
            got = ops.tile_stats(qd, kd, lse, (1, t))
            expected, _ = _oracle_stats(case, q, k, v)
        torch.cuda.synchronize()
        try:
            _compare_stats(got, expected)
        except AssertionError as error:
            failures.append((t, str(error)[:200]))
    assert not failures, failures


def test_routed_tile_stats_skip_out_of_range_tiles(ops, cuda_device):
    """Out-of-range key tiles in a CSR row are skipped by the gathered
    statistics stream wherever they fall, and their cells stay zero."""
    case, q, k, v = _tile_major_inputs((2, 18, 32), 1, seed=11)
    tiles = q.shape[1] // case.tile
    route = random_route(1, tiles, seed=4, keep=0.5).numpy()
    route[..., 0] = True
    rows, bad = [], [-1, tiles, tiles + 5, 1 << 20]
    for qt in range(tiles):
        cols = np.flatnonzero(route[0, qt]).tolist()
        cols.insert(qt % (len(cols) + 1), bad[qt % len(bad)])
        rows.append(cols)
    row_ptr = torch.tensor([0] + np.cumsum([len(r) for r in rows]).tolist(), dtype=torch.int32)
    col_idx = torch.tensor([c for r in rows for c in r], dtype=torch.int32)
    counts = torch.tensor([len(r) for r in rows], dtype=torch.int32)
    csr = ops.RouteCSR(row_ptr.to(cuda_device), col_idx.to(cuda_device), counts.to(cuda_device),
                       1, 1, tiles, tiles, case.tile)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    valid_csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=case.tile)
    _, lse = ops.bsa_fwd(qd, kd, vd, valid_csr, return_lse=True, block_size=case.tile)
    got = ops.tile_stats(qd, kd, lse, case.tile_shape, csr=csr)
    torch.cuda.synchronize()
    expected, _ = _oracle_stats(case, q, k, v, route)
    _compare_stats(got, expected)


@pytest.mark.parametrize("grid,tile,deterministic", [
    ((2, 18, 32), 64, True),    # 9 x 8 = 72 tokens: gathered stream
    ((2, 18, 32), 64, False),   # the same with the aligned walk
    ((2, 15, 26), 64, True),    # 5 x 13 = 65 tokens padded to 72
    ((1, 20, 30), 100, False),  # 10 x 10 = 100 tokens padded to 104
    ((4, 16, 16), 64, True),    # 8 x 8 = 64 tokens: plain stream, 2-wave workgroups
    ((4, 16, 16), 64, False),   # the same with the aligned walk
    ((2, 14, 21), 49, True),    # 7 x 7 = 49 tokens: 2-wave workgroups
    ((2, 12, 16), 96, True),    # 12 x 8 = 96 tokens: 64 + 32 key slots per tile
    ((2, 22, 22), 121, False),  # 11 x 11 = 121 tokens: two 64-key half-tiles per tile
    ((2, 16, 32), 128, True),   # 8 x 16 = 128 tokens
])
def test_fused_step_matches_two_pass_and_oracle(ops, cuda_device, grid, tile, deterministic):
    """dsa_bsa_fwd_tile_stats (attention and the statistics of the same
    softmax in one call) against the separate attention + tile_stats passes
    and the oracle's sparse_chunk: output, LSE, mass and centroids; cells the
    route does not list are zero."""
    case, q, k, v = _tile_major_inputs(grid, 2, seed=sum(grid), tile=tile)
    tiles = q.shape[1] // case.tile
    route = random_route(2, tiles, seed=9, keep=0.55).numpy()
    route[..., 0] = True
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=case.tile)
    out, lse, got = ops.bsa_fwd_tile_stats(qd, kd, vd, csr, case.tile_shape,
                                           deterministic=deterministic)
    ref_out, ref_lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=case.tile,
                                   deterministic=True)
    two_pass = ops.tile_stats(qd, kd, ref_lse, case.tile_shape, csr=csr)
    torch.cuda.synchronize()
    if deterministic:
        assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
    expected, expected_out = _oracle_stats(case, q, k, v, route)
    _compare_stats(got, expected)
    metrics = A.summarize(out.float().cpu().numpy(), expected_out)
    assert metrics["max_absolute_error"] <= 2e-2 and metrics["cosine_similarity"] >= 0.9995
    np.testing.assert_allclose(got["mass"].cpu().numpy(), two_pass["mass"].cpu().numpy(),
                               atol=STAT_ATOL, rtol=2e-3)
    assert (got["mass"].cpu().numpy()[~route] == 0).all()
    # Every query row's mass over its tiles sums to one.
    np.testing.assert_allclose(got["mass"].sum(-1).cpu().numpy(), case.tile / q.shape[1],
                               rtol=2e-3)


@pytest.mark.parametrize("grid,tile", [((2, 18, 32), 64), ((2, 15, 26), 64), ((1, 20, 30), 100),
                                       ((2, 16, 32), 128), ((4, 16, 16), 64), ((2, 12, 16), 96),
                                       ((1, 18, 27), 81), ((2, 22, 22), 121), ((2, 14, 21), 49),
                                       ((2, 12, 12), 36)])
def test_fused_dense_step_matches_oracle(ops, cuda_device, grid, tile):
    """The dense bootstrap through dsa_bsa_fwd_tile_stats (no CSR), every
    tile shape with its statistics from the attention launch: 9 x 8, 8 x 8,
    12 x 8 and 8 x 16 tiles (a multiple of 8 of 64..128 tokens) on 128-token
    blocks, unsplit; 5 x 13, 10 x 10, 9 x 9 and 11 x 11 on blocks of one tile
    (4 waves); 7 x 7 and 6 x 6 on blocks of one tile in 2-wave workgroups; all
    against the oracle's _dense_route statistics and output."""
    case, q, k, v = _tile_major_inputs(grid, 3, seed=sum(grid) + 1, tile=tile)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    out, lse, got = ops.bsa_fwd_tile_stats(qd, kd, vd, None, case.tile_shape)
    ref_out, ref_lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out) or (out.float() - ref_out.float()).abs().max().item() <= 8e-3
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse.cpu().numpy(), atol=1e-4)
    expected, expected_out = _oracle_stats(case, q, k, v)
    _compare_stats(got, expected)
    metrics = A.summarize(out.float().cpu().numpy(), expected_out)
    assert metrics["max_absolute_error"] <= 2e-2 and metrics["cosine_similarity"] >= 0.9995
    np.testing.assert_allclose(got["mass"].sum(-1).cpu().numpy(), case.tile / q.shape[1],
                               rtol=2e-3)


@pytest.mark.parametrize("grid,tile,head_dim,dtype", [
    ((2, 16, 16), 64, 256, torch.bfloat16), ((2, 14, 21), 49, 256, torch.bfloat16),
    ((2, 16, 32), 128, 192, torch.bfloat16), ((1, 22, 22), 121, 136, torch.bfloat16),
    ((2, 18, 32), 72, 256, torch.float16)])
@pytest.mark.parametrize("routed", [True, False])
def test_fused_step_wide_heads(ops, cuda_device, grid, tile, head_dim, dtype, routed):
    """Head dims 136..256 through dsa_bsa_fwd_tile_stats: the fp32-compute
    kernel on blocks of one tile, whose first 128-dim launch also writes the
    statistics (S runs over every dim in both), against the oracle's
    sparse_chunk / _dense_route and against bsa_fwd on the same route."""
    case, q, k, v = _tile_major_inputs(grid, 2, seed=head_dim + tile, tile=tile,
                                       head_dim=head_dim)
    q, k, v = (x.to(dtype) for x in (q, k, v))
    tiles = q.shape[1] // case.tile
    route = None
    csr = None
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    if routed:
        route = random_route(2, tiles, seed=tile, keep=0.55).numpy()
        route[..., 0] = True
        csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=case.tile)
    out, lse, got = ops.bsa_fwd_tile_stats(qd, kd, vd, csr, case.tile_shape, deterministic=True)
    ref_out, ref_lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=case.tile,
                                   deterministic=True)
    torch.cuda.synchronize()
    assert torch.equal(out, ref_out)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse.cpu().numpy(), atol=1e-5)
    expected, expected_out = _oracle_stats(case, q, k, v, route)
    _compare_stats(got, expected)
    metrics = A.summarize(out.float().cpu().numpy(), expected_out)
    assert metrics["max_absolute_error"] <= 2e-2 and metrics["cosine_similarity"] >= 0.9995
    if routed:
        assert (got["mass"].cpu().numpy()[~route] == 0).all()
    np.testing.assert_allclose(got["mass"].sum(-1).cpu().numpy(), case.tile / q.shape[1],
                               rtol=2e-3)


@pytest.mark.parametrize("routed", [True, False])
def test_fused_step_every_tile_size(ops, cuda_device, routed):
    """dsa_bsa_fwd_tile_stats at tiles of 1..128 tokens (as 1 x t rows, 5
    tiles per head), routed and dense, through every statistics instance they
    select (2 or 4 waves; one or two half-tiles, the second of at most 32
    keys or not; the gathered stream for 65..88 and 97..120; dense 128-token
    blocks for multiples of 8 from 64) against the oracle: the statistics and
    the output.  The fused sums take each probability in bf16, as P V does
    (relative error up to 2^-8 per term), so cells of a few keys, such as the
    one-key cells of 1-token tiles, are held to rtol 4e-3."""
    import types
    failures = []
    for t in range(1, 129):
        tiles = 5
        tokens = tiles * t
        q, k, v = clustered_qkv(tokens, 2, 128, group=t, seed=t, dtype=torch.bfloat16)
        case = types.SimpleNamespace(tile=t, tile_shape=(1, t))
        qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
        route = None
        csr = None
        if routed:
            route = random_route(2, tiles, seed=t, keep=0.6).numpy()
            route[..., tiles - 1] = True
            csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=t)
        out, _, got = ops.bsa_fwd_tile_stats(qd, kd, vd, csr, (1, t), deterministic=True)
        torch.cuda.synchronize()
        expected, expected_out = _oracle_stats(case, q, k, v, route)
        try:
            _compare_stats(got, expected, rtol=4e-3)
            metrics = A.summarize(out.float().cpu().numpy(), expected_out)
            assert metrics["max_absolute_error"] <= 2e-2, metrics
            assert metrics["cosine_similarity"] >= 0.9995, metrics
        except AssertionError as error:
            failures.append((t, str(error)[:200]))
    assert not failures, failures


@pytest.mark.parametrize("routed", [True, False])
def test_fused_step_fp16_tile_sizes(ops, cuda_device, routed):
    """The fp16 instances of every statistics variant (2 or 4 waves, one or
    two half-tiles, the gathered stream, the dense token stream) at
    representative tile sizes, against the oracle on the same fp16 inputs."""
    import types
    failures = []
    for t in (1, 16, 33, 48, 64, 72, 81, 96, 100, 121, 128):
        tiles = 5
        q, k, v = clustered_qkv(tiles * t, 2, 128, group=t, seed=t, dtype=torch.float16)
        case = types.SimpleNamespace(tile=t, tile_shape=(1, t))
        qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
        route = None
        csr = None
        if routed:
            route = random_route(2, tiles, seed=t, keep=0.6).numpy()
            route[..., tiles - 1] = True
            csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=t)
        out, _, got = ops.bsa_fwd_tile_stats(qd, kd, vd, csr, (1, t), deterministic=True)
        torch.cuda.synchronize()
        assert out.dtype == torch.float16
        expected, expected_out = _oracle_stats(case, q, k, v, route)
        try:
            # fp16 probabilities: 2^-11 per term.
            _compare_stats(got, expected, rtol=2e-3)
            metrics = A.summarize(out.float().cpu().numpy(), expected_out)
            assert metrics["max_absolute_error"] <= 2e-2, metrics
            assert metrics["cosine_similarity"] >= 0.9995, metrics
        except AssertionError as error:
            failures.append((t, str(error)[:200]))
    assert not failures, failures


@pytest.mark.parametrize("fused", [True, False])
def test_reference_statistics_case(ops, cuda_device, fused):
    """The reference's own statistics known-answer case
    (tests/test_sparse_triton_stats.py:15-50): 3,600 tokens on a 1 x 60 x 60
    grid (6 x 10 tiles of 60 tokens, 60 tiles), 4 heads, head dim 128, unit
    normal bf16 Q/K/V, route ``rand < 0.625`` plus the diagonal, the query
    chunk 0..240 through the oracle's sparse_chunk and the reference's
    tolerances: output atol 2e-3 / rtol 2e-2, raw mass atol 2e-3 / rtol 2e-3,
    centroids atol 2e-3 / rtol 2e-2. The whole sequence is also checked
    against the oracle at the same tolerances."""
    torch.manual_seed(0)
    tokens, heads, head_dim, grid = 3600, 4, 128, (1, 60, 60)
    q = torch.randn(1, tokens, heads, head_dim).to(torch.bfloat16)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    tile_shape = S.sparse_tile_shape(grid, 64, tokens)
    tile = tile_shape[0] * tile_shape[1]
    tiles = tokens // tile
    assert (tile_shape, tiles) == ((6, 10), 60)
    route = torch.rand(heads, tiles, tiles) < 0.625
    route[:, torch.arange(tiles), torch.arange(tiles)] = True
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    csr = ops.route_to_csr(route.to(cuda_device), block_size=tile)
    if fused:
        out, _, got = ops.bsa_fwd_tile_stats(qd, kd, vd, csr, tile_shape)
    else:
        out, lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=tile)
        got = ops.tile_stats(qd, kd, lse, tile_shape, csr=csr)
    torch.cuda.synchronize()
    out = out.float().cpu().numpy()
    raw_mass = got["mass"].cpu().numpy() * np.float32(tokens)
    centroids = {n: got[f"centroid_{n}"].float().cpu().numpy() for n in ("q_y", "q_x", "k_y", "k_x")}

    qf, kf, vf = (x.float().numpy() for x in (q, k, v))
    route_np = route.numpy()
    offsets = S.spatial_offsets(tile_shape, tiles)
    scale = head_dim ** -0.5
    for stop in (240, tokens):
        stats = S.empty_stats(heads, tiles)
        expected = np.concatenate([
            S.sparse_chunk(qf, kf, vf, route_np, tile, start, min(start + 240, stop), scale,
                           stats, offsets)
            for start in range(0, stop, 240)], axis=1)
        rows = stop // tile
        np.testing.assert_allclose(out[:, :stop], expected, atol=2e-3, rtol=2e-2)
        np.testing.assert_allclose(raw_mass[:, :rows], stats["mass"][:, :rows], atol=2e-3,
                                   rtol=2e-3)
        den = np.maximum(stats["mass"], np.float32(1e-12))
        for name, value in centroids.items():
            np.testing.assert_allclose(value[:, :rows], (stats[name] / den)[:, :rows],
                                       atol=2e-3, rtol=2e-2, err_msg=name)
    assert (raw_mass[~route_np] == 0).all()


@pytest.mark.parametrize("tile_shape,tiles", [((5, 8), 400), ((8, 8), 250), ((3, 8), 666)])
def test_small_tiles_at_scale(ops, cuda_device, tile_shape, tiles):
    """Tiles of at most 64 tokens (2-wave workgroups, one staged block at a
    time) over several rounds of workgroups, so the work queue and the split
    tail run: fused statistics against the separate deterministic passes on
    every cell, attention against an fp32 softmax over the routed keys on
    sampled query tiles."""
    heads, head_dim = 8, 128
    tile = tile_shape[0] * tile_shape[1]
    tokens = tiles * tile
    generator = torch.Generator().manual_seed(tiles)
    q, k, v = (torch.randn(1, tokens, heads, head_dim, generator=generator).to(torch.bfloat16)
               for _ in range(3))
    route = random_route(heads, tiles, seed=tile, keep=0.6)
    route[..., 0] = True
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    csr = ops.route_to_csr(route.to(cuda_device), block_size=tile)
    out, lse, got = ops.bsa_fwd_tile_stats(qd, kd, vd, csr, tile_shape)
    _, ref_lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=tile,
                             deterministic=True)
    two_pass = ops.tile_stats(qd, kd, ref_lse, tile_shape, csr=csr)
    torch.cuda.synchronize()
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse.cpu().numpy(), atol=1e-4)
    for name in ("mass", "mass_f16"):
        np.testing.assert_allclose(got[name].float().cpu().numpy(),
                                   two_pass[name].float().cpu().numpy(), atol=STAT_ATOL,
                                   rtol=2e-3, err_msg=name)
    for name in ("centroid_q_y", "centroid_q_x", "centroid_k_y", "centroid_k_x"):
        np.testing.assert_allclose(got[name].float().cpu().numpy(),
                                   two_pass[name].float().cpu().numpy(), atol=CENTROID_ATOL,
                                   err_msg=name)
    assert (got["mass"].cpu().numpy()[~route.numpy()] == 0).all()
    scale = head_dim ** -0.5
    for h in (0, heads - 1):
        for qt in (0, 1, tiles // 2, tiles - 1):
            rows = slice(qt * tile, (qt + 1) * tile)
            keys = torch.repeat_interleave(route[h, qt], tile)
            qf = q[0, rows, h].float()
            kf, vf = k[0, keys, h].float(), v[0, keys, h].float()
            p = torch.softmax(qf @ kf.T * scale, dim=-1)
            expected = (p @ vf).numpy()
            metrics = A.summarize(out[0, rows, h].float().cpu().numpy(), expected)
            assert metrics["max_absolute_error"] <= 2e-2, (h, qt, metrics)
            assert metrics["cosine_similarity"] >= 0.9995, (h, qt, metrics)


def test_fused_step_at_720p_tile_shape(ops, cuda_device):
    """The bench's 720p matrix-sparse step shape (9 x 8 tiles, 800 tiles
    per head) at 4 heads: fused statistics against the two-pass statistics on
    every cell, and the oracle on sampled query tiles."""
    case, q, k, v = _tile_major_inputs((16, 45, 80), 4, seed=21, tile=64)
    tiles = q.shape[1] // case.tile
    route = random_route(4, tiles, seed=2, keep=0.625).numpy()
    route[..., :4] = True
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=case.tile)
    out, lse, got = ops.bsa_fwd_tile_stats(qd, kd, vd, csr, case.tile_shape)
    _, ref_lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=case.tile)
    two_pass = ops.tile_stats(qd, kd, ref_lse, case.tile_shape, csr=csr)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out).all())
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse.cpu().numpy(), atol=1e-4)
    for name in ("mass", "mass_f16"):
        np.testing.assert_allclose(got[name].float().cpu().numpy(),
                                   two_pass[name].float().cpu().numpy(), atol=STAT_ATOL,
                                   rtol=2e-3, err_msg=name)
    for name in ("centroid_q_y", "centroid_q_x", "centroid_k_y", "centroid_k_x"):
        np.testing.assert_allclose(got[name].float().cpu().numpy(),
                                   two_pass[name].float().cpu().numpy(), atol=CENTROID_ATOL,
                                   err_msg=name)
    # Sampled query tiles of head 0 against the oracle's sparse_chunk.
    qf, kf, vf = (x[:, :, :1].float().numpy() for x in (q, k, v))
    stats = S.empty_stats(1, tiles)
    offsets = S.spatial_offsets(case.tile_shape, tiles)
    for qt in (0, 1, 399, 799):
        start = qt * case.tile
        S.sparse_chunk(qf, kf, vf, route[:1], case.tile, start, start + case.tile,
                       128 ** -0.5, stats, offsets)
        want = stats["mass"][0, qt] / np.float32(q.shape[1])
        np.testing.assert_allclose(got["mass"][0, qt].cpu().numpy(), want, atol=STAT_ATOL,
                                   rtol=2e-3, err_msg=f"query tile {qt}")


def test_route_select_up_to_2048_tiles(ops, cuda_device):
    """The 720p tile route has 800 key tiles per row at 61 frames and 1,050 at
    81 frames (one-wave sorts of 1,024 and 2,048 keys)."""
    rng = np.random.default_rng(5)
    for keys in (513, 800, 1024, 1050, 2048):
        mass = rng.dirichlet(np.full(keys, 0.3), size=(3, 40)).astype(np.float32)
        route, counts = ops.route_select(torch.from_numpy(mass).to(cuda_device), 0.95, 0.625,
                                         sink_blocks=100)
        torch.cuda.synchronize()
        expected = R.top_mass_route(mass, 0.95, 0.625)
        expected[..., :100] = True
        np.testing.assert_array_equal(route.cpu().numpy(), expected)
        np.testing.assert_array_equal(counts.cpu().numpy(), expected.sum(-1))


def test_tile_path_beyond_2048_tiles(ops, cuda_device):
    """2,400 tiles of 2x2 tokens (one head), every step the sparse backend
    runs past 2,048 tiles: dense and routed statistics (the 2 KB `listed`
    bitmap), the tile route (a workgroup per row), drop and both expansions,
    against the oracle."""
    case, q, k, v = _tile_major_inputs((1, 60, 160), 1, seed=21, tile=4)
    tiles = q.shape[1] // case.tile
    assert tiles == 2400
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    dense = ops.tile_stats(qd, kd, lse, case.tile_shape)
    torch.cuda.synchronize()
    expected, _ = _oracle_stats(case, q, k, v)
    _compare_stats(dense, expected)
    mask, counts = ops.route_select(dense["mass"], 0.9, 0.625, sink_blocks=80)
    torch.cuda.synchronize()
    expected_mask = R.top_mass_route(dense["mass"].cpu().numpy(), 0.9, 0.625)
    expected_mask[..., :80] = True
    np.testing.assert_array_equal(mask.cpu().numpy(), expected_mask)
    np.testing.assert_array_equal(counts.cpu().numpy(), expected_mask.sum(-1))

    route = random_route(1, tiles, seed=3, keep=0.05).numpy()
    route[..., 0] = True
    csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=case.tile)
    out, lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=case.tile)
    routed = ops.tile_stats(qd, kd, lse, case.tile_shape, csr=csr)
    torch.cuda.synchronize()
    expected, expected_out = _oracle_stats(case, q, k, v, route)
    _compare_stats(routed, expected)
    metrics = A.summarize(out.float().cpu().numpy(), expected_out)
    assert metrics["max_absolute_error"] <= 2e-2 and metrics["cosine_similarity"] >= 0.9995
    assert (routed["mass"].cpu().numpy()[~route] == 0).all()

    mass16 = routed["mass_f16"].cpu().numpy()
    dropped, counts = ops.drop_low_mass(torch.from_numpy(route).to(cuda_device),
                                        routed["mass_f16"], 0.1, sink_tiles=80)
    torch.cuda.synchronize()
    expected_drop = S.drop_low_mass(route, mass16, 0.1)
    expected_drop[..., :80] = True
    np.testing.assert_array_equal(dropped.cpu().numpy(), expected_drop)
    np.testing.assert_array_equal(counts.cpu().numpy(), expected_drop.sum(-1))

    state = {"mask": route, "mass": mass16}
    names = ("q_y", "q_x", "k_y", "k_x")
    for name in names:
        state[f"centroid_{name}"] = routed[f"centroid_{name}"].cpu().numpy()
    grid_tiles = (1, 30, 80)
    for policy in ("all", "directional"):
        expanded = ops.expand_route(torch.from_numpy(route).to(cuda_device), grid_tiles, policy,
                                    mass=routed["mass_f16"],
                                    centroids=[routed[f"centroid_{n}"] for n in names])
        torch.cuda.synchronize()
        np.testing.assert_array_equal(expanded.cpu().numpy(),
                                      S.expand(state, policy, grid_tiles), err_msg=policy)


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("heads,tiles,drop", [(4, 16, 0.1), (8, 800, 0.1), (4, 100, 1.5)])
def test_drop_low_mass_bit_exact(ops, cuda_device, dtype, heads, tiles, drop):
    mass = (route_mass(heads, tiles, seed=tiles) / tiles).to(dtype)
    mask = random_route(heads, tiles, seed=tiles + 1, keep=0.6).numpy()
    mask[0, 3] = False  # an empty row stays empty
    out, counts = ops.drop_low_mass(torch.from_numpy(mask).to(cuda_device),
                                    mass.to(cuda_device), drop, sink_tiles=4)
    torch.cuda.synchronize()
    mnp = mass.numpy() if dtype == torch.float16 else mass.float().numpy()
    expected = S.drop_low_mass(mask, mnp, drop)
    expected[..., :4] = True
    np.testing.assert_array_equal(out.cpu().numpy(), expected)
    np.testing.assert_array_equal(counts.cpu().numpy(), expected.sum(-1))


@pytest.mark.parametrize("policy", ["all", "directional"])
@pytest.mark.parametrize("grid_tiles", [(4, 2, 2), (2, 3, 4), (16, 5, 10)])
def test_expand_route_bit_exact(ops, cuda_device, policy, grid_tiles):
    heads = 3
    tiles = math.prod(grid_tiles)
    mask = random_route(heads, tiles, seed=tiles, keep=0.3).numpy()
    rng = np.random.default_rng(tiles)
    state = {"mask": mask,
             "mass": (rng.random((heads, tiles, tiles)) ** 4 / tiles).astype(np.float16)}
    for name in ("q_y", "q_x", "k_y", "k_x"):
        state[f"centroid_{name}"] = rng.uniform(-0.6, 0.6, (heads, tiles, tiles)).astype(
            np.float16)
    centroids = [torch.from_numpy(state[f"centroid_{n}"]).to(cuda_device)
                 for n in ("q_y", "q_x", "k_y", "k_x")]
    out = ops.expand_route(torch.from_numpy(mask).to(cuda_device), grid_tiles, policy,
                           mass=torch.from_numpy(state["mass"]).to(cuda_device),
                           centroids=centroids)
    torch.cuda.synchronize()
    expected = S.expand(state, policy, grid_tiles)
    np.testing.assert_array_equal(out.cpu().numpy(), expected)


@pytest.mark.parametrize("policy", ["reuse", "all", "directional"])
def test_backend_steps_match_oracle(ops, cuda_device, policy):
    """Four steps of MatrixSparseBackend on a 9x8-tile grid.  At every step the
    output matches the oracle's attention over the route the backend used, and
    the stored mask equals the oracle's selection (step 0) or drop + sink
    (later steps) of the same mass, recomputed with the same kernels; the
    route used is the oracle's expansion of the previous stored state."""
    from dit_sparse_atten_amd.attention_backends import context
    from dit_sparse_atten_amd.attention_backends.sparse import MatrixSparseBackend, SparseConfig
    grid, heads = (2, 18, 32), 3
    case = S.SparsePathCase(grid, tile=64)
    tokens = grid[0] * grid[1] * grid[2]
    perm = torch.as_tensor(case.permutation, dtype=torch.long)
    sink = case.block_h * case.block_w
    grid_tiles = (grid[0], case.block_h, case.block_w)
    backend = MatrixSparseBackend(SparseConfig(tile=64, keep=0.625, mass_target=0.95,
                                               policy=policy))
    context.reset_runtime_state()
    try:
        previous = None
        for step in range(4):
            q, k, v = clustered_qkv(tokens, heads, 128, group=64, seed=60 + step,
                                    permutation=perm, dtype=torch.bfloat16)
            context.set_routing_context(attention_id=2, step=step, branch=0, grid=grid)
            out = backend(q.to(cuda_device), k.to(cuda_device), v.to(cuda_device))
            torch.cuda.synchronize()
            state = {key: val.cpu().numpy() for key, val in
                     next(iter(backend.state.values())).items() if torch.is_tensor(val)}
            # Tile-major inputs, as the backend sees them.
            qt, kt, vt = (x[:, perm].to(cuda_device) for x in (q, k, v))
            route_used = None if previous is None else S.expand(previous, policy, grid_tiles)
            expected_out, _ = A.block_sparse_attention(
                *(x.float().cpu().numpy() for x in (qt, kt, vt)), route_used, case.tile)
            restored = np.empty_like(expected_out)
            restored[:, perm.numpy()] = expected_out
            metrics = A.summarize(out.float().cpu().numpy(), restored)
            assert metrics["max_absolute_error"] <= 2e-2, (step, metrics)
            assert metrics["cosine_similarity"] >= 0.9995, (step, metrics)
            if route_used is None:
                _, lse = ops.bsa_fwd(qt, kt, vt, return_lse=True)
                mass = ops.tile_stats(qt, kt, lse, case.tile_shape)["mass"].cpu().numpy()
                expected_mask = R.top_mass_route(mass, 0.95, 0.625)
            elif policy == "reuse":
                expected_mask = S.drop_low_mass(route_used, previous["mass"], 0.1)
            else:
                csr = ops.route_to_csr(torch.from_numpy(route_used).to(cuda_device),
                                       block_size=case.tile)
                _, lse = ops.bsa_fwd(qt, kt, vt, csr, return_lse=True, block_size=case.tile)
                mass = ops.tile_stats(qt, kt, lse, case.tile_shape, csr=csr)["mass"]
                expected_mask = S.drop_low_mass(route_used, mass.cpu().numpy(), 0.1)
            expected_mask = np.array(expected_mask, copy=True)
            expected_mask[..., :sink] = True
            np.testing.assert_array_equal(state["mask"], expected_mask, err_msg=f"step {step}")
            previous = state
    finally:
        context.reset_runtime_state()


def _config0_call(cuda_device, dtype):
    """BASELINE config 0 through the GPU ``sparse`` backend as the reference's
    fixture ran it (tests/golden/make_golden.py): 12 heads, grid (4, 16, 16),
    8x8 tiles, the step-0 dense bootstrap (top-mass 0.95, cap 10 of 16, the
    4 frame-0 tiles as key sink), then step 1 on that route.  Returns the
    fixture, both outputs and the bootstrap route."""
    from dit_sparse_atten_amd.attention_backends import context
    from dit_sparse_atten_amd.attention_backends.sparse import MatrixSparseBackend, SparseConfig
    from tests.golden.inputs import clustered_qkv
    data = np.load(Path(__file__).resolve().parent / "golden" / "sparse_config0.npz",
                   allow_pickle=False)
    order = torch.as_tensor(data["order"], dtype=torch.long)
    q, k, v = clustered_qkv(1024, 12, 128, group=64, seed=0, permutation=order)
    np.testing.assert_allclose([q.double().sum().item(), k.double().sum().item(),
                                v.double().sum().item()], data["checksum"])
    qd, kd, vd = (x.to(cuda_device, dtype) for x in (q, k, v))
    backend = MatrixSparseBackend(SparseConfig(tile=64, keep=0.625, mass_target=0.95,
                                               prefetch_route=False))
    context.reset_runtime_state()
    try:
        context.set_routing_context(attention_id=1, step=0, branch=0, grid=(4, 16, 16))
        out0 = backend(qd, kd, vd, dtype=dtype)
        route = next(iter(backend.state.values()))["mask"].clone()
        context.set_routing_context(step=1)
        out1 = backend(qd, kd, vd, dtype=dtype)
        torch.cuda.synchronize()
    finally:
        context.reset_runtime_state()
    return data, out0, out1, route


@pytest.mark.parametrize("dtype,max_abs,cosine", [(torch.bfloat16, 2e-2, 0.9995),
                                                   (torch.float32, 5e-6, 0.99999999)])
def test_config0_full_call_matches_reference_outputs(cuda_device, dtype, max_abs, cosine):
    """The whole config-0 call, bootstrap route included, against the
    reference's own float32 outputs (sparse_config0.npz: heads 0 and 7, the
    first 256 tokens of step 0 and step 1): in bfloat16 at max-abs 2e-2 /
    cosine 0.9995, and in float32, as the reference computed them, at fp32
    rounding (max-abs 5e-6)."""
    data, out0, out1, route = _config0_call(cuda_device, dtype)
    heads = [int(h) for h in data["heads"]]
    # The bootstrap route (the 4 frame-0 tiles included) is the reference's.
    np.testing.assert_array_equal(route.cpu().numpy(), data["route"])
    for got, name in ((out0, "out0"), (out1, "out1")):
        assert got.dtype == dtype
        sample = got[0, :256][:, heads].float().cpu().numpy()
        metrics = A.summarize(sample, data[name])
        print(dtype, name, metrics)
        assert metrics["max_absolute_error"] <= max_abs and metrics["cosine_similarity"] >= cosine, (
            name, metrics)

"""GPU parity of the float32 calls (the fp32 matrix-core kernel,
csrc/bsa_fwd_f32.hip) against float64 closed forms and the oracle.

The reference computes in the dtype it is given: DenseBackend hands
``dtype`` to SDPA (attention_backends/dense.py:34-47) and MatrixSparseBackend
computes in q's own dtype (sparse.py:700-708), which is how its float32
golden fixtures were written.  The kernel forms fp32 products with fp32
accumulation and keeps the probabilities in fp32, so the bar is fp32
rounding: outputs within 2e-5 of the float64 closed form (values of order
one), LSE within 2e-5, statistics within rtol 1e-5.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import sparse_path as S
from tests.golden.inputs import clustered_qkv, random_route

pytestmark = pytest.mark.gpu

OUT_ATOL = 2e-5
LSE_ATOL = 2e-5
MASS_RTOL = 1e-5


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _qkv(batch, q_tokens, kv_tokens, heads, head_dim, seed):
    generator = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, q_tokens, heads, head_dim, generator=generator)
    k = torch.randn(batch, kv_tokens, heads, head_dim, generator=generator)
    v = torch.randn(batch, kv_tokens, heads, head_dim, generator=generator)
    return q, k, v


def _check(out, lse, want_out, want_lse):
    out = out.double().cpu().numpy()
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out, want_out, atol=OUT_ATOL, rtol=0)
    if lse is not None:
        np.testing.assert_allclose(lse.double().cpu().numpy(), want_lse, atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("batch,q_tokens,kv_tokens,heads,head_dim,causal", [
    (1, 1000, 1000, 3, 128, False),
    (2, 333, 333, 2, 64, True),
    (1, 256, 256, 2, 8, False),
    (2, 200, 517, 2, 128, False),   # cross-attention (unequal lengths)
])
def test_fp32_dense_matches_float64(ops, cuda_device, batch, q_tokens, kv_tokens, heads,
                                    head_dim, causal):
    q, k, v = _qkv(batch, q_tokens, kv_tokens, heads, head_dim, seed=q_tokens + head_dim)
    out, lse = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), return_lse=True,
                           causal=causal)
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    want_out, want_lse = A.block_sparse_attention(q.numpy(), k.numpy(), v.numpy(), None, 128,
                                                  causal=causal)
    _check(out, lse, want_out, want_lse)


@pytest.mark.parametrize("tokens,block", [(1024, 128), (1000, 64), (720, 72), (1000, 100),
                                          (512, 16), (40, 1)])
def test_fp32_routed_matches_float64(ops, cuda_device, tokens, block):
    """Routed calls of whole and partial blocks of 1..128 tokens, rows with
    empty routes included, against the float64 closed form."""
    heads = 2
    q, k, v = _qkv(1, tokens, tokens, heads, 128, seed=tokens + block)
    blocks = math.ceil(tokens / block)
    route = random_route(heads, blocks, seed=block, keep=0.5).numpy()
    route[0, 0] = False  # one empty row
    csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=block)
    out, lse = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), csr, return_lse=True,
                           block_size=block)
    torch.cuda.synchronize()
    want_out, want_lse = A.block_sparse_attention(q.numpy(), k.numpy(), v.numpy(), route, block)
    _check(out, lse, want_out, want_lse)
    assert (out[0, :block, 0] == 0).all()


def _tile_inputs(grid, tile, heads, seed):
    case = S.SparsePathCase(grid, tile=tile)
    tokens = grid[0] * grid[1] * grid[2]
    perm = torch.as_tensor(case.permutation, dtype=torch.long)
    q, k, v = clustered_qkv(tokens, heads, 128, group=case.tile, seed=seed, permutation=perm)
    return case, q[:, perm].contiguous(), k[:, perm].contiguous(), v[:, perm].contiguous()


def _oracle(case, q, k, v, route):
    qf, kf, vf = (x.numpy() for x in (q, k, v))
    tokens, heads = qf.shape[1:3]
    tiles = tokens // case.tile
    stats = S.empty_stats(heads, tiles)
    offsets = S.spatial_offsets(case.tile_shape, tiles)
    scale = 128 ** -0.5
    if route is None:
        _, _, out = S.dense_route(qf, kf, vf, case.tile, 256, 0.95, 0.625, scale, stats, offsets)
    else:
        out = np.empty_like(qf)
        for start in range(0, tokens, case.tile * 4):
            end = min(start + case.tile * 4, tokens)
            out[:, start:end] = S.sparse_chunk(qf, kf, vf, route, case.tile, start, end, scale,
                                               stats, offsets)
    return stats, out


@pytest.mark.parametrize("routed", [True, False])
@pytest.mark.parametrize("grid,tile", [((4, 16, 16), 64), ((2, 18, 32), 64), ((2, 15, 26), 64),
                                       ((2, 22, 22), 121), ((2, 12, 12), 36)])
def test_fp32_tile_step_matches_oracle(ops, cuda_device, routed, grid, tile):
    """dsa_bsa_fwd_tile_stats in float32 (8 x 8, 9 x 8, 5 x 13, 11 x 11 and
    6 x 6 tiles, routed and dense) against the oracle's sparse_chunk /
    _dense_route restatement in float32: output, mass at rtol 1e-5, the fp16
    mass and centroids at fp16 rounding."""
    case, q, k, v = _tile_inputs(grid, tile, 2, seed=sum(grid) + tile)
    tokens = q.shape[1]
    tiles = tokens // case.tile
    route = None
    csr = None
    if routed:
        route = random_route(2, tiles, seed=tile, keep=0.55).numpy()
        route[..., 0] = True
        csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=case.tile)
    out, _, got = ops.bsa_fwd_tile_stats(*(x.to(cuda_device) for x in (q, k, v)), csr,
                                         case.tile_shape, deterministic=True)
    torch.cuda.synchronize()
    stats, want_out = _oracle(case, q, k, v, route)
    np.testing.assert_allclose(out.double().cpu().numpy(), want_out, atol=OUT_ATOL, rtol=0)
    mass = stats["mass"] / np.float32(tokens)
    np.testing.assert_allclose(got["mass"].cpu().numpy(), mass, rtol=MASS_RTOL, atol=1e-9)
    np.testing.assert_allclose(got["mass_f16"].float().cpu().numpy(), mass, rtol=1e-3, atol=1e-7)
    den = np.maximum(stats["mass"], np.float32(1e-12))
    for name in ("q_y", "q_x", "k_y", "k_x"):
        np.testing.assert_allclose(got[f"centroid_{name}"].float().cpu().numpy(),
                                   stats[name] / den, atol=1e-3, err_msg=name)
    if routed:
        assert (got["mass"].cpu().numpy()[~route] == 0).all()


def test_fp32_block_mass_matches_float64(ops, cuda_device):
    """The exact 128-token block mass of a float32 dense call (the flex
    backend's exact bootstrap) against the float64 closed form."""
    q, k, v = _qkv(1, 640, 640, 2, 128, seed=5)
    out, lse, mass = ops.bsa_fwd_block_mass(*(x.to(cuda_device) for x in (q, k, v)))
    torch.cuda.synchronize()
    want_out, want_lse = A.block_sparse_attention(q.numpy(), k.numpy(), v.numpy(), None, 128)
    _check(out, lse, want_out, want_lse)
    qd, kd = q.double().numpy()[0], k.double().numpy()[0]
    blocks = 5
    want = np.zeros((2, blocks, blocks))
    for h in range(2):
        p = np.exp(qd[:, h] @ kd[:, h].T * 128 ** -0.5 - want_lse[0, h][:, None])
        want[h] = p.reshape(blocks, 128, blocks, 128).sum((1, 3))
    np.testing.assert_allclose(mass.double().cpu().numpy(), want, rtol=MASS_RTOL, atol=1e-9)


def test_fp32_through_the_dense_and_flex_backends(cuda_device):
    """DenseBackend with dtype=float32, and FlexReuseBackend's float32 calls
    (exact bootstrap on the fp32 block mass, then a routed step), against the
    float64 closed form of the route each step used."""
    from dit_sparse_atten_amd.attention_backends import context
    from dit_sparse_atten_amd.attention_backends.dense import DenseBackend
    from dit_sparse_atten_amd.attention_backends.flex import FlexReuseBackend, FlexReuseConfig
    q, k, v = _qkv(1, 1024, 1024, 2, 128, seed=9)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    dense = DenseBackend()(qd, kd, vd, dtype=torch.float32)
    want, _ = A.block_sparse_attention(q.numpy(), k.numpy(), v.numpy(), None, 128)
    np.testing.assert_allclose(dense.double().cpu().numpy(), want, atol=OUT_ATOL, rtol=0)

    backend = FlexReuseBackend(FlexReuseConfig(keep=0.5))
    context.reset_runtime_state()
    try:
        context.set_routing_context(attention_id=1, step=0, branch=0, grid=None)
        out0 = backend(qd, kd, vd, dtype=torch.float32)
        state = next(iter(backend.state.values()))
        route = state["route"].clone()
        context.set_routing_context(step=1)
        out1 = backend(qd, kd, vd, dtype=torch.float32)
        torch.cuda.synchronize()
    finally:
        context.reset_runtime_state()
    assert out0.dtype == torch.float32 and out1.dtype == torch.float32
    np.testing.assert_allclose(out0.double().cpu().numpy(), want, atol=OUT_ATOL, rtol=0)
    routed, _ = A.block_sparse_attention(q.numpy(), k.numpy(), v.numpy(),
                                         route.cpu().numpy(), 128)
    np.testing.assert_allclose(out1.double().cpu().numpy(), routed, atol=OUT_ATOL, rtol=0)
    assert not route.cpu().numpy().all()


def test_fp32_batched_routes_and_strided_views(ops, cuda_device):
    """Two batch items with their own routes (route_batches 2), read through
    the transposed views of BHSD storage the Diffusers processor passes, with
    a partial last block, against the float64 closed form."""
    batch, heads, tokens, block = 2, 3, 700, 128
    generator = torch.Generator().manual_seed(12)
    bhsd = [torch.randn(batch, heads, tokens, 64, generator=generator) for _ in range(3)]
    q, k, v = (x.to(cuda_device).transpose(1, 2) for x in bhsd)
    assert not q.is_contiguous()
    blocks = math.ceil(tokens / block)
    route = np.stack([random_route(heads, blocks, seed=20 + b, keep=0.6).numpy()
                      for b in range(batch)])
    csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=block)
    out, lse = ops.bsa_fwd(q, k, v, csr, return_lse=True, block_size=block)
    torch.cuda.synchronize()
    want, want_lse = A.block_sparse_attention(*(x.transpose(1, 2).numpy() for x in bhsd),
                                              route, block)
    _check(out, lse, want, want_lse)

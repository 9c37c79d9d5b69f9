"""fp16 inputs through every kernel whose reference counterpart computes in
the input dtype (the Wan processor passes dtype=query.dtype,
wan_diffusers.py:58-68; DenseBackend and FlexReuseBackend cast to it,
dense.py:36-47, flex.py:687-691; the matrix-sparse path computes in the input
dtype, sparse.py:700-708), against the same float64 oracle and bars as the
bf16 tests; and the one dtype rejection, float32 compute, raised alike by all
three backends."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import exact as E
from tests.golden.inputs import clustered_qkv, random_route

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COSINE = 0.9995


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _inputs(batch, tokens, heads, seed):
    generator = torch.Generator().manual_seed(seed)
    return [torch.randn(batch, tokens, heads, 128, generator=generator).to(torch.float16)
            for _ in range(3)]


def _check(out, q, k, v, route, block=128):
    assert out.dtype == torch.float16
    expected, _ = A.block_sparse_attention(q.float().numpy(), k.float().numpy(),
                                           v.float().numpy(), route, block)
    metrics = A.summarize(out.float().cpu().numpy(), expected)
    assert metrics["max_absolute_error"] <= MAX_ABS, metrics
    assert metrics["cosine_similarity"] >= MIN_COSINE, metrics
    np.testing.assert_allclose(out.float().cpu().numpy(), expected, atol=5e-3, rtol=3e-2)


@pytest.mark.parametrize("tokens", [250, 1000])
def test_fp16_dense_matches_oracle(ops, cuda_device, tokens):
    q, k, v = _inputs(1, tokens, 2, seed=tokens)
    out, lse = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), return_lse=True)
    torch.cuda.synchronize()
    _check(out, q, k, v, None)
    _, expected_lse = A.block_sparse_attention(q.float().numpy(), k.float().numpy(),
                                               v.float().numpy(), None, 128)
    np.testing.assert_allclose(lse.cpu().numpy(), expected_lse, atol=1e-3, rtol=1e-4)


@pytest.mark.parametrize("block,tokens,batch", [(128, 1280, 2), (128, 8192, 1), (72, 1440, 1),
                                                (40, 600, 1), (100, 777, 1), (127, 1270, 1)])
def test_fp16_routed_matches_oracle(ops, cuda_device, block, tokens, batch):
    """128-token blocks (B=2 with per-batch routes; 8,192 tokens with the split
    last round), the gathered key stream (72, 127), 2-wave blocks (40) and the
    sub-tile skip (100, partial last block)."""
    q, k, v = _inputs(batch, tokens, 2, seed=block)
    blocks = math.ceil(tokens / block)
    generator = torch.Generator().manual_seed(block + 1)
    route = torch.rand(batch, 2, blocks, blocks, generator=generator) < 0.55
    route[..., 0] = True
    csr = ops.route_to_csr(route.to(cuda_device), block_size=block)
    out = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), csr, block_size=block)
    torch.cuda.synchronize()
    for b in range(batch):
        _check(out[b:b + 1], q[b:b + 1], k[b:b + 1], v[b:b + 1], route[b].numpy(), block)


def test_fp16_strided_views_and_mixed_dtype_rejected(ops, cuda_device):
    generator = torch.Generator().manual_seed(5)
    base = [torch.randn(1, 3, 384, 128, generator=generator).to(torch.float16)
            for _ in range(3)]
    views = [t.to(cuda_device).transpose(1, 2) for t in base]
    out = ops.bsa_fwd(*views)
    torch.cuda.synchronize()
    _check(out, *(t.transpose(1, 2) for t in base), None)
    with pytest.raises(ValueError, match="like q"):
        ops.bsa_fwd(views[0], views[1].bfloat16(), views[2])


@pytest.mark.parametrize("tokens", [130, 1024])
def test_fp16_block_mass_matches_oracle(ops, cuda_device, tokens):
    q, k, v = clustered_qkv(tokens, 2, 128, group=64, seed=tokens, dtype=torch.float16)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    mass = ops.block_mass(qd, kd, lse)
    torch.cuda.synchronize()
    expected = E.exact_block_mass(q.float().numpy(), k.float().numpy(), lse[0].cpu().numpy(),
                                  128)
    np.testing.assert_allclose(mass.cpu().numpy(), expected, rtol=1e-4, atol=1e-6)


@pytest.mark.parametrize("routed", [False, True])
def test_fp16_tile_stats_match_oracle(ops, cuda_device, routed):
    from tests.test_gpu_matrix_sparse import _compare_stats, _oracle_stats, _tile_major_inputs
    case, q, k, v = _tile_major_inputs((2, 18, 32), 2, seed=11, tile=64)
    q, k, v = (x.to(torch.float16) for x in (q, k, v))
    tiles = q.shape[1] // case.tile
    route = None
    csr = None
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    if routed:
        route = random_route(2, tiles, seed=3, keep=0.5).numpy()
        route[..., 0] = True
        csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=case.tile)
        _, lse = ops.bsa_fwd(qd, kd, vd, csr, return_lse=True, block_size=case.tile)
    else:
        _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    got = ops.tile_stats(qd, kd, lse, case.tile_shape, csr=csr)
    torch.cuda.synchronize()
    expected, _ = _oracle_stats(case, q, k, v, route)
    _compare_stats(got, expected)


@pytest.mark.parametrize("name", ["dense", "flex_reuse", "sparse"])
def test_fp16_through_every_backend(cuda_device, name):
    """The Diffusers processor's call with fp16 storage and dtype=query.dtype:
    step 0 (dense output and route bootstrap), then step 1 (the sparse route
    for flex_reuse and sparse), each against the float64 closed form of the
    route the backend actually used."""
    from dit_sparse_atten_amd.attention_backends import BACKENDS, context
    from dit_sparse_atten_amd.attention_backends.flex import FlexReuseConfig
    from dit_sparse_atten_amd.attention_backends.sparse import SparseConfig
    context.reset_runtime_state()
    try:
        if name == "flex_reuse":
            backend = BACKENDS[name](FlexReuseConfig(
                bootstrap_mode="sampled", route_samples=12, mass_target=0.9, keep=0.5,
                dense_route_threshold=None, spatial_reorder=False, total_steps=3))
        elif name == "sparse":
            backend = BACKENDS[name](SparseConfig(tile=64, keep=0.5, policy="reuse"))
        else:
            backend = BACKENDS[name]()
        grid = (2, 16, 32)
        tokens, heads = math.prod(grid), 2
        q, k, v = clustered_qkv(tokens, heads, 128, group=64, seed=9, dtype=torch.float16)
        views = [x.transpose(1, 2).contiguous().to(cuda_device).transpose(1, 2)
                 for x in (q, k, v)]
        expected, _ = A.block_sparse_attention(q.float().numpy(), k.float().numpy(),
                                               v.float().numpy(), None, 128)
        for step in (0, 1):
            context.set_routing_context(attention_id=1, step=step, branch=0, grid=grid)
            out = backend(*views, dropout_p=0.0, softmax_scale=None, causal=False,
                          window_size=(-1, -1), dtype=views[0].dtype, attention_mask=None)
            torch.cuda.synchronize()
            assert out.shape == views[0].shape and out.dtype == torch.float16
            metrics = A.summarize(out.float().cpu().numpy(), expected)
            if step == 0:
                assert metrics["max_absolute_error"] <= MAX_ABS, metrics
                assert metrics["cosine_similarity"] >= MIN_COSINE, metrics
            else:
                # A sparse route drops some mass: close to, not equal to, dense.
                assert metrics["cosine_similarity"] >= 0.9, metrics
        if name == "flex_reuse":
            assert backend.phase_counts["sampled_bootstrap"] == 1
            assert backend.phase_counts["sparse_reuse"] == 1
    finally:
        context.reset_runtime_state()


@pytest.mark.parametrize("name", ["dense", "flex_reuse", "sparse"])
def test_float64_compute_is_rejected_alike(cuda_device, name):
    """float64 compute has no kernel: every backend raises the same
    ValueError (dense and flex_reuse for dtype=float64, sparse for float64
    inputs, since it computes in the input dtype)."""
    from dit_sparse_atten_amd.attention_backends import BACKENDS, context
    context.reset_runtime_state()
    try:
        backend = BACKENDS[name]()
        grid = (2, 16, 32)
        q, k, v = (torch.randn(1, math.prod(grid), 2, 128, device=cuda_device,
                               dtype=torch.float64) for _ in range(3))
        context.set_routing_context(attention_id=1, step=0, branch=0, grid=grid)
        with pytest.raises(ValueError, match="bfloat16, float16 or float32"):
            backend(q, k, v, dtype=torch.float64)
    finally:
        context.reset_runtime_state()

"""The boundary beyond the Wan shapes: head dims below 128 (the reference's
own tests run d = 32 on the GPU, tests/test_flex_backend.py:82-153) and causal
dense attention (SDPA's is_causal, which the reference's dense backend passes
through, dense.py:40-47), against the float64 oracle."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import exact as E
from oracle import route as R
from tests.golden.inputs import clustered_qkv

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COSINE = 0.9995


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _check(out, q, k, v, route=None, block=128, causal=False, scale=None):
    expected, expected_lse = A.block_sparse_attention(
        q.float().numpy(), k.float().numpy(), v.float().numpy(), route, block, scale=scale,
        causal=causal)
    got = out.float().cpu().numpy()
    metrics = A.summarize(got, expected)
    assert metrics["max_absolute_error"] <= MAX_ABS, metrics
    assert metrics["cosine_similarity"] >= MIN_COSINE, metrics
    np.testing.assert_allclose(got, expected, atol=5e-3, rtol=3e-2)
    return expected_lse


def _randn(shape, seed, dtype=torch.bfloat16):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed)).to(dtype)


# -- the reference's d = 32 GPU tests, restated on libdsa ---------------------

def test_reference_block_mass_explicit_softmax_d32(ops, cuda_device):
    """tests/test_flex_backend.py:82-98: 250 tokens, 2 heads, d = 32, bf16,
    LSE from the float32 scores; mass == padded softmax block sums within
    2e-5."""
    tokens, heads, head_dim, block = 250, 2, 32, 128
    q = _randn((1, tokens, heads, head_dim), 3).to(cuda_device)
    k = _randn((1, tokens, heads, head_dim), 4).to(cuda_device)
    scores = (q.transpose(1, 2).float() @ k.transpose(1, 2).float().transpose(-1, -2).contiguous()
              ) * head_dim ** -0.5
    lse = scores.logsumexp(-1)
    actual = ops.block_mass(q, k, lse, block)
    probabilities = scores.softmax(-1)[0]
    padded = torch.nn.functional.pad(probabilities, (0, 6, 0, 6))
    expected = padded.reshape(heads, 2, block, 2, block).sum((2, 4))
    torch.testing.assert_close(actual, expected, atol=2e-5, rtol=2e-5)


def test_reference_dense_bootstrap_matches_sdpa_d32(cuda_device):
    """tests/test_flex_backend.py:101-119: the exact bootstrap's dense output
    at 250 tokens (partial last block), 2 heads, d = 32 equals SDPA (float32
    here, atol 2e-3 / rtol 2e-2) and yields a [2, 2, 2] route."""
    from dit_sparse_atten_amd.attention_backends import context
    from dit_sparse_atten_amd.attention_backends.flex import FlexReuseBackend, FlexReuseConfig
    context.reset_runtime_state()
    try:
        q, k, v = (_randn((1, 250, 2, 32), seed).to(cuda_device) for seed in (0, 1, 2))
        backend = FlexReuseBackend(FlexReuseConfig(
            bootstrap_mode="exact", mass_target=0.90, keep=0.625, spatial_reorder=False))
        context.set_routing_context(attention_id=1, step=0, branch=0, grid=None)
        output = backend(q, k, v)
        reference = torch.nn.functional.scaled_dot_product_attention(
            *(x.transpose(1, 2).float() for x in (q, k, v))).transpose(1, 2)
        torch.testing.assert_close(output.float(), reference, atol=2e-3, rtol=2e-2)
        state = next(iter(backend.state.values()))
        assert tuple(state["route"].shape) == (2, 2, 2)
    finally:
        context.reset_runtime_state()


def test_reference_flex_output_explicit_block_mask_d32(ops, cuda_device):
    """tests/test_flex_backend.py:122-148: block-diagonal route over 250
    tokens, d = 32, against the float32 masked softmax (atol 5e-3, rtol
    3e-2)."""
    tokens, heads, head_dim, block = 250, 2, 32, 128
    q, k, v = (_randn((1, tokens, heads, head_dim), seed).to(cuda_device) for seed in (1, 2, 3))
    route = torch.eye(2, device=cuda_device, dtype=torch.bool).expand(heads, -1, -1).contiguous()
    output = ops.bsa_fwd(q, k, v, ops.route_to_csr(route))
    qh, kh, vh = (x.transpose(1, 2).float() for x in (q, k, v))
    block_ids = torch.arange(tokens, device=cuda_device) // block
    allowed = route[:, block_ids[:, None], block_ids[None, :]].unsqueeze(0)
    scores = (qh @ kh.transpose(-1, -2).contiguous()) * head_dim ** -0.5
    reference = scores.masked_fill(~allowed, -torch.inf).softmax(-1) @ vh
    torch.testing.assert_close(output.transpose(1, 2).float(), reference, atol=5e-3, rtol=3e-2)


# -- head dims below 128 ------------------------------------------------------

@pytest.mark.parametrize("head_dim", [8, 16, 40, 64, 96, 120])
def test_head_dims_dense_and_routed(ops, cuda_device, head_dim):
    """Dense and routed 128-token blocks (with the split last round: 64
    blocks x 2 heads) and the gathered stream of 72-token tiles, contiguous
    [B,T,H,D] and views of BHSD storage."""
    tokens, heads = 8192, 2
    q, k, v = (_randn((1, tokens, heads, head_dim), head_dim + s) for s in range(3))
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    out, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    torch.cuda.synchronize()
    rows = [(0, h, qb) for h in range(heads) for qb in (0, 17, 63)]
    expected, _ = A.block_sparse_attention(q.float().numpy(), k.float().numpy(),
                                           v.float().numpy(), None, 128, rows=rows)
    mask = ~np.isnan(expected)
    metrics = A.summarize(out.float().cpu().numpy()[mask], expected[mask])
    assert metrics["max_absolute_error"] <= MAX_ABS and metrics["cosine_similarity"] >= MIN_COSINE
    generator = torch.Generator().manual_seed(head_dim)
    route = torch.rand(heads, 64, 64, generator=generator) < 0.5
    route[..., 0] = True
    views = [x.transpose(1, 2).contiguous().to(cuda_device).transpose(1, 2) for x in (q, k, v)]
    out = ops.bsa_fwd(*views, ops.route_to_csr(route.to(cuda_device)))
    torch.cuda.synchronize()
    expected, _ = A.block_sparse_attention(q.float().numpy(), k.float().numpy(),
                                           v.float().numpy(), route.numpy(), 128, rows=rows)
    metrics = A.summarize(out.float().cpu().numpy()[mask], expected[mask])
    assert metrics["max_absolute_error"] <= MAX_ABS and metrics["cosine_similarity"] >= MIN_COSINE
    # Gathered stream, 72-token tiles.
    q, k, v = (_randn((1, 1440, heads, head_dim), 7 * head_dim + s) for s in range(3))
    route = torch.rand(heads, 20, 20, generator=generator) < 0.5
    route[..., 0] = True
    out = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)),
                      ops.route_to_csr(route.to(cuda_device), block_size=72), block_size=72)
    torch.cuda.synchronize()
    _check(out, q, k, v, route.numpy(), block=72)


@pytest.mark.parametrize("head_dim", [8, 32, 64])
def test_head_dims_sampled_mass(ops, cuda_device, head_dim):
    q, k, _ = clustered_qkv(1000, 2, head_dim, group=128, seed=head_dim, dtype=torch.bfloat16)
    got = ops.sampled_block_mass(q.to(cuda_device), k.to(cuda_device), 128, 16)
    torch.cuda.synchronize()
    expected = R.sampled_block_mass(q.float().numpy(), k.float().numpy(), 128, 16)
    np.testing.assert_allclose(got.cpu().numpy(), expected, atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("head_dim", [16, 64])
def test_head_dims_block_mass(ops, cuda_device, head_dim):
    q, k, v = clustered_qkv(300, 2, head_dim, group=64, seed=head_dim, dtype=torch.bfloat16)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    mass = ops.block_mass(qd, kd, lse)
    torch.cuda.synchronize()
    expected = E.exact_block_mass(q.float().numpy(), k.float().numpy(), lse[0].cpu().numpy(), 128,
                                  scale=head_dim ** -0.5)
    np.testing.assert_allclose(mass.cpu().numpy(), expected, rtol=1e-4, atol=1e-6)


def test_head_dim_32_tile_stats(ops, cuda_device):
    from tests.test_gpu_matrix_sparse import _compare_stats, _oracle_stats, _tile_major_inputs
    case, q, k, v = _tile_major_inputs((2, 18, 32), 2, seed=13, tile=64)
    # The first 32 dims of the 128-dim clustered inputs, at the oracle's scale.
    q, k, v = (x[..., :32].contiguous() for x in (q, k, v))
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    scale = 128 ** -0.5
    _, lse = ops.bsa_fwd(qd, kd, vd, scale=scale, return_lse=True)
    got = ops.tile_stats(qd, kd, lse, case.tile_shape, scale=scale)
    torch.cuda.synchronize()
    expected, _ = _oracle_stats(case, q, k, v, scale=scale)
    _compare_stats(got, expected)


# -- causal ---------------------------------------------------------------------

@pytest.mark.parametrize("q_tokens,kv_tokens,heads", [(1000, 1000, 2), (300, 700, 2),
                                                      (700, 300, 2), (8192, 8192, 2)])
def test_causal_dense_matches_oracle(ops, cuda_device, q_tokens, kv_tokens, heads):
    """Self-attention (8,192 tokens: rows of 1..64 key blocks, the split last
    round), and top-left aligned causal masks for unequal lengths, with LSE."""
    q = _randn((1, q_tokens, heads, 64), q_tokens)
    k = _randn((1, kv_tokens, heads, 64), kv_tokens)
    v = _randn((1, kv_tokens, heads, 64), kv_tokens + 1)
    out, lse = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), return_lse=True, causal=True)
    torch.cuda.synchronize()
    expected_lse = _check(out, q, k, v, causal=True)
    np.testing.assert_allclose(lse.cpu().numpy(), expected_lse, atol=1e-3, rtol=1e-4)


def test_causal_through_the_backends(cuda_device):
    """causal=True: the dense backend computes it; flex_reuse routes such a
    call to dense, as the reference does (flex.py:655-668)."""
    from dit_sparse_atten_amd.attention_backends import DenseBackend, context
    from dit_sparse_atten_amd.attention_backends.flex import FlexReuseBackend
    context.reset_runtime_state()
    try:
        q, k, v = (_randn((1, 600, 2, 128), s) for s in (5, 6, 7))
        views = [x.to(cuda_device) for x in (q, k, v)]
        context.set_routing_context(attention_id=1, step=0, branch=0, grid=None)
        for backend in (DenseBackend(), FlexReuseBackend()):
            out = backend(*views, causal=True)
            torch.cuda.synchronize()
            _check(out, q, k, v, causal=True)
    finally:
        context.reset_runtime_state()

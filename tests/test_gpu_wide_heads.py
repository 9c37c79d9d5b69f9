"""GPU parity for head dims above 128 (136..256): SDPA takes any head dim
(the reference's DenseBackend, attention_backends/dense.py:34-47); here such
calls run the fp32-compute kernel for every input type (S over 256 dims, O in
two launches of 128 dims), against the float64 closed form."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import dropout as D
from tests.golden.inputs import random_route

pytestmark = pytest.mark.gpu

# fp32 rounding for fp32 inputs; the output's own rounding for 16-bit inputs.
ATOL = {torch.float32: 2e-5, torch.bfloat16: 1e-2, torch.float16: 2e-3}


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _qkv(batch, q_tokens, kv_tokens, heads, head_dim, seed, dtype):
    generator = torch.Generator().manual_seed(seed)
    q = torch.randn(batch, q_tokens, heads, head_dim, generator=generator).to(dtype)
    k = torch.randn(batch, kv_tokens, heads, head_dim, generator=generator).to(dtype)
    v = torch.randn(batch, kv_tokens, heads, head_dim, generator=generator).to(dtype)
    return q, k, v


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("head_dim,causal", [(136, False), (192, True), (256, False)])
def test_wide_heads_dense_match_float64(ops, cuda_device, dtype, head_dim, causal):
    q, k, v = _qkv(2, 300, 300, 2, head_dim, seed=head_dim, dtype=dtype)
    out, lse = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), return_lse=True,
                           causal=causal)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    want, want_lse = A.block_sparse_attention(q.float().numpy(), k.float().numpy(),
                                              v.float().numpy(), None, 128, causal=causal)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, atol=ATOL[dtype], rtol=0)
    np.testing.assert_allclose(lse.double().cpu().numpy(), want_lse, atol=2e-5, rtol=0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("block", [128, 64, 72])
def test_wide_heads_routed_match_float64(ops, cuda_device, dtype, block):
    tokens, heads = 700, 2
    q, k, v = _qkv(1, tokens, tokens, heads, 256, seed=block, dtype=dtype)
    blocks = math.ceil(tokens / block)
    route = random_route(heads, blocks, seed=block, keep=0.5).numpy()
    csr = ops.route_to_csr(torch.from_numpy(route).to(cuda_device), block_size=block)
    out = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), csr, block_size=block)
    torch.cuda.synchronize()
    want, _ = A.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                       route, block)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, atol=ATOL[dtype], rtol=0)


def test_wide_heads_dropout_matches_oracle_mask(ops, cuda_device):
    q, k, v = _qkv(1, 200, 200, 2, 256, seed=4, dtype=torch.float32)
    out = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), dropout_p=0.3, seed=77,
                      offset=2)
    torch.cuda.synchronize()
    keep = D.keep_mask(1, 2, 200, 200, 0.3, 77, 2)
    want = D.dropout_attention(q.numpy(), k.numpy(), v.numpy(), keep, 0.3)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, atol=2e-5, rtol=0)


def test_wide_heads_through_the_backends(cuda_device):
    """DenseBackend computes them; flex_reuse and sparse send them to dense
    (their route estimates take head dims up to 128)."""
    from dit_sparse_atten_amd.attention_backends import context
    from dit_sparse_atten_amd.attention_backends.dense import DenseBackend
    from dit_sparse_atten_amd.attention_backends.flex import FlexReuseBackend
    from dit_sparse_atten_amd.attention_backends.sparse import MatrixSparseBackend
    q, k, v = _qkv(1, 1024, 1024, 2, 192, seed=8, dtype=torch.bfloat16)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    dense = DenseBackend()(qd, kd, vd)
    want, _ = A.block_sparse_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                       None, 128)
    np.testing.assert_allclose(dense.double().cpu().numpy(), want, atol=1e-2, rtol=0)
    context.reset_runtime_state()
    try:
        context.set_routing_context(attention_id=1, step=0, branch=0, grid=(4, 16, 16))
        for backend in (FlexReuseBackend(), MatrixSparseBackend()):
            out = backend(qd, kd, vd)
            torch.cuda.synchronize()
            assert torch.equal(out, dense), backend.name
    finally:
        context.reset_runtime_state()

"""GPU parity of dense attention with dropout (dsa_bsa_fwd_dropout, the
fp32-compute kernel) against the oracle (oracle/dropout.py) with the same
Philox4x32-10 mask: the reference's DenseBackend hands dropout_p to SDPA
(attention_backends/dense.py:40-47).  torch's random stream is not
reproduced, so parity is to the oracle's mask, which the known-answer
vectors pin (tests/test_oracle_dropout.py)."""

import numpy as np
import pytest
import torch

from oracle import dropout as D

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _qkv(batch, q_tokens, kv_tokens, heads, head_dim, seed, dtype=torch.float32):
    generator = torch.Generator().manual_seed(seed)
    shape_q = (batch, q_tokens, heads, head_dim)
    shape_k = (batch, kv_tokens, heads, head_dim)
    return (torch.randn(shape_q, generator=generator).to(dtype),
            torch.randn(shape_k, generator=generator).to(dtype),
            torch.randn(shape_k, generator=generator).to(dtype))


@pytest.mark.parametrize("dtype,atol", [(torch.float32, 2e-5), (torch.bfloat16, 1.6e-2),
                                        (torch.float16, 2e-3)])
@pytest.mark.parametrize("batch,q_tokens,kv_tokens,heads,head_dim,p,causal", [
    (1, 300, 300, 2, 128, 0.2, False),
    (2, 130, 130, 3, 64, 0.5, True),
    (1, 77, 203, 2, 128, 0.1, False),   # cross-attention, partial key group of 4
])
def test_dropout_matches_oracle_mask(ops, cuda_device, dtype, atol, batch, q_tokens,
                                     kv_tokens, heads, head_dim, p, causal):
    q, k, v = _qkv(batch, q_tokens, kv_tokens, heads, head_dim, seed=q_tokens, dtype=dtype)
    seed, offset = (0x1234 << 32) | 0xBEEF, 11
    out, lse = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), causal=causal,
                           dropout_p=p, seed=seed, offset=offset, return_lse=True)
    again = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), causal=causal,
                        dropout_p=p, seed=seed, offset=offset)
    other = ops.bsa_fwd(*(x.to(cuda_device) for x in (q, k, v)), causal=causal,
                        dropout_p=p, seed=seed + 1, offset=offset)
    torch.cuda.synchronize()
    assert out.dtype == dtype
    assert torch.equal(out, again) and not torch.equal(out, other)
    keep = D.keep_mask(batch, heads, q_tokens, kv_tokens, p, seed, offset)
    want = D.dropout_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), keep, p,
                               causal=causal)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, atol=atol, rtol=0)
    assert np.isfinite(lse.cpu().numpy()).all()


def test_dropout_through_the_backends(cuda_device):
    """DenseBackend with dropout_p draws its seed from torch's CPU generator;
    flex_reuse and sparse send such calls to it, as the reference's do."""
    from dit_sparse_atten_amd.attention_backends.dense import DenseBackend
    from dit_sparse_atten_amd.attention_backends.flex import FlexReuseBackend
    q, k, v = _qkv(1, 256, 256, 2, 128, seed=3)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    torch.manual_seed(7)
    out = DenseBackend()(qd, kd, vd, dropout_p=0.25, dtype=torch.float32)
    torch.manual_seed(7)
    seed = int(torch.randint(0, 2 ** 63 - 1, (), dtype=torch.int64).item())
    keep = D.keep_mask(1, 2, 256, 256, 0.25, seed, 0)
    want = D.dropout_attention(q.numpy(), k.numpy(), v.numpy(), keep, 0.25)
    np.testing.assert_allclose(out.double().cpu().numpy(), want, atol=2e-5, rtol=0)
    torch.manual_seed(7)
    flex = FlexReuseBackend()(qd, kd, vd, dropout_p=0.25, dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(flex, out)

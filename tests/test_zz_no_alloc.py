"""dsa_bsa_fwd_noalloc (no workspace argument, library-owned split scratch)
against dsa_bsa_fwd with its workspace, through the C-ABI: two calls in a row
on one stream, the second smaller, both with a split last round, each both
deterministic (bit for bit) and with the aligned walk (oracle tolerance)."""

import math

import numpy as np
import pytest
import torch

from oracle.attention import block_sparse_attention, summarize

pytestmark = pytest.mark.gpu


def _case(tokens, heads, seed, device):
    generator = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, tokens, heads, 128, generator=generator).to(torch.bfloat16)
               for _ in range(3))
    blocks = math.ceil(tokens / 128)
    route = torch.rand(heads, blocks, blocks, generator=generator) < 0.55
    route[..., 0] = True
    return q, k, v, route


def _strides(q, k, v, o):
    from dit_sparse_atten_amd import _lib
    return _lib.int64_array(list(q.stride()[:3]) + list(k.stride()[:3]) + list(v.stride()[:3])
                            + list(o.stride()[:3]))


def test_noalloc_matches_workspace_entry_point(cuda_device):
    from dit_sparse_atten_amd import _lib, ops
    lib = _lib.load()
    stream = torch.cuda.current_stream(cuda_device).cuda_stream
    # 8,192 tokens x 3 heads: 192 query blocks in one partial round, each run
    # as key ranges; then 2,048 tokens x 2 heads (16 key blocks, 2 parts).
    for tokens, heads, seed in ((8192, 3, 1), (2048, 2, 2)):
        q, k, v, route = _case(tokens, heads, seed, cuda_device)
        qd, kd, vd = (t.to(cuda_device) for t in (q, k, v))
        csr = ops.route_to_csr(route.to(cuda_device))
        want = torch.empty_like(qd)
        got = torch.empty_like(qd)
        want_lse = torch.empty((1, heads, tokens), dtype=torch.float32, device=cuda_device)
        got_lse = torch.empty_like(want_lse)
        strides = _strides(qd, kd, vd, got)
        bytes_ = lib.dsa_bsa_workspace_bytes(1, heads, tokens, 128)
        assert bytes_ > 0
        workspace = torch.empty(bytes_, dtype=torch.uint8, device=cuda_device)
        expected, expected_lse = block_sparse_attention(
            q.float().numpy(), k.float().numpy(), v.float().numpy(), route.numpy(), 128)
        # deterministic = 1: same kernels, same split plan, identical bits;
        # deterministic = 0 (aligned walk): the oracle's tolerance.
        for deterministic in (1, 0):
            args = (strides, 1, tokens, tokens, heads, 128, 128, csr.row_ptr.data_ptr(),
                    csr.col_idx.data_ptr(), 1, 128 ** -0.5, 0, deterministic)
            _lib.check(lib.dsa_bsa_fwd(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                       want.data_ptr(), 0, *args, want_lse.data_ptr(),
                                       workspace.data_ptr(), bytes_, stream), "dsa_bsa_fwd")
            _lib.check(lib.dsa_bsa_fwd_noalloc(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(),
                                               got.data_ptr(), 0, *args, got_lse.data_ptr(),
                                               stream), "dsa_bsa_fwd_noalloc")
            torch.cuda.synchronize()
            if deterministic:
                assert torch.equal(got, want), (tokens, heads)
                assert torch.equal(got_lse, want_lse), (tokens, heads)
            for out, lse in ((got, got_lse), (want, want_lse)):
                metrics = summarize(out.float().cpu().numpy(), expected)
                assert metrics["max_absolute_error"] <= 2e-2, (deterministic, metrics)
                assert metrics["cosine_similarity"] >= 0.9995, (deterministic, metrics)
                np.testing.assert_allclose(lse.cpu().numpy(), expected_lse, atol=1e-3, rtol=1e-4)


def test_noalloc_validates_before_launch(cuda_device):
    from dit_sparse_atten_amd import _lib
    lib = _lib.load()
    status = lib.dsa_bsa_fwd_noalloc(None, None, None, None, 0, _lib.int64_array([8] * 12), 1, 128,
                                     128, 1, 128, 128, None, None, 1, 0.1, 0, 0, None, None)
    assert status == _lib.DSA_EINVAL and "null" in _lib.last_error()

"""GPU parity of the exact route estimator: the dense forward's LSE, the exact
block-mass pass (dsa_block_mass) and the exact bootstrap / refresh phases of
the backend, against the oracle (oracle/exact.py) on the same bf16 inputs.

Tolerances: LSE within 1e-4 absolute (fp32 accumulation of exact bf16
products); block mass within 1e-4 relative + 1e-6 absolute of the fp64
restatement fed the same LSE; routes bit-exact given the same fp32 mass."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import exact as E
from oracle import route as R
from tests.golden.inputs import clustered_qkv

pytestmark = pytest.mark.gpu

LSE_ATOL = 1e-4
MASS_RTOL = 1e-4
MASS_ATOL = 1e-6


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _inputs(tokens, heads, seed, group=128):
    q, k, v = clustered_qkv(tokens, heads, 128, group=group, seed=seed, dtype=torch.bfloat16)
    return q, k, v


@pytest.mark.parametrize("tokens", [130, 300, 1024])
def test_dense_lse_matches_oracle(ops, cuda_device, tokens):
    q, k, v = _inputs(tokens, 2, seed=tokens)
    _, lse = ops.bsa_fwd(q.to(cuda_device), k.to(cuda_device), v.to(cuda_device),
                         return_lse=True)
    torch.cuda.synchronize()
    expected = E.dense_lse(q.float().numpy(), k.float().numpy())
    np.testing.assert_allclose(lse[0].cpu().numpy(), expected, atol=LSE_ATOL, rtol=0)


@pytest.mark.parametrize("tokens", [64, 130, 192, 300, 1024])
def test_block_mass_matches_oracle(ops, cuda_device, tokens):
    """Partial last blocks of 2, 64 and 44 keys and a half-tile wholly past
    the end (130 tokens) are all covered."""
    q, k, v = _inputs(tokens, 2, seed=7 + tokens, group=64)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    mass = ops.block_mass(qd, kd, lse)
    torch.cuda.synchronize()
    got = mass.cpu().numpy()
    expected = E.exact_block_mass(q.float().numpy(), k.float().numpy(),
                                  lse[0].cpu().numpy(), 128)
    np.testing.assert_allclose(got, expected, rtol=MASS_RTOL, atol=MASS_ATOL)
    blocks = math.ceil(tokens / 128)
    valid = np.minimum(tokens - np.arange(blocks) * 128, 128)
    np.testing.assert_allclose(got.sum(-1), np.broadcast_to(valid, got.shape[:2]), rtol=1e-4)


@pytest.mark.parametrize("tokens", [128, 1024, 1000])
def test_dense_with_block_mass_matches_oracle(ops, cuda_device, tokens):
    """dsa_bsa_fwd_block_mass: the dense output, its LSE and the exact block
    mass in one call (fused for whole 128-token blocks, the separate pass for
    1,000 tokens) against the oracle and the two-call path."""
    q, k, v = _inputs(tokens, 3, seed=11 + tokens, group=64)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    out, lse, mass = ops.bsa_fwd_block_mass(qd, kd, vd)
    ref_out, ref_lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    ref_mass = ops.block_mass(qd, kd, ref_lse)
    torch.cuda.synchronize()
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse.cpu().numpy(), atol=LSE_ATOL)
    assert (out.float() - ref_out.float()).abs().max().item() <= 8e-3
    expected = E.exact_block_mass(q.float().numpy(), k.float().numpy(),
                                  lse[0].cpu().numpy(), 128)
    # P enters the fused sums in bf16, as it enters P V (unbiased rounding,
    # at most 2^-9 per term).
    np.testing.assert_allclose(mass.cpu().numpy(), expected, rtol=5e-4, atol=MASS_ATOL)
    np.testing.assert_allclose(mass.cpu().numpy(), ref_mass.cpu().numpy(), rtol=5e-4,
                               atol=MASS_ATOL)
    valid = np.minimum(128, tokens - 128 * np.arange(mass.shape[1]))
    np.testing.assert_allclose(mass.sum(-1).cpu().numpy(),
                               np.broadcast_to(valid, mass.shape[:2]), rtol=2e-4)


def test_block_mass_explicit_softmax_reference_test(ops, cuda_device):
    """tests/test_flex_backend.py:78-99 at head_dim 128: 250 tokens, 2 heads;
    LSE from an fp32 logsumexp rather than the attention kernel."""
    generator = torch.Generator().manual_seed(3)
    q = torch.randn(1, 250, 2, 128, generator=generator).to(torch.bfloat16)
    k = torch.randn(1, 250, 2, 128, generator=generator).to(torch.bfloat16)
    scores = (q.transpose(1, 2).float() @ k.transpose(1, 2).float().transpose(-1, -2)) * 128 ** -0.5
    lse = scores.logsumexp(-1)
    got = ops.block_mass(q.to(cuda_device), k.to(cuda_device), lse.to(cuda_device))
    torch.cuda.synchronize()
    probabilities = scores.softmax(-1)[0]
    padded = torch.nn.functional.pad(probabilities, (0, 6, 0, 6))
    expected = padded.reshape(2, 2, 128, 2, 128).sum((2, 4))
    torch.testing.assert_close(got.cpu(), expected, atol=2e-5, rtol=2e-5)


def test_block_mass_strided_views(ops, cuda_device):
    """The Diffusers processor's [B,H,T,D].transpose(1,2) views give the same mass."""
    q, k, v = _inputs(640, 3, seed=5)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    qt, kt, vt = (x.transpose(1, 2).contiguous().transpose(1, 2) for x in (qd, kd, vd))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    a = ops.block_mass(qd, kd, lse)
    b = ops.block_mass(qt, kt, lse[0])
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_block_mass_is_deterministic(ops, cuda_device):
    """Full size: a cross-wave LDS handoff that races shows up as run-to-run
    differences (and as wrong row sums below)."""
    q, k, v = _inputs(57600, 2, seed=9)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    a = ops.block_mass(qd, kd, lse)
    b = ops.block_mass(qd, kd, lse)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_block_mass_full_size_rows(ops, cuda_device):
    """57,600 tokens (450 blocks), 2 heads: every row sums to 128 and sampled
    (h, qb) rows match the fp64 restatement."""
    tokens, heads = 57600, 2
    q, k, v = _inputs(tokens, heads, seed=21)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    mass = ops.block_mass(qd, kd, lse)
    torch.cuda.synchronize()
    got = mass.cpu().numpy()
    np.testing.assert_allclose(got.sum(-1), 128.0, rtol=1e-4)
    rows = [(0, 0), (0, 224), (1, 449), (1, 17)]
    expected = E.exact_block_mass_rows(q.float().numpy(), k.float().numpy(),
                                       lse[0].cpu().numpy(), 128, rows)
    for i, (h, qb) in enumerate(rows):
        np.testing.assert_allclose(got[h, qb], expected[i], rtol=MASS_RTOL, atol=MASS_ATOL)


def test_block_mass_rejects_bad_arguments(ops, cuda_device):
    q, k, v = _inputs(256, 2, seed=1)
    qd, kd = q.to(cuda_device), k.to(cuda_device)
    lse = torch.zeros(1, 2, 256, device=cuda_device)
    with pytest.raises(ValueError):
        ops.block_mass(qd, kd, lse[:, :, :100])
    with pytest.raises(ValueError):
        ops.block_mass(qd, kd, lse.double())
    with pytest.raises(ValueError):
        ops.block_mass(torch.cat([qd, qd]), torch.cat([kd, kd]), lse)


@pytest.fixture
def backends():
    from dit_sparse_atten_amd.attention_backends import context, flex
    context.reset_runtime_state()
    yield flex, context
    context.reset_runtime_state()


def test_exact_bootstrap_then_sparse_reuse(backends, ops, cuda_device):
    """Default bootstrap_mode="exact": step 0 is dense; the route is the
    top-mass route of the exact mass plus the sink; step 1 runs sparse on it."""
    flex, context = backends
    tokens, heads, grid = 2048, 4, (2, 16, 64)
    q, k, v = _inputs(tokens, heads, seed=31)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(keep=0.625, mass_target=0.95,
                                                         total_steps=3))
    context.set_routing_context(attention_id=2, step=0, branch=0, grid=grid)
    out0 = backend(qd, kd, vd)
    torch.cuda.synchronize()
    dense, _ = A.block_sparse_attention(*(x.float().numpy() for x in (q, k, v)), None, 128)
    metrics = A.summarize(out0.float().cpu().numpy(), dense)
    assert metrics["max_absolute_error"] <= 2e-2 and metrics["cosine_similarity"] >= 0.9995
    assert backend.phase_counts["dense_bootstrap"] == 1
    state = next(iter(backend.state.values()))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    mass = ops.block_mass(qd, kd, lse).cpu().numpy()
    expected = E.exact_route(mass, 0.95, 0.625, grid=grid)
    assert (state["route"].cpu().numpy() == expected).all()
    # The mass itself is the oracle's within tolerance.
    oracle_mass = E.exact_block_mass(q.float().numpy(), k.float().numpy(),
                                      lse[0].cpu().numpy(), 128)
    np.testing.assert_allclose(mass, oracle_mass, rtol=MASS_RTOL, atol=MASS_ATOL)
    context.set_routing_context(attention_id=2, step=1, branch=0, grid=grid)
    out1 = backend(qd, kd, vd)
    torch.cuda.synchronize()
    sparse, _ = A.block_sparse_attention(*(x.float().numpy() for x in (q, k, v)), expected, 128)
    metrics = A.summarize(out1.float().cpu().numpy(), sparse)
    assert metrics["max_absolute_error"] <= 2e-2 and metrics["cosine_similarity"] >= 0.9995
    assert backend.phase_counts["sparse_reuse"] == 1


def test_periodic_exact_refresh_replaces_route(backends, cuda_device):
    """tests/test_flex_route_update.py:7-38 at head_dim 128: an exact refresh
    every 2 steps replaces a pre-seeded empty route."""
    flex, context = backends
    tokens, heads, head_dim = 256, 2, 128
    context.set_routing_context(attention_id=1, step=1, branch=0)
    q = torch.randn(1, tokens, heads, head_dim, device=cuda_device, dtype=torch.bfloat16)
    k = torch.randn_like(q)
    v = torch.randn_like(q)
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        block_size=128, keep=.5, mass_target=.9, compile_kernel=False, update_interval=2))
    backend.state[(1, 0, tokens, heads, head_dim, q.device, None)] = {
        "route": torch.zeros(heads, 2, 2, device=cuda_device, dtype=torch.bool),
        "block_mask": object(),
        "step": -1,
        "grid": None,
        "layout": None,
    }
    output = backend(q, k, v)
    torch.cuda.synchronize()
    assert output.shape == q.shape[:3] + (head_dim,)
    state = next(iter(backend.state.values()))
    assert state["step"] == 1
    assert state["route"].any()
    assert state["block_mask"] is not None
    assert backend.phase_counts["exact_refresh"] == 1
    expected, _ = A.block_sparse_attention(*(x.float().cpu().numpy() for x in (q, k, v)),
                                           None, 128)
    metrics = A.summarize(output.float().cpu().numpy(), expected)
    assert metrics["max_absolute_error"] <= 2e-2 and metrics["cosine_similarity"] >= 0.9995


def test_exact_refresh_route_matches_oracle_selection(backends, ops, cuda_device):
    """The refreshed route is the oracle's top-mass selection of the exact mass
    (cap ceil(K * keep), sink after the cap), bit for bit."""
    flex, context = backends
    tokens, heads, grid = 4096, 2, (4, 16, 64)
    q, k, v = _inputs(tokens, heads, seed=41)
    qd, kd, vd = (x.to(cuda_device) for x in (q, k, v))
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        keep=0.5, mass_target=0.9, update_interval=1, total_steps=4))
    for step in range(2):
        context.set_routing_context(attention_id=1, step=step, branch=0, grid=grid)
        backend(qd, kd, vd)
    torch.cuda.synchronize()
    assert backend.phase_counts["dense_bootstrap"] == 1
    assert backend.phase_counts["exact_refresh"] == 1
    state = next(iter(backend.state.values()))
    _, lse = ops.bsa_fwd(qd, kd, vd, return_lse=True)
    mass = ops.block_mass(qd, kd, lse).cpu().numpy()
    route = R.first_frame_sink(R.top_mass_route(mass, 0.9, 0.5), grid, 128)
    assert (state["route"].cpu().numpy() == route).all()

"""GPU tests of the backend mirror (flex_reuse / dense): the reference's own
backend tests re-run on the HIP path, plus the north-star 5-step schedule
checked step by step against the oracle."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import route as R
from tests.golden.inputs import clustered_qkv

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MIN_COSINE = 0.9995


@pytest.fixture
def backends(monkeypatch):
    from dit_sparse_atten_amd.attention_backends import context, flex
    context.reset_runtime_state()
    yield flex, context
    context.reset_runtime_state()


def _assert_close(actual, expected):
    metrics = A.summarize(actual, expected)
    assert metrics["max_absolute_error"] <= MAX_ABS, metrics
    assert metrics["cosine_similarity"] >= MIN_COSINE, metrics


def _oracle_with_layout(q, k, v, route, permutation, block=128):
    """Attention whose blocks are formed in the permuted token order."""
    qp, kp, vp = (x.float().numpy()[:, permutation] for x in (q, k, v))
    out, _ = A.block_sparse_attention(qp, kp, vp, route, block)
    restored = np.empty_like(out)
    restored[:, permutation] = out
    return restored


def test_first_layer_is_always_dense(backends, cuda_device):
    """tests/test_flex_route_update.py:115-132, in bf16 on the GPU."""
    flex, context = backends
    context.set_routing_context(attention_id=0, step=3, branch=1, grid=(2, 2, 2))
    q, k, v = (torch.randn(1, 8, 2, 128, device=cuda_device) for _ in range(3))
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(bootstrap_mode="sampled"))
    output = backend(q, k, v)
    assert output.dtype == torch.float32 and output.shape == q.shape
    expected, _ = A.block_sparse_attention(*(x.bfloat16().float().cpu().numpy()
                                             for x in (q, k, v)), None, 128)
    _assert_close(output.cpu().numpy(), expected)
    assert backend.state == {}
    assert backend.phase_counts["first_layer_dense"] == 1


def test_spatial_sampled_bootstrap_restores_original_order(backends, cuda_device):
    """tests/test_flex_route_update.py:76-103: grid (1,4,64), micro-tile (4,8)."""
    flex, context = backends
    context.set_routing_context(attention_id=1, step=0, branch=0, grid=(1, 4, 64))
    generator = torch.Generator().manual_seed(8)
    q, k, v = (torch.randn(1, 256, 2, 128, generator=generator).to(torch.bfloat16)
               for _ in range(3))
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        bootstrap_mode="sampled", prefetch_sampled_bootstrap=False, spatial_reorder=True,
        spatial_microtile_tokens=32, route_samples=2, total_steps=2))
    output = backend(q.to(cuda_device), k.to(cuda_device), v.to(cuda_device))
    expected, _ = A.block_sparse_attention(q.float().numpy(), k.float().numpy(),
                                           v.float().numpy(), None, 128)
    _assert_close(output.float().cpu().numpy(), expected)
    state = next(iter(backend.state.values()))
    assert state["layout"].microtile_shape == (4, 8)
    assert state["route"] is not None and state["block_mask"] is not None


def test_sampled_update_can_switch_route_to_dense(backends, cuda_device, monkeypatch):
    """tests/test_flex_route_update.py:41-73: an all-ones route at threshold .75."""
    flex, context = backends
    context.set_routing_context(attention_id=1, step=1, branch=0)
    q, k, v = (torch.randn(1, 128, 1, 128, device=cuda_device).bfloat16() for _ in range(3))
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        bootstrap_mode="sampled", sampled_update_interval=1, prefetch_sampled_update=False,
        dense_route_threshold=.75, total_steps=3))
    key = (1, 0, 128, 1, 128, q.device, None)
    backend.state[key] = {
        "route": torch.eye(1, dtype=torch.bool, device=cuda_device).unsqueeze(0),
        "block_mask": None, "step": 0, "dense": False, "grid": None, "layout": None}
    monkeypatch.setattr(backend, "_sampled_route", lambda state, query, k_, scale: {
        "route": torch.ones(1, 1, 1, dtype=torch.bool, device=cuda_device), "frontier": None})
    output = backend(q, k, v)
    expected, _ = A.block_sparse_attention(*(x.float().cpu().numpy() for x in (q, k, v)),
                                           None, 128)
    _assert_close(output.float().cpu().numpy(), expected)
    assert backend.state[key]["dense"] is True
    assert backend.phase_counts["dense_dispatch"] == 1


def test_dense_dispatched_state_skips_reorder(backends, cuda_device, monkeypatch):
    """A dense-dispatched (layer, branch) with a spatial layout runs dense
    attention on the caller's token order: same output as the dense oracle,
    no reorder or restore, released on the final step."""
    flex, context = backends
    grid = (2, 16, 32)
    tokens = math.prod(grid)
    q, k, v = clustered_qkv(tokens, 2, 128, group=64, seed=21, dtype=torch.bfloat16)
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        bootstrap_mode="sampled", dense_route_threshold=0.58, total_steps=4,
        spatial_reorder=True))
    layout = backend._spatial_layout(grid, tokens)
    key = (2, 1, tokens, 2, 128, cuda_device, layout.signature)

    def no_permute(*args, **kwargs):
        raise AssertionError("a dense-dispatched state must not permute tokens")

    monkeypatch.setattr(type(layout), "reorder_qkv", no_permute)
    monkeypatch.setattr(type(layout), "restore", no_permute)
    for step in (2, 3):
        backend.state[key] = {"route": None, "block_mask": None, "step": 1, "dense": True,
                              "keep": 0.7, "grid": grid, "layout": layout}
        context.set_routing_context(attention_id=2, step=step, branch=1, grid=grid)
        output = backend(q.to(cuda_device), k.to(cuda_device), v.to(cuda_device))
        expected, _ = A.block_sparse_attention(*(x.float().numpy() for x in (q, k, v)),
                                               None, 128)
        _assert_close(output.float().cpu().numpy(), expected)
        assert backend.phase_counts["dense_dispatch"] == step - 1
    assert key not in backend.state
    assert backend.finished_routes == [{"keep": 0.7, "frontier_fraction": None, "dense": True}]


def test_sampled_route_is_bit_exact_to_oracle_selection(backends, cuda_device):
    """The backend's route equals the oracle's prior+top-mass+sink on the same mass."""
    flex, context = backends
    tokens, heads, grid = 2048, 4, (2, 16, 64)
    q, k, _ = clustered_qkv(tokens, heads, 128, group=128, seed=3, dtype=torch.bfloat16)
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        bootstrap_mode="sampled", route_samples=16, mass_target=0.95, keep=0.625))
    generator = torch.Generator().manual_seed(4)
    previous = (torch.rand(heads, 16, 16, generator=generator) < 0.625).to(cuda_device)
    state = {"route": previous, "grid": grid, "layout": None}
    qd, kd = q.to(cuda_device), k.to(cuda_device)
    result = backend._sampled_route(state, qd, kd, None)
    mass = flex._sampled_block_mass(qd, kd, 128, samples=16).cpu().numpy()
    expected = R.sampled_route(None, None, 128, 16, 0.95, 0.625,
                               previous=previous.cpu().numpy(), rho=0.5, grid=grid, mass=mass)
    assert (result["route"].cpu().numpy() == expected).all()
    assert (result["counts"].cpu().numpy() == expected.sum(-1)).all()


def test_north_star_schedule_step_by_step(backends, cuda_device):
    """Sampled bootstrap with prefetch, sampled update every 2 steps without
    prefetch, dense dispatch at keep >= .58, spatial reorder, 5 steps, one CFG
    pair; each output checked against the oracle on the route actually used."""
    flex, context = backends
    grid = (4, 16, 32)  # 2048 tokens, 16 blocks, micro-tile 1x16 -> 2x16? (chosen by layout)
    tokens, heads = math.prod(grid), 4
    config = flex.FlexReuseConfig(
        bootstrap_mode="sampled", prefetch_sampled_bootstrap=True,
        sampled_update_interval=2, prefetch_sampled_update=False, route_samples=16,
        mass_target=0.95, keep=0.625, dense_route_threshold=0.58, total_steps=5,
        spatial_reorder=True)
    backend = flex.FlexReuseBackend(config)
    layout = backend._spatial_layout(grid, tokens)
    permutation = layout.permutation_cpu.numpy()
    inputs = {}
    for step in range(5):
        for branch in range(2):
            q, k, v = clustered_qkv(tokens, heads, 128, group=64, seed=10 * step + branch,
                                    dtype=torch.bfloat16)
            context.set_routing_context(attention_id=3, step=step, branch=branch, grid=grid)
            key = (3, branch, tokens, heads, 128, cuda_device, layout.signature)
            before = backend.state.get(key)
            output = backend(q.to(cuda_device), k.to(cuda_device), v.to(cuda_device))
            torch.cuda.synchronize()
            after = backend.state.get(key, before)
            used = None
            if step > 0 and after is not None and not after.get("dense"):
                used = after["route"].cpu().numpy() if after.get("route") is not None else None
            if step == 0 or used is None:
                expected, _ = A.block_sparse_attention(
                    *(x.float().numpy() for x in (q, k, v)), None, 128)
            else:
                expected = _oracle_with_layout(q, k, v, used, permutation)
            _assert_close(output.float().cpu().numpy(), expected)
            inputs[(step, branch)] = (q, k)
    counts = backend.phase_counts
    assert counts["sampled_bootstrap"] == 2
    # Steps 1..4 of two branches run sparse or dense, never both.
    assert counts["sparse_reuse"] + counts["dense_dispatch"] == 8
    assert counts["sampled_update"] <= 2
    # Final step released every route.
    assert backend.state == {}
    assert len(backend.finished_routes) == 2
    summary = backend.profile_summary()
    assert summary["released_routes"] == 2


def test_dense_backend_dtype_and_q_scale(cuda_device):
    from dit_sparse_atten_amd.attention_backends import DenseBackend
    generator = torch.Generator().manual_seed(2)
    q, k, v = (torch.randn(2, 300, 3, 128, generator=generator) for _ in range(3))
    out = DenseBackend()(q.to(cuda_device), k.to(cuda_device), v.to(cuda_device),
                         q_scale=0.5, softmax_scale=0.1)
    assert out.dtype == torch.float32
    qs = (q.bfloat16() * 0.5).bfloat16()
    expected, _ = A.block_sparse_attention(qs.float().numpy(), k.bfloat16().float().numpy(),
                                           v.bfloat16().float().numpy(), None, 128, scale=0.1)
    _assert_close(out.cpu().numpy(), expected)


@pytest.mark.parametrize("name", ["dense", "flex_reuse", "sparse"])
def test_diffusers_processor_call_pattern(cuda_device, name):
    """wan_diffusers.py:52-68: [B,T,H,D] views of BHSD storage, the processor's
    keywords (attention_mask included), output [B,T,H,D] in the caller's dtype;
    infer.py:259-260 sets an attribute on the backend."""
    from dit_sparse_atten_amd.attention_backends import BACKENDS, context
    context.reset_runtime_state()
    try:
        backend = BACKENDS[name]()
        backend.svg_operator_status = {"enabled": False}
        grid = (2, 8, 16)
        tokens, heads = math.prod(grid), 2
        generator = torch.Generator().manual_seed(31)
        storage = [torch.randn(1, heads, tokens, 128, generator=generator).bfloat16()
                   for _ in range(3)]
        q, k, v = (x.to(cuda_device).transpose(1, 2) for x in storage)
        assert q.stride() == (heads * tokens * 128, 128, tokens * 128, 1)
        # Layer 1, step 0: flex_reuse and sparse bootstrap (dense output + route).
        context.set_routing_context(attention_id=1, step=0, branch=0, grid=grid)
        out = backend(q, k, v, dropout_p=0.0, softmax_scale=None, causal=False,
                      window_size=(-1, -1), dtype=q.dtype, attention_mask=None)
        assert out.shape == q.shape and out.dtype == q.dtype
        expected, _ = A.block_sparse_attention(
            *(x.transpose(1, 2).float().numpy() for x in storage), None, 128)
        _assert_close(out.float().cpu().numpy(), expected)
    finally:
        context.reset_runtime_state()


def test_flex_hybrid_at_81_frames(backends, cuda_device):
    """Wan's default 81 frames at 720p: grid (21, 45, 80), 75,600 tokens, 591
    blocks (above the 512 of a one-wave 8-key-per-lane sort).  Sampled
    bootstrap, activation with frontier, sampled update; routes hold the sink
    and stay within the cap; outputs are finite and sampled rows match a
    float32 softmax over the route's key blocks."""
    flex, context = backends
    grid = (21, 45, 80)
    tokens, heads = math.prod(grid), 2
    generator = torch.Generator(device=cuda_device).manual_seed(81)
    q, k, v = (torch.randn(1, tokens, heads, 128, device=cuda_device,
                           generator=generator).bfloat16() for _ in range(3))
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        bootstrap_mode="sampled", prefetch_sampled_bootstrap=True, sampled_update_interval=2,
        prefetch_sampled_update=False, route_samples=16, mass_target=0.95, keep=0.625,
        total_steps=5, spatial_reorder=True))
    layout = backend._spatial_layout(grid, tokens)
    blocks = layout.neighbors_cpu.shape[0]
    assert blocks == 591
    cap = math.ceil(blocks * 0.625)
    sink = math.ceil(45 * 80 / 128)
    for step in range(3):
        context.set_routing_context(attention_id=4, step=step, branch=0, grid=grid)
        out = backend(q, k, v)
        torch.cuda.synchronize()
        assert torch.isfinite(out.float()).all()
    state = next(iter(backend.state.values()))
    route = state["route"]
    assert route.shape == (heads, blocks, blocks) and route[..., :sink].all()
    assert int(route.sum(-1).max()) <= cap + sink
    assert backend.phase_counts["sampled_bootstrap"] == 1
    assert backend.phase_counts["sampled_update"] == 1
    # 32 sampled query rows of head 1 against a float32 softmax over the route.
    perm = layout.permutation_cpu.long()
    qp, kp, vp = (x[0, perm.to(cuda_device), 1].float() for x in (q, k, v))
    rows = torch.randperm(tokens, generator=torch.Generator().manual_seed(5))[:32]
    keys_on = route[1][(rows // 128).to(cuda_device)].repeat_interleave(128, dim=-1)[:, :tokens]
    scores = qp[rows.to(cuda_device)] @ kp.T * 128 ** -0.5
    probs = torch.softmax(scores.masked_fill(~keys_on, float("-inf")), dim=-1)
    expected = probs @ vp
    got = out[0, perm.to(cuda_device)[rows.to(cuda_device)], 1].float()
    cosine = torch.nn.functional.cosine_similarity(got.flatten(), expected.flatten(), dim=0)
    assert (got - expected).abs().max().item() <= MAX_ABS and cosine.item() >= MIN_COSINE

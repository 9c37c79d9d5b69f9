"""GPU checks of the end-to-end loop's pieces: the DiT elementwise kernels
against plain torch float32 references of the same ops, a small Wan-shaped
DiT forward against a float32 torch restatement with the same weights, and the
5-step CFG loop through the flex_reuse hybrid (phase counts as the reference's
schedule produces them)."""

import math

import pytest
import torch
import torch.nn.functional as F

from tests.golden.inputs import apply_rope, wan_rope_angles

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops():
    from dit_sparse_atten_amd import ops as module
    return module


def _cos(a, b):
    a, b = a.float().reshape(-1), b.float().reshape(-1)
    return float(torch.dot(a, b) / (a.norm() * b.norm()))


def test_layernorm_modulate_matches_torch(ops, cuda_device):
    gen = torch.Generator(device=cuda_device).manual_seed(1)
    x = torch.randn(2, 300, 1536, device=cuda_device, generator=gen).bfloat16()
    shift = torch.randn(2, 1536, device=cuda_device, generator=gen) * 0.1
    scale = torch.randn(2, 1536, device=cuda_device, generator=gen) * 0.1
    weight = 1 + torch.randn(1536, device=cuda_device, generator=gen) * 0.1
    bias = torch.randn(1536, device=cuda_device, generator=gen) * 0.1
    ln = F.layer_norm(x.float(), (1536,), eps=1e-6)
    got = ops.layernorm_modulate(x, shift=shift, scale=scale)
    want = ln * (1 + scale[:, None]) + shift[:, None]
    torch.testing.assert_close(got.float(), want, atol=2e-2, rtol=1e-2)
    got = ops.layernorm_modulate(x, weight=weight, bias=bias)
    torch.testing.assert_close(got.float(), ln * weight + bias, atol=2e-2, rtol=1e-2)


def test_rmsnorm_rope_matches_torch(ops, cuda_device):
    from dit_sparse_atten_amd.wan_dit import rope_cos_sin
    grid = (3, 10, 10)
    tokens = math.prod(grid)
    gen = torch.Generator(device=cuda_device).manual_seed(2)
    x = torch.randn(1, tokens, 1536, device=cuda_device, generator=gen).bfloat16()
    weight = 1 + torch.randn(1536, device=cuda_device, generator=gen) * 0.1
    got = ops.rmsnorm_rope(x, weight, 128, rope_cos_sin(grid, device=cuda_device))
    xf = x.float()
    normed = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * weight
    want = apply_rope(normed.view(1, tokens, 12, 128).cpu().double(), wan_rope_angles(grid))
    torch.testing.assert_close(got.float().cpu(), want.float().reshape(1, tokens, 1536),
                               atol=2e-2, rtol=1e-2)
    # Without a table: RMSNorm only.
    got = ops.rmsnorm_rope(x, weight, 128, None)
    torch.testing.assert_close(got.float(), normed, atol=2e-2, rtol=1e-2)


def test_gated_residual_matches_torch(ops, cuda_device):
    gen = torch.Generator(device=cuda_device).manual_seed(3)
    x = torch.randn(1, 100, 512, device=cuda_device, generator=gen).bfloat16()
    y = torch.randn(1, 100, 512, device=cuda_device, generator=gen).bfloat16()
    gate = torch.randn(1, 512, device=cuda_device, generator=gen)
    torch.testing.assert_close(ops.gated_residual(x, y, gate).float(),
                               x.float() + gate * y.float(), atol=2e-2, rtol=1e-2)
    z = x.clone()
    ops.gated_residual(z, y, out=z)
    torch.testing.assert_close(z.float(), x.float() + y.float(), atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("dim", [8, 520, 1536, 5120, 8192])
def test_row_kernels_every_chunk_count_in_place(ops, cuda_device, dim):
    """Each chunk-count instantiation (dim / 512 rounded up: 1, 2, 3, 16 with
    bounds), a row count that leaves the last workgroup partial, two groups,
    and in-place output."""
    gen = torch.Generator(device=cuda_device).manual_seed(dim)
    rows_per_group, groups, head_dim = 37, 2, 8
    x = torch.randn(groups, rows_per_group, dim, device=cuda_device, generator=gen).bfloat16()
    y = torch.randn_like(x)
    shift, scale, gate = (torch.randn(groups, dim, device=cuda_device, generator=gen) * 0.1
                          for _ in range(3))
    weight = 1 + torch.randn(dim, device=cuda_device, generator=gen) * 0.1
    angles = torch.rand(rows_per_group, head_dim // 2, device=cuda_device, generator=gen) * 6
    cos_sin = torch.stack([angles.cos(), angles.sin()], dim=-1).contiguous()

    ln = F.layer_norm(x.float(), (dim,), eps=1e-6) * (1 + scale[:, None]) + shift[:, None]
    z = x.clone()
    ops.layernorm_modulate(z, shift=shift, scale=scale, out=z)
    torch.testing.assert_close(z.float(), ln, atol=2e-2, rtol=1e-2)

    xf = x.float()
    normed = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * weight
    pairs = normed.view(groups, rows_per_group, dim // head_dim, head_dim // 2, 2)
    c, s = cos_sin[None, :, None, :, 0], cos_sin[None, :, None, :, 1]
    rotated = torch.stack([pairs[..., 0] * c - pairs[..., 1] * s,
                           pairs[..., 0] * s + pairs[..., 1] * c], dim=-1).reshape(x.shape)
    z = x.clone()
    ops.rmsnorm_rope(z, weight, head_dim, cos_sin, out=z)
    torch.testing.assert_close(z.float(), rotated, atol=2e-2, rtol=1e-2)

    z = x.clone()
    ops.gated_residual(z, y, gate, out=z)
    torch.testing.assert_close(z.float(), xf + gate[:, None] * y.float(), atol=2e-2, rtol=1e-2)


def _small_config():
    from dit_sparse_atten_amd.wan_dit import WanDiTConfig
    return WanDiTConfig(layers=2, dim=256, heads=2, ffn_dim=512, text_dim=64, freq_dim=32)


def _torch_forward(model, latents, timestep, text):
    """float32 torch restatement of WanDiT.forward with the model's weights."""
    from dit_sparse_atten_amd.wan_dit import _sinusoidal
    c = model.config
    f32 = lambda pair: (pair[0].float(), pair[1].float())  # noqa: E731
    _, channels, frames, height, width = latents.shape
    grid = (frames, height // 2, width // 2)
    tokens = math.prod(grid)
    p = latents.float().reshape(1, channels, grid[0], 1, grid[1], 2, grid[2], 2)
    p = p.permute(0, 2, 4, 6, 1, 3, 5, 7).reshape(1, tokens, -1)
    x = F.linear(p, *f32(model.patch))
    ctx = F.linear(F.gelu(F.linear(text.float(), *f32(model.text1)), approximate="tanh"),
                   *f32(model.text2))
    t = _sinusoidal(timestep, c.freq_dim).to(latents.device)
    temb = F.linear(F.silu(F.linear(t, *f32(model.time1))), *f32(model.time2))
    temb6 = F.linear(F.silu(temb), *f32(model.time_proj)).view(6, c.dim)
    angles = wan_rope_angles(grid).to(latents.device)

    def rms(v, w):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + c.eps) * w

    def rope(v):
        return apply_rope(v.view(1, -1, c.heads, 128).double(), angles).float().reshape(v.shape)

    def attention(q, k, v):
        q, k, v = (t.view(1, -1, c.heads, 128).transpose(1, 2) for t in (q, k, v))
        probs = torch.softmax(q @ k.transpose(-1, -2).contiguous() * 128 ** -0.5, dim=-1)
        return (probs @ v).transpose(1, 2).reshape(1, -1, c.dim)

    for blk in model.blocks:
        mod = blk["table"] + temb6
        h = F.layer_norm(x, (c.dim,), eps=c.eps) * (1 + mod[1]) + mod[0]
        q = rope(rms(F.linear(h, *f32(blk["q"])), blk["norm_q"]))
        k = rope(rms(F.linear(h, *f32(blk["k"])), blk["norm_k"]))
        v = F.linear(h, *f32(blk["v"]))
        x = x + mod[2] * F.linear(attention(q, k, v), *f32(blk["o"]))
        h = F.layer_norm(x, (c.dim,), blk["norm2_w"], blk["norm2_b"], eps=c.eps)
        q = rms(F.linear(h, *f32(blk["cq"])), blk["cnorm_q"])
        k = rms(F.linear(ctx, *f32(blk["ck"])), blk["cnorm_k"])
        v = F.linear(ctx, *f32(blk["cv"]))
        x = x + F.linear(attention(q, k, v), *f32(blk["co"]))
        h = F.layer_norm(x, (c.dim,), eps=c.eps) * (1 + mod[4]) + mod[3]
        x = x + mod[5] * F.linear(F.gelu(F.linear(h, *f32(blk["ffn1"])), approximate="tanh"),
                                  *f32(blk["ffn2"]))
    shift_scale = model.head_table + temb.view(1, c.dim)
    h = F.layer_norm(x, (c.dim,), eps=c.eps) * (1 + shift_scale[1]) + shift_scale[0]
    out = F.linear(h, *f32(model.head)).reshape(1, *grid, channels, 1, 2, 2)
    return out.permute(0, 4, 1, 5, 2, 6, 3, 7).reshape(latents.shape)


def test_small_dit_forward_matches_torch(cuda_device):
    from dit_sparse_atten_amd.attention_backends import context
    from dit_sparse_atten_amd.attention_backends.dense import DenseBackend
    from dit_sparse_atten_amd.wan_dit import WanDiT
    context.reset_runtime_state()
    model = WanDiT(_small_config(), device=cuda_device, seed=1)
    gen = torch.Generator(device=cuda_device).manual_seed(4)
    latents = torch.randn(1, 16, 2, 16, 32, device=cuda_device, generator=gen).bfloat16()
    text = torch.randn(1, 24, 64, device=cuda_device, generator=gen).bfloat16()
    got = model(latents, 952.0, model.embed_text(text), DenseBackend())
    want = _torch_forward(model, latents, 952.0, text)
    torch.cuda.synchronize()
    assert got.shape == latents.shape
    assert _cos(got, want) >= 0.999
    context.reset_runtime_state()


def test_denoise_loop_with_flex_hybrid(cuda_device):
    """5 steps x CFG pair through flex_reuse with the reference's hybrid
    settings: every layer but the first bootstraps (sampled, prefetched),
    updates every 2 steps and releases its routes on the final step."""
    from dit_sparse_atten_amd.attention_backends import context, flex
    from dit_sparse_atten_amd.wan_dit import WanDiT, denoise
    context.reset_runtime_state()
    model = WanDiT(_small_config(), device=cuda_device, seed=2)
    backend = flex.FlexReuseBackend(flex.FlexReuseConfig(
        bootstrap_mode="sampled", prefetch_sampled_bootstrap=True, sampled_update_interval=2,
        prefetch_sampled_update=False, route_samples=16, mass_target=0.95, keep=0.625,
        dense_route_threshold=None, total_steps=5, spatial_reorder=True))
    gen = torch.Generator(device=cuda_device).manual_seed(5)
    latents = torch.randn(1, 16, 2, 32, 64, device=cuda_device, generator=gen).bfloat16()
    cond = torch.randn(1, 24, 64, device=cuda_device, generator=gen).bfloat16()
    out = denoise(model, backend, latents, cond, torch.zeros_like(cond))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    counts = backend.phase_counts
    assert counts["first_layer_dense"] == 10          # layer 0, 5 steps x 2 branches
    assert counts["sampled_bootstrap"] == 2           # layer 1, two branches
    assert counts["sparse_reuse"] == 8                # steps 1..4 of layer 1
    assert backend.profile_summary()["released_routes"] == 2
    context.reset_runtime_state()

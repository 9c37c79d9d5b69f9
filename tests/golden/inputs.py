"""Seeded synthetic inputs shared by the golden-fixture writer, the tests and
the bench (torch CPU generator, so every machine regenerates the same values).

The clustered distribution is BASELINE config 0: Q/K = 0.5*N(0,1) noise plus a
per-group centroid ~N(0,1) shared by the group's tokens; V ~ N(0,1).
"""

from __future__ import annotations

import torch


def group_of_tokens(tokens, group, permutation=None):
    """Group id of every original token.

    Without a permutation, consecutive runs of ``group`` tokens form a group.
    With one (permutation[p] = original token at layout position p), a group is
    ``group`` consecutive layout positions, e.g. one spatial tile.
    """
    positions = torch.arange(tokens)
    if permutation is None:
        return positions // group
    group_of = torch.empty(tokens, dtype=torch.long)
    group_of[torch.as_tensor(permutation, dtype=torch.long)] = positions // group
    return group_of


def clustered_qkv(tokens, heads, head_dim=128, group=64, seed=0, permutation=None,
                  dtype=torch.float32):
    """Return q, k, v as [1, tokens, heads, head_dim] CPU tensors."""
    generator = torch.Generator().manual_seed(seed)
    groups = -(-tokens // group)
    shape = (1, tokens, heads, head_dim)
    q_noise = torch.randn(shape, generator=generator)
    k_noise = torch.randn(shape, generator=generator)
    q_centroid = torch.randn((1, groups, heads, head_dim), generator=generator)
    k_centroid = torch.randn((1, groups, heads, head_dim), generator=generator)
    v = torch.randn(shape, generator=generator)
    group_of = group_of_tokens(tokens, group, permutation)
    q = 0.5 * q_noise + q_centroid[:, group_of]
    k = 0.5 * k_noise + k_centroid[:, group_of]
    return q.to(dtype), k.to(dtype), v.to(dtype)


def route_mass(heads, blocks, seed):
    """Heavy-tailed non-negative block mass [heads, blocks, blocks] float32:
    u^4 for u ~ U[0, 1).  Only elementwise fp32 products of the generator's
    output, so every machine reproduces it bit for bit."""
    generator = torch.Generator().manual_seed(seed)
    u = torch.rand((heads, blocks, blocks), generator=generator)
    u2 = u * u
    return u2 * u2


def random_route(heads, blocks, seed, keep=0.625):
    """Bernoulli(keep) boolean route [heads, blocks, blocks]."""
    generator = torch.Generator().manual_seed(seed)
    return torch.rand((heads, blocks, blocks), generator=generator) < keep


def wan_rope_angles(grid, head_dim=128, theta=10000.0):
    """Rotation angles [tokens, head_dim // 2] of a 3D RoPE over the (F, H, W)
    latent grid, flattened frame-major: head dims split into a time part of
    head_dim - 2 * 2 * (head_dim // 6) and two spatial parts of
    2 * (head_dim // 6) each (44 / 42 / 42 at d = 128); each part rotates its
    consecutive (even, odd) pairs by position * theta^(-2j / part)."""
    frames, height, width = grid
    spatial = 2 * (head_dim // 6)
    parts = (head_dim - 2 * spatial, spatial, spatial)
    positions = torch.stack(torch.meshgrid(
        torch.arange(frames), torch.arange(height), torch.arange(width), indexing="ij"),
        dim=-1).reshape(-1, 3).to(torch.float64)
    angles = []
    for axis, part in enumerate(parts):
        freqs = theta ** (-torch.arange(0, part, 2, dtype=torch.float64) / part)
        angles.append(positions[:, axis:axis + 1] * freqs[None])
    return torch.cat(angles, dim=-1)


def apply_rope(x, angles):
    """Rotate the (even, odd) pairs of x [B, T, H, D] by angles [T, D/2];
    computed in float64 and returned in x's dtype."""
    x64 = x.to(torch.float64)
    cos = torch.cos(angles)[None, :, None, :]
    sin = torch.sin(angles)[None, :, None, :]
    even, odd = x64[..., 0::2], x64[..., 1::2]
    out = torch.empty_like(x64)
    out[..., 0::2] = even * cos - odd * sin
    out[..., 1::2] = even * sin + odd * cos
    return out.to(x.dtype)


def rope_qkv(grid, batch, heads, head_dim=128, seed=0, dtype=torch.bfloat16):
    """BASELINE config 1 inputs: Q/K/V ~ N(0,1) [B, T, H, D], 3D RoPE on Q and K."""
    tokens = grid[0] * grid[1] * grid[2]
    generator = torch.Generator().manual_seed(seed)
    shape = (batch, tokens, heads, head_dim)
    q, k, v = (torch.randn(shape, generator=generator) for _ in range(3))
    angles = wan_rope_angles(grid, head_dim)
    return apply_rope(q, angles).to(dtype), apply_rope(k, angles).to(dtype), v.to(dtype)


def block_mass_like(heads, blocks, seed, centroid_dim=4, sharpness=16.0):
    """Softmax-shaped non-negative block mass [heads, blocks, blocks] float32
    with the structure of a sampled block mass: per block a query and a key
    centroid c ~ U(-1, 1)^centroid_dim, score s = <c_q, c_k> (summed in a fixed
    order), mass = 2^-16 max(0, 1 + s / sharpness)^16 (0.5 + u), u ~ U[0, 1),
    i.e. roughly exp(16 s / sharpness) with per-entry noise, entries below 1.
    Built from the torch CPU generator's uniform draws with elementwise fp32
    adds, multiplies and a clamp only, so every machine reproduces it bit for
    bit (no exp, no reduction)."""
    generator = torch.Generator().manual_seed(seed)
    cq = torch.rand((heads, blocks, 1, centroid_dim), generator=generator) * 2 - 1
    ck = torch.rand((heads, 1, blocks, centroid_dim), generator=generator) * 2 - 1
    noise = torch.rand((heads, blocks, blocks), generator=generator) + 0.5
    score = cq[..., 0] * ck[..., 0]
    for j in range(1, centroid_dim):
        score = score + cq[..., j] * ck[..., j]
    t = torch.clamp_min(score * (1.0 / sharpness) + 1.0, 0.0)
    for _ in range(4):
        t = t * t
    return t * noise * (2.0 ** -16)

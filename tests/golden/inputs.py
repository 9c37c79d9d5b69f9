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

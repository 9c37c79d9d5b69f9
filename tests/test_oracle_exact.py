"""Pins of the exact route-estimator oracle (CPU): the reference's own
identities for the exact block mass, the row-sum invariant, and planted
mistakes that each check must catch."""

import numpy as np
import pytest

from oracle import exact as E
from oracle import route as R
from tests.golden.inputs import clustered_qkv


def _qk(tokens, heads, dim, seed, group=16):
    q, k, _ = clustered_qkv(tokens, heads, dim, group=group, seed=seed)
    return q.numpy().astype(np.float64), k.numpy().astype(np.float64)


def test_full_sampling_equals_exact_over_block():
    """tests/test_flex_backend.py:43-53: sampling every token of every block
    gives mass_sampled = mass_exact / block."""
    q, k = _qk(12, 2, 8, seed=4, group=4)
    lse = E.dense_lse(q, k)
    exact = E.exact_block_mass(q, k, lse, 4)
    sampled = R.sampled_block_mass(q, k, 4, samples=4, bf16_scores=False)
    np.testing.assert_allclose(sampled, exact / 4, atol=1e-6, rtol=1e-6)


def test_matches_explicit_padded_softmax():
    """tests/test_flex_backend.py:62-76: 259 tokens, 3 blocks of 128."""
    q, k = _qk(259, 3, 16, seed=2)
    lse = E.dense_lse(q, k)
    actual = E.exact_block_mass(q, k, lse, 128)
    s = np.einsum("qhd,khd->hqk", q[0], k[0]) * 16 ** -0.5
    p = np.exp(s - s.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    padded = np.pad(p, ((0, 0), (0, 125), (0, 125)))
    expected = padded.reshape(3, 3, 128, 3, 128).sum((2, 4))
    np.testing.assert_allclose(actual, expected, atol=2e-12, rtol=1e-10)


@pytest.mark.parametrize("tokens,block", [(259, 128), (300, 128), (130, 64), (64, 64)])
def test_rows_sum_to_valid_queries(tokens, block):
    q, k = _qk(tokens, 2, 16, seed=tokens)
    mass = E.exact_block_mass(q, k, E.dense_lse(q, k), block)
    blocks = -(-tokens // block)
    valid = np.minimum(tokens - np.arange(blocks) * block, block)
    np.testing.assert_allclose(mass.sum(-1), np.broadcast_to(valid, mass.shape[:2]), rtol=1e-12)
    assert (mass >= 0).all()


def test_lse_is_the_row_normaliser():
    q, k = _qk(70, 2, 8, seed=1)
    lse = E.dense_lse(q, k)
    s = E.scores(q, k)
    np.testing.assert_allclose(np.exp(s - lse[..., None]).sum(-1), 1.0, rtol=1e-12)
    # Uniform scores: lse = log(T) + s.
    zeros = np.zeros((1, 70, 2, 8))
    np.testing.assert_allclose(E.dense_lse(zeros, zeros), np.log(70.0), rtol=1e-12)


def test_planted_mistakes_fail():
    """Each plausible slip changes the result beyond the tolerances above."""
    q, k = _qk(259, 2, 16, seed=3)
    lse = E.dense_lse(q, k)
    good = E.exact_block_mass(q, k, lse, 128)
    # Transposed block axes (query/key swapped).
    assert not np.allclose(good, good.transpose(0, 2, 1), rtol=1e-4)
    # A wrong scale (no d^-1/2).
    bad_scale = E.exact_block_mass(q, k, E.dense_lse(q, k, 1.0), 128, scale=1.0)
    assert not np.allclose(good, bad_scale, rtol=1e-4)
    # Normalising with another row's lse.
    assert not np.allclose(good, E.exact_block_mass(q, k, np.roll(lse, 1, axis=1), 128), rtol=1e-4)


def test_exact_route_adds_sink_after_cap():
    """The sink columns are OR-ed after the top-mass cap (flex.py:708-716)."""
    mass = np.zeros((1, 4, 8), np.float32)
    mass[..., -1] = 1.0
    route = E.exact_route(mass, 0.9, 0.125, grid=(2, 4, 16), block_size=64)
    assert route[..., -1].all()
    assert route[..., 0].all()
    assert route.sum(-1).tolist() == [[2, 2, 2, 2]]

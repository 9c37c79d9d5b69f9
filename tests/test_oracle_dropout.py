"""The dropout oracle (oracle/dropout.py) pinned on the CPU: Philox4x32-10
against the Random123 known-answer vectors, the uniformity of the mask, and
dropout_p -> 0 reducing to the closed form of oracle.attention."""

import numpy as np
import pytest

from oracle import attention as A
from oracle import dropout as D

# Random123's known-answer vectors for philox4x32-10: counter, key, output.
KAT = [
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF),
     (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter,key,want", KAT)
def test_philox_known_answers(counter, key, want):
    got = D.philox4x32_10(np.array(counter, dtype=np.uint32), np.array(key, dtype=np.uint32))
    assert [int(x) for x in got] == list(want)


def test_philox_broadcasts_like_single_calls():
    counters = np.array([c for c, _, _ in KAT], dtype=np.uint32)
    keys = np.array([k for _, k, _ in KAT], dtype=np.uint32)
    assert (D.philox4x32_10(counters, keys) == np.array([w for _, _, w in KAT])).all()


def test_planted_round_constant_fails_the_known_answer():
    """A wrong multiplier (a plausible slip) changes the first vector."""
    saved = D._M0
    try:
        D._M0 = np.uint64(0xD2511F55)
        got = D.philox4x32_10(np.zeros(4, dtype=np.uint32), np.zeros(2, dtype=np.uint32))
    finally:
        D._M0 = saved
    assert [int(x) for x in got] != list(KAT[0][2])


@pytest.mark.parametrize("p", [0.1, 0.5, 0.9])
def test_keep_fraction_is_one_minus_p(p):
    keep = D.keep_mask(2, 3, 64, 200, p, seed=1234, offset=7)
    n = keep.size
    sigma = np.sqrt(p * (1 - p) / n)
    assert abs(keep.mean() - (1 - p)) < 5 * sigma
    # Different seeds and offsets give different masks.
    assert (keep != D.keep_mask(2, 3, 64, 200, p, seed=1235, offset=7)).any()
    assert (keep != D.keep_mask(2, 3, 64, 200, p, seed=1234, offset=8)).any()


def test_keep_mask_layout():
    """Key k of row t takes word k % 4 of the counter (k // 4, t, bh, offset)."""
    seed, offset = (5 << 32) | 9, 3
    keep = D.keep_mask(1, 2, 3, 10, 0.5, seed, offset)
    words = D.philox4x32_10(np.array([2, 1, 1, offset], dtype=np.uint32),
                            np.array([9, 5], dtype=np.uint32))
    assert list(keep[0, 1, 1, 8:10]) == [bool(words[0] >= 2 ** 31), bool(words[1] >= 2 ** 31)]


def test_small_p_reduces_to_the_closed_form():
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((1, 40, 2, 16)) for _ in range(3))
    keep = np.ones((1, 2, 40, 40), dtype=bool)
    want, _ = A.block_sparse_attention(q, k, v, None, 128)
    np.testing.assert_allclose(D.dropout_attention(q, k, v, keep, 0.0), want, atol=1e-12)
    # Dropping every key but one leaves that key's weighted value.
    keep = np.zeros_like(keep)
    keep[..., 3] = True
    got = D.dropout_attention(q, k, v, keep, 0.5)
    scores = np.einsum("thd,khd->htk", q[0], k[0]) * 16 ** -0.5
    w = np.exp(scores - scores.max(-1, keepdims=True))
    w /= w.sum(-1, keepdims=True)
    expected = (w[:, :, 3:4] * v[0, 3][:, None, :]).transpose(1, 0, 2) / 0.5
    np.testing.assert_allclose(got[0], expected, atol=1e-12)

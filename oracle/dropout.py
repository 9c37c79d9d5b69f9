"""CPU restatement of dense attention with dropout (test infrastructure only).

The reference's DenseBackend hands ``dropout_p`` to SDPA
(attention_backends/dense.py:40-47), and ``flex_reuse`` sends calls with
dropout to it (flex.py:655-668).  SDPA applies dropout to the attention
probabilities: O = (keep * softmax(scale q k^T)) v / (1 - p), the softmax
normalised over every key.  torch's random stream is not reproduced (it is
torch's own); this build draws keep from Philox4x32-10 (Salmon, Moraes, Dror
and Shaw, "Parallel random numbers: as easy as 1, 2, 3", SC 2011), restated
here from the paper:

    round(c, k): (hi0, lo0) = 0xD2511F53 * c0, (hi1, lo1) = 0xCD9E8D57 * c2,
                 c' = (hi1 ^ c1 ^ k0, lo1, hi0 ^ c3 ^ k1, lo0)
    ten rounds, the key bumped by (0x9E3779B9, 0xBB67AE85) before each round
    but the first.

Pinned by: the Random123 known-answer vectors for philox4x32-10 (three
counter/key pairs), the uniformity of its outputs, and dropout_p -> 0
reducing to the closed form of oracle.attention (tests/test_oracle_dropout.py).
It is never imported by the product path.
"""

from __future__ import annotations

import numpy as np

_M0, _M1 = np.uint64(0xD2511F53), np.uint64(0xCD9E8D57)
_W0, _W1 = np.uint32(0x9E3779B9), np.uint32(0xBB67AE85)
_LOW = np.uint64(0xFFFFFFFF)


def philox4x32_10(counter, key):
    """Philox4x32-10 of counters [..., 4] and keys [..., 2] (uint32, broadcast);
    returns [..., 4] uint32."""
    c = [np.asarray(counter, dtype=np.uint32)[..., i] for i in range(4)]
    k0 = np.asarray(key, dtype=np.uint32)[..., 0].copy()
    k1 = np.asarray(key, dtype=np.uint32)[..., 1].copy()
    with np.errstate(over="ignore"):
        for round_ in range(10):
            if round_:
                k0 = k0 + _W0
                k1 = k1 + _W1
            p0 = c[0].astype(np.uint64) * _M0
            p1 = c[2].astype(np.uint64) * _M1
            hi0, lo0 = (p0 >> np.uint64(32)).astype(np.uint32), (p0 & _LOW).astype(np.uint32)
            hi1, lo1 = (p1 >> np.uint64(32)).astype(np.uint32), (p1 & _LOW).astype(np.uint32)
            c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return np.stack(c, axis=-1)


def keep_mask(batch, heads, q_tokens, kv_tokens, dropout_p, seed, offset=0):
    """keep[b, h, t, k]: the uniform of key k is word k % 4 of Philox4x32-10
    with counter (k // 4, t, b * heads + h, offset) and key (seed low word,
    seed high word); kept when it is >= round(dropout_p * 2^32) (at least 1),
    the layout of dsa_bsa_fwd_dropout (include/dsa.h)."""
    thresh = min(max(int(round(dropout_p * 2.0 ** 32)), 1), 2 ** 32 - 1)
    groups = -(-kv_tokens // 4)
    g, t, bh = np.meshgrid(np.arange(groups), np.arange(q_tokens), np.arange(batch * heads),
                           indexing="ij")
    counter = np.stack([g, t, bh, np.full_like(g, offset)], axis=-1).astype(np.uint32)
    key = np.array([seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF], dtype=np.uint32)
    words = philox4x32_10(counter, key)               # [groups, T, BH, 4]
    uniforms = words.transpose(2, 1, 0, 3).reshape(batch * heads, q_tokens, groups * 4)
    keep = uniforms[..., :kv_tokens] >= np.uint32(thresh)
    return keep.reshape(batch, heads, q_tokens, kv_tokens)


def dropout_attention(q, k, v, keep, dropout_p, scale=None, causal=False):
    """Dense attention with the given keep mask in float64: q [B,Tq,H,D],
    k/v [B,Tk,H,D], keep [B,H,Tq,Tk].  Returns O [B,Tq,H,D] float64."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    batch, q_tokens, heads, head_dim = q.shape
    kv_tokens = k.shape[1]
    if scale is None:
        scale = head_dim ** -0.5
    out = np.zeros_like(q)
    for b in range(batch):
        for h in range(heads):
            scores = q[b, :, h] @ k[b, :, h].T * scale
            if causal:
                later = np.arange(kv_tokens)[None, :] > np.arange(q_tokens)[:, None]
                scores = np.where(later, -np.inf, scores)
            weights = np.exp(scores - scores.max(-1, keepdims=True))
            weights /= weights.sum(-1, keepdims=True)
            out[b, :, h] = (weights * keep[b, h]) @ v[b, :, h] / (1.0 - dropout_p)
    return out

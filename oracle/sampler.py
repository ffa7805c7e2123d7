"""CPU restatement of the decode sampler (numpy).  TEST INFRASTRUCTURE.

sample_gumbel follows utils/sampler.py:35-53 of the reference:
    argmax( softmax(logits / T) / clamp(Exp(1) noise, 1e-10) )
with the noise supplied.  philox4x32_10 is the counter-based generator the
HIP sampler draws its noise from (Salmon, Moraes, Dror, Shaw, "Parallel
random numbers: as easy as 1, 2, 3", SC'11: 10 rounds of two 32x32->64-bit
multiplies by 0xD2511F53 / 0xCD9E8D57 with Weyl key increments 0x9E3779B9 /
0xBB67AE85), and exp_noise maps its words to Exp(1) variates exactly as the
kernel does: u = (w + 1) * 2^-32 in (0, 1], e = -log(u).

Pinning (tests/test_oracle_sampler.py): philox4x32_10 against the published
known-answer vectors of the Random123 distribution; sample_gumbel against a
brute-force scalar loop; the noise map against the Exp(1) moments.
"""
from __future__ import annotations

import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
MASK = 0xFFFFFFFF


def philox4x32_10(ctr, key):
    """ctr: 4 uint32 words (array-like [..., 4]); key: 2 uint32 words
    ([..., 2]).  Returns uint32 [..., 4]."""
    c = np.asarray(ctr, dtype=np.uint64).copy()
    k = np.asarray(key, dtype=np.uint64).copy()
    c0, c1, c2, c3 = c[..., 0], c[..., 1], c[..., 2], c[..., 3]
    k0, k1 = k[..., 0], k[..., 1]
    for r in range(10):
        if r:
            k0 = (k0 + W0) & MASK
            k1 = (k1 + W1) & MASK
        p0 = c0 * M0
        p1 = c2 * M1
        hi0, lo0 = p0 >> 32, p0 & MASK
        hi1, lo1 = p1 >> 32, p1 & MASK
        c0, c1, c2, c3 = (hi1 ^ c1 ^ k0) & MASK, lo1, (hi0 ^ c3 ^ k1) & MASK, lo0
    return np.stack([c0, c1, c2, c3], axis=-1).astype(np.uint32)


def noise_words(B, V, seed, offset):
    """The uint32 word of element (b, i): Philox with counter
    (i // 4 + offset_lo, offset_hi, b, 0x53414D50) and key (seed_lo, seed_hi),
    word i % 4 -- the layout of lfs_sample_gumbel."""
    i = np.arange(V, dtype=np.uint64)
    b = np.arange(B, dtype=np.uint64)
    lo = (i // 4 + (offset & MASK)) & MASK
    ctr = np.zeros((B, V, 4), np.uint64)
    ctr[..., 0] = lo[None, :]
    ctr[..., 1] = ((offset >> 32) & MASK) + ((i // 4 + (offset & MASK)) >> 32)[None, :]
    ctr[..., 2] = b[:, None]
    ctr[..., 3] = 0x53414D50
    key = np.array([seed & MASK, (seed >> 32) & MASK], np.uint64)
    out = philox4x32_10(ctr, np.broadcast_to(key, (B, V, 2)))
    return out[np.arange(B)[:, None], np.arange(V)[None, :], (i % 4).astype(np.int64)[None, :]]


def exp_noise(words):
    """u = (w + 1) * 2^-32 in (0, 1], e = -log(u) (float64)."""
    u = (np.asarray(words, np.float64) + 1.0) * 2.0 ** -32
    return -np.log(u)


def sample_gumbel(logits, temperatures, noise, dtype=np.float64):
    """utils/sampler.py:46-52: probs = softmax(logits / T); argmax(probs /
    clamp(noise, 1e-10)) per row (first index on ties)."""
    x = np.asarray(logits, dtype) / np.asarray(temperatures, dtype)[:, None]
    x = x - x.max(axis=1, keepdims=True)
    p = np.exp(x)
    p = p / p.sum(axis=1, keepdims=True)
    score = p / np.maximum(np.asarray(noise, dtype), 1e-10)
    return score.argmax(axis=1), score

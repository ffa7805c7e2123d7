"""Pins the sampler oracle (no GPU).

  * philox4x32_10 reproduces the known-answer vectors published with the
    Random123 library (kat_vectors: philox4x32 10 rounds);
  * sample_gumbel equals a scalar brute force of utils/sampler.py:46-52;
  * exp_noise of uniform words has the Exp(1) mean and variance.
"""
import math

import numpy as np

from oracle import sampler as S


def test_philox_known_answers():
    kat = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in kat:
        got = S.philox4x32_10(np.array(ctr, np.uint32), np.array(key, np.uint32))
        assert [int(x) for x in got] == list(want), f"ctr={ctr} key={key}: {[hex(int(x)) for x in got]}"


def test_sample_gumbel_brute_force():
    rng = np.random.default_rng(3)
    B, V = 5, 17
    logits = rng.standard_normal((B, V)) * 3
    temps = np.array([0.5, 1.0, 2.0, 0.7, 1.3])
    noise = rng.exponential(1.0, (B, V))
    noise[0, 3] = 0.0  # clamped to 1e-10
    pick, _ = S.sample_gumbel(logits, temps, noise)
    for b in range(B):
        xs = [logits[b, i] / temps[b] for i in range(V)]
        m = max(xs)
        es = [math.exp(x - m) for x in xs]
        z = sum(es)
        sc = [es[i] / z / max(noise[b, i], 1e-10) for i in range(V)]
        assert pick[b] == max(range(V), key=lambda i: (sc[i], -i))


def test_exp_noise_moments_and_layout():
    w = S.noise_words(4, 50000, seed=123456789, offset=77)
    e = S.exp_noise(w)
    assert abs(e.mean() - 1.0) < 0.01 and abs(e.var() - 1.0) < 0.03
    assert np.all(e >= 0)
    # four consecutive elements share one Philox call; the next offset shifts by one call
    w2 = S.noise_words(4, 50000, seed=123456789, offset=78)
    np.testing.assert_array_equal(w2[:, :-4], w[:, 4:])

"""Pins the CPU oracle of the paged-KV path (no GPU).

  * sdpa reproduces the reference's own golden vectors
    (tests/_snapshots/test_{,4d_}scaled_dot_product_attention.npz there,
    copied into tests/golden/sdpa_snapshots.npz with their seeded inputs);
  * paged_decode equals sdpa on contiguous K/V scattered into a random pool,
    and satisfies L=1 -> v0, constant V -> V, pool-permutation invariance,
    L=0 -> 0, GQA head map h -> h // G;
  * store_kvcache touches exactly the targeted slots; -1 is skipped;
  * decode_slots matches a brute-force enumeration of every position.
"""
from pathlib import Path

import numpy as np

from oracle import paged_kv as P

GOLDEN = Path(__file__).parent / "golden" / "sdpa_snapshots.npz"


def test_sdpa_matches_reference_snapshots():
    g = np.load(GOLDEN)
    out3 = P.sdpa(g["q"], g["k"], g["v"], g["mask"])
    np.testing.assert_allclose(out3, g["expected_3d"], atol=1e-6, rtol=0)
    q4, k4, v4 = (g[n].reshape(2, 2, *g[n].shape[1:]) for n in ("q", "k", "v"))
    m4 = g["mask"].reshape(2, 2, 12, 16)
    np.testing.assert_allclose(P.sdpa(q4, k4, v4, m4), g["expected_4d"], atol=1e-6, rtol=0)


def _random_paged(rng, B, Hq, Hkv, D, BS, NB, lens):
    """Contiguous per-sequence K/V scattered into a pool through random tables."""
    maxb = max(1, max(-(-L // BS) for L in lens))
    perm = rng.permutation(NB)
    bt = np.full((B, maxb), -1, np.int32)
    k_cache = rng.standard_normal((NB, BS, Hkv, D)).astype(np.float32) * 100  # poison
    v_cache = rng.standard_normal((NB, BS, Hkv, D)).astype(np.float32) * 100
    seqs, pos = [], 0
    for b, L in enumerate(lens):
        nb = -(-L // BS)
        bt[b, :nb] = perm[pos:pos + nb]
        pos += nb
        K = rng.standard_normal((L, Hkv, D)).astype(np.float32)
        V = rng.standard_normal((L, Hkv, D)).astype(np.float32)
        slots = np.array([bt[b, t // BS] * BS + t % BS for t in range(L)], np.int64)
        P.store_kvcache(K, V, k_cache, v_cache, slots)
        seqs.append((K, V))
    return k_cache, v_cache, bt, seqs


def test_paged_decode_equals_contiguous_sdpa():
    rng = np.random.default_rng(0)
    B, Hq, Hkv, D, BS, NB = 5, 8, 2, 16, 16, 64
    lens = [1, 17, 32, 50, 0]
    kc, vc, bt, seqs = _random_paged(rng, B, Hq, Hkv, D, BS, NB, lens)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    out = P.paged_decode(q, kc, vc, np.array(lens), bt, scale=0.25)
    G = Hq // Hkv
    for b, (K, V) in enumerate(seqs):
        if lens[b] == 0:
            assert np.all(out[b] == 0)
            continue
        for h in range(Hq):
            ref = P.sdpa(q[b, h][None], K[:, h // G], V[:, h // G], scale=0.25)[0]
            np.testing.assert_allclose(out[b, h], ref, rtol=1e-12, atol=1e-12)
    # L = 1 -> v0 of the matching kv head
    for h in range(Hq):
        np.testing.assert_allclose(out[0, h], seqs[0][1][0, h // G], rtol=1e-12)


def test_paged_decode_invariants():
    rng = np.random.default_rng(1)
    B, Hq, Hkv, D, BS, NB = 3, 4, 4, 8, 16, 32
    lens = [40, 7, 16]
    kc, vc, bt, _ = _random_paged(rng, B, Hq, Hkv, D, BS, NB, lens)
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    base = P.paged_decode(q, kc, vc, np.array(lens), bt, scale=0.3)
    # permuting the pool and remapping the tables changes nothing
    perm = rng.permutation(NB)
    inv = np.argsort(perm)
    bt2 = np.where(bt >= 0, inv[np.maximum(bt, 0)], -1).astype(np.int32)
    got = P.paged_decode(q, kc[perm], vc[perm], np.array(lens), bt2, scale=0.3)
    np.testing.assert_allclose(got, base, rtol=1e-12, atol=1e-12)
    # constant V -> output equals that constant
    vconst = np.full_like(vc, 0.75)
    np.testing.assert_allclose(P.paged_decode(q, kc, vconst, np.array(lens), bt, scale=0.3), 0.75, rtol=1e-12)


def test_store_kvcache_exact_slots():
    rng = np.random.default_rng(2)
    NB, BS, H, D = 8, 16, 2, 8
    kc = rng.integers(0, 2 ** 16, (NB, BS, H, D), dtype=np.uint16)
    vc = rng.integers(0, 2 ** 16, (NB, BS, H, D), dtype=np.uint16)
    k0, v0 = kc.copy(), vc.copy()
    T = 10
    key = rng.integers(0, 2 ** 16, (T, H, D), dtype=np.uint16)
    val = rng.integers(0, 2 ** 16, (T, H, D), dtype=np.uint16)
    slots = rng.choice(NB * BS, T, replace=False).astype(np.int64)
    slots[[2, 7]] = -1
    P.store_kvcache(key, val, kc, vc, slots)
    flat_k, flat_v = kc.reshape(-1, H, D), vc.reshape(-1, H, D)
    touched = set(slots[slots >= 0].tolist())
    for s in range(NB * BS):
        if s in touched:
            t = int(np.where(slots == s)[0][0])
            assert np.array_equal(flat_k[s], key[t]) and np.array_equal(flat_v[s], val[t])
        else:
            assert np.array_equal(flat_k[s], k0.reshape(-1, H, D)[s])
            assert np.array_equal(flat_v[s], v0.reshape(-1, H, D)[s])


def test_decode_slots_brute_force():
    rng = np.random.default_rng(3)
    BS = 4
    lens = [0, 1, 4, 5, 8, 13]
    bt = np.full((len(lens), 4), -1, np.int32)
    perm = rng.permutation(64)
    pos = 0
    for b, L in enumerate(lens):
        nb = -(-L // BS)
        bt[b, :nb] = perm[pos:pos + nb]
        pos += nb
    got = P.decode_slots(bt, lens, BS)
    for b, L in enumerate(lens):
        if L == 0:
            assert got[b] == -1
            continue
        # enumerate every slot of the sequence in order; the newest is the last
        slots = [int(bt[b, j]) * BS + o for j in range(-(-L // BS)) for o in range(BS)][:L]
        assert got[b] == slots[-1]

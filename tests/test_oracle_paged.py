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


def _prefill_batch(rng, lens_q, lens_k, Hq, Hkv, D):
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(lens_k)]).astype(np.int32)
    q = rng.standard_normal((int(cu_q[-1]), Hq, D)).astype(np.float32)
    k = rng.standard_normal((int(cu_k[-1]), Hkv, D)).astype(np.float32)
    v = rng.standard_normal((int(cu_k[-1]), Hkv, D)).astype(np.float32)
    return q, k, v, cu_q, cu_k


def test_prefill_attention_whole_prompt_is_causal_sdpa():
    """lq == lk: per (sequence, head) the reference's causal SDPA (the
    snapshot-pinned sdpa with a lower-triangular mask), GQA map h -> h // G."""
    rng = np.random.default_rng(5)
    Hq, Hkv, D = 8, 2, 16
    lens = [1, 7, 20]
    q, k, v, cu_q, cu_k = _prefill_batch(rng, lens, lens, Hq, Hkv, D)
    out = P.prefill_attention(q, k, v, cu_q, cu_k, scale=0.3)
    G = Hq // Hkv
    for i, L in enumerate(lens):
        s = slice(int(cu_q[i]), int(cu_q[i + 1]))
        for h in range(Hq):
            ref = P.sdpa(q[s, h], k[s, h // G], v[s, h // G], mask=np.tril(np.ones((L, L), bool)), scale=0.3)
            np.testing.assert_allclose(out[s, h], ref, rtol=1e-12, atol=1e-12)


def test_prefill_attention_brute_force_tiny():
    """Scalar loops with math.exp: query p of a sequence attends to keys 0..p."""
    import math
    rng = np.random.default_rng(6)
    Hq, Hkv, D = 4, 2, 3
    lens = [3, 4]
    q, k, v, cu_q, cu_k = _prefill_batch(rng, lens, lens, Hq, Hkv, D)
    out = P.prefill_attention(q, k, v, cu_q, cu_k, scale=0.5)
    for i in range(len(lens)):
        base = int(cu_q[i])
        for p in range(lens[i]):
            for h in range(Hq):
                kv = h // (Hq // Hkv)
                sc = [0.5 * sum(float(q[base + p, h, d]) * float(k[base + t, kv, d]) for d in range(D)) for t in range(p + 1)]
                mx = max(sc)
                w = [math.exp(x - mx) for x in sc]
                ref = [sum(w[t] * float(v[base + t, kv, d]) for t in range(p + 1)) / sum(w) for d in range(D)]
                np.testing.assert_allclose(out[base + p, h], ref, rtol=1e-12, atol=1e-12)


def test_prefill_attention_cached_prefix_and_paged_keys():
    """A cached prefix (lq < lk) gives the last lq rows of the whole prompt's
    result; keys gathered from a randomly permuted pool give the same as the
    contiguous keys."""
    rng = np.random.default_rng(7)
    Hq, Hkv, D, BS, NB = 6, 3, 16, 16, 40
    lens_k = [33, 16, 70]
    lens_q = [5, 16, 1]
    qf, k, v, cu_qf, cu_k = _prefill_batch(rng, lens_k, lens_k, Hq, Hkv, D)
    full = P.prefill_attention(qf, k, v, cu_qf, cu_k, scale=0.25)
    # the last lq query tokens of each prompt
    rows = np.concatenate([np.arange(int(cu_qf[i + 1]) - lq, int(cu_qf[i + 1])) for i, lq in enumerate(lens_q)])
    cu_q = np.concatenate([[0], np.cumsum(lens_q)]).astype(np.int32)
    part = P.prefill_attention(qf[rows], k, v, cu_q, cu_k, scale=0.25)
    np.testing.assert_allclose(part, full[rows], rtol=1e-12, atol=1e-12)
    # same keys in a pool through block tables
    maxb = max(-(-L // BS) for L in lens_k)
    perm = rng.permutation(NB)
    bt = np.full((len(lens_k), maxb), -1, np.int32)
    kc = rng.standard_normal((NB, BS, Hkv, D)) * 100
    vc = rng.standard_normal((NB, BS, Hkv, D)) * 100
    pos = 0
    for i, L in enumerate(lens_k):
        nb = -(-L // BS)
        bt[i, :nb] = perm[pos:pos + nb]
        pos += nb
        slots = np.array([bt[i, t // BS] * BS + t % BS for t in range(L)], np.int64)
        P.store_kvcache(k[int(cu_k[i]):int(cu_k[i + 1])], v[int(cu_k[i]):int(cu_k[i + 1])], kc, vc, slots)
    paged = P.prefill_attention(qf[rows], kc, vc, cu_q, cu_k, scale=0.25, block_tables=bt)
    np.testing.assert_allclose(paged, full[rows], rtol=1e-12, atol=1e-12)

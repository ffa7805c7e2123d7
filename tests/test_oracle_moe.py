"""Pins the MoE dispatch oracle (no GPU).

  * moe_align against a brute force written independently (one pass over
    the entries per expert, sorted by flat index) and its invariants;
  * grouped_gemm against the pinned fp8_gemm oracle (identity rows, one
    expert; gathered rows per tile);
  * moe_combine against scalar loops;
  * segment_reduce_weighted / scatter_add_weighted against a one-hot
    matrix product, and each other on a sorted permutation.
"""
import numpy as np

from oracle import fp8 as F
from oracle import moe as MO


def rand_picks(rng, T, E, k, bad=0):
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.05, 1.0, (T, k)).astype(np.float32)
    for _ in range(bad):
        idx[rng.integers(T), rng.integers(k)] = rng.choice([-1, E, E + 5])
    return idx, w


def test_moe_align_brute_force_and_invariants():
    rng = np.random.default_rng(0)
    for T, E, k, S, bad in [(1, 4, 2, 1, 0), (37, 8, 2, 1, 3), (300, 16, 4, 0, 5), (129, 64, 6, 0, 0)]:
        idx, w = rand_picks(rng, T, E, k, bad)
        rt, rw, te, er = MO.moe_align(idx, w, E, S)
        kk = k + S
        # brute force, written independently: flat entry list, stable sort by expert
        flat = []
        for t in range(T):
            for j in range(kk):
                e = (idx[t, j] if 0 <= idx[t, j] < E else -1) if j < k else E + j - k
                flat.append((e, t * kk + j, t, w[t, j] if j < k else 1.0))
        row = 0
        for e in range(E + S):
            mine = sorted(f for f in flat if f[0] == e)
            for r, (_, i, t, wt) in enumerate(mine):
                assert rt[row + r] == t and rw[row + r] == np.float32(wt) and er.reshape(-1)[i] == row + r
            pad = -(-len(mine) // 128) * 128
            assert np.all(rt[row + len(mine):row + pad] == -1) and np.all(rw[row + len(mine):row + pad] == 0)
            assert np.all(te[row // 128:(row + pad) // 128] == e)
            row += pad
        assert np.all(te[row // 128:] == -1) and np.all(rt[row:] == -1)
        dropped = [i for (e, i, _, _) in flat if e < 0]
        assert np.all(er.reshape(-1)[dropped] == -1)
        kept = er.reshape(-1)[er.reshape(-1) >= 0]
        assert len(np.unique(kept)) == len(kept) == len(flat) - len(dropped)
        assert len(te) == MO.align_tiles(T, k, E, S) and row <= len(te) * 128


def codes(rng, *shape):
    return F.e4m3_encode(rng.standard_normal(shape).astype(np.float32) * 4)


def test_grouped_gemm_reduces_to_fp8_gemm():
    rng = np.random.default_rng(1)
    M, N, K, E = 256, 200, 256, 3
    a, a_s = codes(rng, M, K), rng.uniform(0.01, 1, (M, K // 128)).astype(np.float32)
    b = np.stack([codes(rng, N, K) for _ in range(E)])
    b_s = rng.uniform(0.01, 1, (E, 2, K // 128)).astype(np.float32)
    bias = rng.standard_normal((E, N)).astype(np.float32)
    # identity rows, one expert: the plain GEMM
    got = MO.grouped_gemm(a, a_s, None, np.array([1, 1]), b, b_s, bias)
    np.testing.assert_array_equal(got, F.fp8_gemm(a, a_s, b[1], b_s[1], bias[1]))
    # gathered rows, a tile per expert, an unused tile
    rows = rng.integers(-1, M, 3 * 128).astype(np.int32)
    te = np.array([2, 0, -1])
    got = MO.grouped_gemm(a, a_s, rows, te, b, b_s, round_bf16=False)
    for i, e in enumerate(te):
        blk = got[i * 128:(i + 1) * 128]
        if e < 0:
            assert np.all(np.isnan(blk))
            continue
        src = np.maximum(rows[i * 128:(i + 1) * 128], 0)
        dq = F.e4m3_decode(a[src]).astype(np.float64) * np.repeat(a_s[src], 128, 1)
        dw = F.e4m3_decode(b[e]).astype(np.float64) * np.repeat(np.repeat(b_s[e], 128, 0)[:N], 128, 1)
        np.testing.assert_allclose(blk, dq @ dw.T, rtol=1e-12, atol=1e-9)


def test_moe_combine_scalar_loops():
    rng = np.random.default_rng(2)
    T, E, k, S, d = 9, 5, 2, 1, 16
    idx, w = rand_picks(rng, T, E, k, bad=2)
    rt, rw, te, er = MO.moe_align(idx, w, E, S)
    out = rng.standard_normal((len(rt), d))
    b2 = rng.standard_normal((E + S, d)).astype(np.float32)
    y = MO.moe_combine(out, er, idx, w, E, S, b2)
    for t in range(T):
        acc = np.zeros(d)
        for j in range(k + S):
            e = (idx[t, j] if 0 <= idx[t, j] < E else -1) if j < k else E + j - k
            if e < 0:
                continue
            wt = float(w[t, j]) if j < k else 1.0
            acc += out[er[t, j]] + wt * b2[e].astype(np.float64)
        np.testing.assert_array_equal(y[t], F.bf16_round(acc.astype(np.float32)))


def test_segment_and_scatter_reduce():
    rng = np.random.default_rng(3)
    n, T, d = 200, 40, 24
    x = rng.standard_normal((n, d))
    w = rng.uniform(0, 2, n)
    idx = rng.integers(-2, T + 2, n)
    onehot = np.zeros((T, n))
    for i, t in enumerate(idx):
        if 0 <= t < T:
            onehot[t, i] = w[i]
    want = onehot @ x
    np.testing.assert_allclose(MO.scatter_add_weighted(x, idx, w, T), want, rtol=1e-12, atol=1e-12)
    keep = (idx >= 0) & (idx < T)
    order = np.argsort(idx[keep], kind="stable")
    sx, sw, si = x[keep][order], w[keep][order], idx[keep][order]
    np.testing.assert_allclose(MO.segment_reduce_weighted(sx, sw, si, T), want, rtol=1e-12, atol=1e-12)

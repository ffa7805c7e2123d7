"""Pins the CPU oracle of the FP8 path (no GPU).

Each check is chosen so that a plausible slip in the oracle (wrong rounding,
a dropped clamp, a transposed scale, a wrong constant) fails it:
  * the e4m3fn codec against torch's CPU float8_e4m3fn cast, exhaustively
    over bf16 and over dense fp32 samples incl. every RNE midpoint;
  * the codec against a brute-force nearest-value search;
  * act_quant / weight_quant invariants (max code 448, floor, ue8m0 bounds,
    half-ulp error) and a per-element Python restatement;
  * weight_dequant against torch's fp32 product + bf16 cast;
  * fp8_gemm against the textbook product of the dequantised operands and an
    exact small-integer case.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as F


def torch_e4m3(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


# ------------------------------------------------------------------ codec --
def test_decode_table_matches_torch():
    t = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    both_nan = np.isnan(t) & np.isnan(F.E4M3_VALUES)
    assert np.array_equal(t[~both_nan], F.E4M3_VALUES[~both_nan])
    assert both_nan.sum() == 2  # 0x7F and 0xFF only
    assert F.E4M3_VALUES[0x7E] == 448.0 and F.E4M3_VALUES[0x01] == 2.0 ** -9


def test_encode_all_bf16_in_range_matches_torch():
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    x = bits.view(np.float32)
    x = x[np.isfinite(x) & (np.abs(x) <= 448)]
    assert np.array_equal(F.e4m3_encode(x), torch_e4m3(x))


def test_encode_fp32_samples_and_midpoints_match_torch():
    rng = np.random.default_rng(0)
    x = rng.uniform(-448, 448, 1 << 20).astype(np.float32)
    tiny = (rng.standard_normal(1 << 18) * 2.0 ** -8).astype(np.float32)
    vals = np.unique(np.abs(F.E4M3_VALUES[np.isfinite(F.E4M3_VALUES)]).astype(np.float64))
    mids = ((vals[1:] + vals[:-1]) / 2).astype(np.float32)  # exact in fp32
    near = np.concatenate([mids, np.nextafter(mids, 0), np.nextafter(mids, 1000)])
    allx = np.concatenate([x, tiny, near, -near, np.float32([0.0, -0.0, 448.0, -448.0])])
    assert np.array_equal(F.e4m3_encode(allx), torch_e4m3(allx))


def test_encode_brute_force_nearest():
    """Independent restatement: nearest finite e4m3 value, ties to even code."""
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-448, 448, 2000), rng.standard_normal(2000) * 0.01]).astype(np.float32)
    fin = [c for c in range(256) if np.isfinite(F.E4M3_VALUES[c])]
    got = F.e4m3_encode(x)
    for xi, ci in zip(x.tolist(), got.tolist()):
        best = min(fin, key=lambda c: (abs(float(F.E4M3_VALUES[c]) - xi), c & 1,
                                       (c >> 7) != (1 if np.signbit(np.float32(xi)) else 0)))
        assert F.E4M3_VALUES[best] == F.E4M3_VALUES[ci], (xi, best, ci)
    assert F.e4m3_encode(np.float32([-0.0]))[0] == 0x80
    assert F.e4m3_encode(np.float32([-1e-6]))[0] == 0x80  # rounds to -0


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(1 << 18) * 10).astype(np.float32)
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(F.bf16_round(x), ref)


# -------------------------------------------------------------- act_quant --
def _bf16(a):
    return F.bf16_round(np.asarray(a, np.float32))


def _act_input(M, K, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    idx = rng.choice(M * K, max(1, M * K // 1000), replace=False)
    x.reshape(-1)[idx] = np.where(rng.random(idx.size) < 0.5, -40.0, 40.0)
    x[0, :128] = 0.0            # all-zero group
    x[1, :128] *= 1e-6          # amax below the 1e-4 floor
    return _bf16(x)


def test_act_quant_invariants():
    x = _act_input(64, 512, 3)
    y, s = F.act_quant(x, 128)
    assert y.dtype == np.uint8 and s.shape == (64, 4) and s.dtype == np.float32
    g = x.reshape(64, 4, 128)
    amax = np.abs(g).max(-1)
    floor = np.float32(1e-4) * np.float32(1 / 448)
    assert s[0, 0] == floor and np.all(y[0, :128] == 0)
    assert s[1, 0] == floor
    big = amax >= 1e-4
    maxcode = (y.reshape(64, 4, 128) & 0x7F).max(-1)
    assert np.all(maxcode[big] == 0x7E)
    # |dequant - x/s| <= half an e4m3 ulp at x/s
    q = g / s[..., None]
    d = F.e4m3_decode(y).reshape(g.shape)
    aq = np.abs(q)
    e = np.floor(np.log2(np.maximum(aq, 2.0 ** -6)))
    half_ulp = 2.0 ** (e - 3) / 2
    assert np.all(np.abs(d - q) <= half_ulp * (1 + 1e-6))


def test_act_quant_python_restatement():
    x = _act_input(4, 256, 4)
    y, s = F.act_quant(x, 128)
    for r in range(4):
        for gi in range(2):
            grp = [float(v) for v in x[r, gi * 128:(gi + 1) * 128]]
            amax = max(max(abs(v) for v in grp), float(np.float32(1e-4)))
            sc = np.float32(np.float32(amax) * np.float32(1.0 / 448.0))
            assert s[r, gi] == sc
            for j, v in enumerate(grp):
                qv = float(np.float32(np.float32(v) / sc))
                qv = min(max(qv, -448.0), 448.0)
                assert F.E4M3_VALUES[y[r, gi * 128 + j]] == F.E4M3_VALUES[torch_e4m3(np.float32([qv]))[0]]


def test_act_quant_ue8m0_scales():
    x = _act_input(32, 256, 5)
    _, s = F.act_quant(x, 128, scale_fmt="ue8m0")
    amax = np.maximum(np.abs(x.reshape(32, 2, 128)).max(-1), np.float32(1e-4))
    ref = (amax * np.float32(1 / 448)).astype(np.float32)
    m, _ = np.frexp(s)
    assert np.all(m == 0.5)  # powers of two
    assert np.all(s >= ref) and np.all(s / 2 < ref)


@pytest.mark.parametrize("bs", [32, 64])
def test_act_quant_small_groups(bs):
    x = _act_input(8, 256, 6)
    y, s = F.act_quant(x, bs)
    assert s.shape == (8, 256 // bs)
    for gi in range(256 // bs):
        yy, ss = F.act_quant(x[:, gi * bs:(gi + 1) * bs], bs)
        assert np.array_equal(yy, y[:, gi * bs:(gi + 1) * bs]) and np.array_equal(ss[:, 0], s[:, gi])


def test_act_quant_rejects_ragged():
    with pytest.raises(AssertionError):
        F.act_quant(np.zeros((2, 100), np.float32), 128)


# ------------------------------------------------------ weight quant/deq --
def test_weight_quant_ragged_blocks():
    rng = np.random.default_rng(7)
    w = _bf16(rng.standard_normal((200, 136)) * 0.02)
    y, s = F.weight_quant(w, 128)
    assert s.shape == (2, 2)
    for bi in range(2):
        for bj in range(2):
            blk = w[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            amax = max(float(np.abs(blk).max()), float(np.float32(1e-4)))
            assert s[bi, bj] == np.float32(np.float32(amax) * np.float32(1 / 448))
            yb = y[bi * 128:(bi + 1) * 128, bj * 128:(bj + 1) * 128]
            assert (yb & 0x7F).max() == 0x7E
            ref = torch_e4m3(np.clip((blk / s[bi, bj]).astype(np.float32), -448, 448))
            assert np.array_equal(yb, ref)


def test_weight_dequant_matches_torch():
    rng = np.random.default_rng(8)
    w = _bf16(rng.standard_normal((300, 256)) * 0.02)
    y, s = F.weight_quant(w, 128)
    got = F.weight_dequant(y, s, 128)
    wt = torch.from_numpy(y).view(torch.float8_e4m3fn).float()
    st = torch.from_numpy(s).repeat_interleave(128, 0).repeat_interleave(128, 1)[:300, :256]
    ref = (wt * st).to(torch.bfloat16).float().numpy()
    assert np.array_equal(got, ref)
    # dequant(quant(w)) is within half an e4m3 ulp (<= 16 s = amax/28) of w
    assert np.max(np.abs(got - w)) <= np.abs(w).max() / 28 * 1.01


# --------------------------------------------------------------- fp8_gemm --
def _rand_codes(rng, shape):
    c = rng.integers(0, 256, shape, dtype=np.uint8)
    c[(c & 0x7F) == 0x7F] = 0x00  # no NaN codes
    return c


def test_fp8_gemm_matches_dequantised_product():
    rng = np.random.default_rng(9)
    M, N, K = 33, 200, 384
    a, b = _rand_codes(rng, (M, K)), _rand_codes(rng, (N, K))
    a_s = rng.uniform(0.001, 0.01, (M, K // 128)).astype(np.float32)
    b_s = rng.uniform(0.001, 0.01, (2, K // 128)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    A = F.e4m3_decode(a).astype(np.float64) * np.repeat(a_s, 128, 1)
    B = F.e4m3_decode(b).astype(np.float64) * np.repeat(np.repeat(b_s, 128, 0)[:N], 128, 1)
    ref = A @ B.T + bias
    got64 = F.fp8_gemm(a, a_s, b, b_s, bias)
    got32 = F.fp8_gemm(a, a_s, b, b_s, bias, accum=np.float32)
    assert np.array_equal(got64, F.bf16_round((ref).astype(np.float32)))
    np.testing.assert_allclose(got32, ref, rtol=1e-2, atol=2e-2)


def test_fp8_gemm_exact_small_integers():
    rng = np.random.default_rng(10)
    M, N, K = 40, 70, 256
    ints = np.array([0, 1, 2, 3, 4, 5, 6, 7, 8, -1, -2, -3, -4, -5, -6, -7, -8], np.float32)
    a = F.e4m3_encode(rng.choice(ints, (M, K)))
    b = F.e4m3_encode(rng.choice(ints, (N, K)))
    ones_a = np.ones((M, 2), np.float32)
    ones_b = np.ones((1, 2), np.float32)
    exact = F.e4m3_decode(a).astype(np.int64) @ F.e4m3_decode(b).astype(np.int64).T
    want = F.bf16_round(exact.astype(np.float32))
    assert np.array_equal(F.fp8_gemm(a, ones_a, b, ones_b), want)
    assert np.array_equal(F.fp8_gemm(a, ones_a, b, ones_b, accum=np.float32), want)


def test_fp8_index_brute_force_and_invariants():
    """The indexer score (utils.py:175-227) by scalar loops on a tiny case;
    ReLU zeroes all-negative dot products; the score is linear in q_s and k_s."""
    rng = np.random.default_rng(12)
    B, M, N, H, D = 2, 3, 5, 4, 8
    q = F.e4m3_encode(rng.standard_normal((B, M, H, D)))
    k = F.e4m3_encode(rng.standard_normal((B, N, D)))
    qs = rng.uniform(0.1, 2.0, (B, M, H))
    ks = rng.uniform(0.1, 2.0, (B, N))
    o = F.fp8_index(q, qs, k, ks)
    qd, kd = F.e4m3_decode(q).astype(float), F.e4m3_decode(k).astype(float)
    for b in range(B):
        for m in range(M):
            for n in range(N):
                tot = 0.0
                for h in range(H):
                    dot = sum(qd[b, m, h, d] * kd[b, n, d] for d in range(D))
                    tot += max(dot, 0.0) * qs[b, m, h]
                assert abs(o[b, m, n] - tot * ks[b, n]) <= 1e-12 * max(1.0, abs(tot))
    # all q.k < 0: q = -|x|, k = +|y| elementwise
    qn = F.e4m3_encode(-np.abs(rng.standard_normal((1, 2, 3, 8))) - 0.5)
    kp = F.e4m3_encode(np.abs(rng.standard_normal((1, 4, 8))) + 0.5)
    assert np.all(F.fp8_index(qn, np.ones((1, 2, 3)), kp, np.ones((1, 4))) == 0)
    np.testing.assert_allclose(F.fp8_index(q, 3 * qs, k, ks), 3 * o, rtol=1e-12)
    np.testing.assert_allclose(F.fp8_index(q, qs, k, 0.5 * ks), 0.5 * o, rtol=1e-12)

"""GPU parity of the FP8 kernels against the CPU oracle (through the C ABI).

Bar: act_quant / weight_quant codes and scales and weight_dequant outputs
bit-exact; fp8_gemm within rtol 1e-2 / atol 2e-2 of the float64 oracle on
the same codes and scales (bf16 output, fp32 accumulation), and bit-exact on
small-integer operands with unit scales (every partial sum is an exact fp32
integer, so the order of accumulation cannot matter).
"""
import numpy as np
import pytest
import torch

from llm_from_scratch_amd import kernels as K
from llm_from_scratch_amd import workloads as W
from oracle import fp8 as F

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-2, 2e-2


def codes(t):
    return t.view(torch.uint8).cpu().numpy()


def f32(t):
    return t.float().cpu().numpy()


def check_act_quant(x, block_size=128, scale_fmt=None):
    y, s = K.act_quant(x, block_size, scale_fmt)
    torch.cuda.synchronize()
    ry, rs = F.act_quant(f32(x), block_size, scale_fmt)
    assert y.dtype == torch.float8_e4m3fn and y.shape == x.shape
    assert s.shape == (*x.shape[:-1], x.shape[-1] // block_size)
    np.testing.assert_array_equal(f32(s), rs)
    got = codes(y)
    bad = np.argwhere(got != ry)
    assert bad.size == 0, f"{len(bad)} code mismatches, first at {bad[:3].tolist()}"
    return y, s


# -------------------------------------------------------------- act_quant --
def test_act_quant_cfg1():
    check_act_quant(W.activation(256, 512, seed=0, outliers=False).to(DEV))


@pytest.mark.parametrize("M", [1, 16, 128, 4096])
@pytest.mark.parametrize("Kd", [1024, 4096, 2048])
def test_act_quant_cfg2_outliers(M, Kd):
    check_act_quant(W.activation(M, Kd, seed=1 + M + Kd).to(DEV))


@pytest.mark.parametrize("Kd", [1024, 4096, 2048])
def test_act_quant_m16384_bitexact(Kd):
    """cfg2's largest activations (16384 rows, 0.1% outliers at +-40): codes
    and scales bit-exact against the oracle over every row (the oracle runs
    on row blocks in parallel threads; numpy releases the GIL)."""
    from concurrent.futures import ThreadPoolExecutor
    M = 16384
    x = W.activation(M, Kd, seed=60 + Kd)
    y, s = K.act_quant(x.to(DEV))
    torch.cuda.synchronize()
    xf = f32(x)
    blocks = [(r, min(M, r + 512)) for r in range(0, M, 512)]
    with ThreadPoolExecutor(16) as ex:
        res = list(ex.map(lambda rr: F.act_quant(xf[rr[0]:rr[1]]), blocks))
    ry = np.concatenate([r[0] for r in res])
    rs = np.concatenate([r[1] for r in res])
    np.testing.assert_array_equal(f32(s), rs)
    bad = np.argwhere(codes(y) != ry)
    assert bad.size == 0, f"{len(bad)} code mismatches, first at {bad[:3].tolist()}"


def test_act_quant_every_bf16_quotient():
    """Groups whose amax is 448*2^k have s == 2^k exactly (448*fp32(1/448)
    rounds to 1), so x/s runs over every bf16 value in [-448, 448]: an
    exhaustive check of the divide + e4m3 rounding path incl. ties and
    subnormals."""
    bits = np.arange(1 << 16, dtype=np.uint32) << 16
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals) & (np.abs(vals) <= 448)]
    rows = []
    for k in (0, -3, 5):
        v = vals * np.float32(2.0 ** k)
        n = -(-len(v) // 127)
        v = np.concatenate([v, np.zeros(n * 127 - len(v), np.float32)]).reshape(n, 127)
        grp = np.concatenate([np.full((n, 1), 448 * 2.0 ** k, np.float32), v], axis=1)
        rows.append(grp)
    x = torch.from_numpy(np.concatenate(rows).reshape(-1, 128)).to(torch.bfloat16)
    y, s = check_act_quant(x.to(DEV))
    sc = f32(s).reshape(-1)
    assert set(np.unique(sc).tolist()) == {1.0, 2.0 ** -3, 32.0}


def _every_scale_quotient_groups():
    """Groups of 128 = [amax, 127 others] that reach every fp32 quotient
    x / s act_quant can form with a full-mantissa scale.  s = amax * fp32(1/448)
    depends on amax's 8-bit mantissa only (up to a power of two), and the
    fp32 rounding of x / s on x's mantissa and on the binade only where e4m3
    is subnormal; so one amax per bf16 mantissa (128, spread over exponents),
    each with every bf16 x in [amax * 2^-22, amax] of both signs, covers every
    (scale, element) mantissa pair in every binade from e4m3 subnormals to
    448.  One more amax below the 1e-4 floor takes every bf16 x under it."""
    bits = (np.arange(1 << 16, dtype=np.uint32) << 16).view(np.float32)
    allv = bits[np.isfinite(bits) & (bits != 0)]
    rows = []
    amaxes = [np.float32((1 + m / 128) * 2.0 ** (m % 7 - 3)) for m in range(128)]
    amaxes.append(np.float32(torch.tensor(6.1e-5).to(torch.bfloat16).item()))
    for amax in amaxes:
        lo = amax * np.float32(2.0 ** -22) if amax >= 1e-4 else 0
        v = allv[(np.abs(allv) <= amax) & (np.abs(allv) >= lo)]
        n = -(-len(v) // 127)
        v = np.concatenate([v, np.zeros(n * 127 - len(v), np.float32)]).reshape(n, 127)
        rows.append(np.concatenate([np.full((n, 1), amax, np.float32), v], axis=1))
    return np.concatenate(rows)


def test_act_quant_every_scale_quotient():
    """Codes for quotients x / s with full-mantissa scales, which act_quant
    forms as x times the group's reciprocal with an IEEE-divide fallback near
    e4m3 rounding midpoints: every (scale mantissa, element mantissa, binade)
    case, bit-exact against the oracle's correctly rounded divide."""
    g = _every_scale_quotient_groups()
    assert len(np.unique(g[:, 0].view(np.uint32) & 0x7F0000)) == 128
    pad = -len(g) % 4
    g = np.concatenate([g, np.zeros((pad, 128), np.float32)])
    x = torch.from_numpy(g.reshape(-1, 512)).to(torch.bfloat16)
    assert torch.equal(x.float().reshape(-1, 128), torch.from_numpy(g))
    check_act_quant(x.to(DEV))


def test_act_quant_edge_groups():
    x = torch.randn(8, 256).to(torch.bfloat16)
    x[0, :128] = 0.0
    x[1, :128] = -0.0
    x[2, :128] *= 1e-7                     # below the 1e-4 amax floor
    x[3, :128] = torch.tensor(-1e-40)      # bf16 subnormal, negative
    x[4, 5] = 3.0e38                       # huge amax, everything else -> +-0
    x[5, :] = 448.0
    x[6, :] = -1.0
    check_act_quant(x.to(DEV))


@pytest.mark.parametrize("bs", [32, 64, 128])
def test_act_quant_block_sizes_and_ue8m0(bs):
    x = W.activation(64, 512, seed=11).to(DEV)
    check_act_quant(x, bs)
    check_act_quant(x, bs, "ue8m0")


def test_act_quant_batched_shape_and_asserts():
    x = W.activation(6, 384, seed=12).reshape(2, 3, 384).to(DEV)
    check_act_quant(x)
    with pytest.raises(AssertionError, match="contiguous"):
        K.act_quant(x.transpose(0, 1))
    with pytest.raises(AssertionError, match="divisible"):
        K.act_quant(W.activation(2, 200, seed=1).to(DEV))
    y, s = K.act_quant(torch.empty(0, 256, dtype=torch.bfloat16, device=DEV))
    assert y.shape == (0, 256) and s.shape == (0, 2)


# ---------------------------------------------------- weight quant/dequant --
@pytest.mark.parametrize("shape", [(1344, 512), (200, 136), (4096, 1024), (72, 8)])
def test_weight_quant_bitexact(shape):
    w = W.weight(*shape, seed=13).to(DEV)
    y, s = K.weight_quant(w)
    torch.cuda.synchronize()
    ry, rs = F.weight_quant(f32(w))
    np.testing.assert_array_equal(f32(s), rs)
    np.testing.assert_array_equal(codes(y), ry)


@pytest.mark.parametrize("shape", [(1344, 512), (200, 136), (5632, 2048)])
def test_weight_dequant_bitexact(shape):
    w = W.weight(*shape, seed=14).to(DEV)
    y, s = K.weight_quant(w)
    d = K.weight_dequant(y, s)
    torch.cuda.synchronize()
    ref = F.weight_dequant(codes(y), f32(s))
    np.testing.assert_array_equal(f32(d), ref)
    # and against torch's own fp32 product + bf16 cast of the same operands
    st = s.repeat_interleave(128, 0).repeat_interleave(128, 1)[: shape[0], : shape[1]]
    np.testing.assert_array_equal(f32(d), f32((y.float() * st).to(torch.bfloat16)))


# ---------------------------------------------------------------- fp8_gemm --
def gemm_oracle(a, a_s, b, b_s, bias=None, rows=None):
    an, asn = codes(a), f32(a_s)
    bn = None if bias is None else f32(bias)
    if rows is not None:
        an, asn = an[rows], asn[rows]
        if bn is not None and bn.ndim == 2:
            bn = bn[rows]
    return F.fp8_gemm(an, asn, codes(b), f32(b_s), bn)


def assert_close(got, ref, what=""):
    err = np.abs(got - ref)
    tol = ATOL + RTOL * np.abs(ref)
    bad = np.argwhere(err > tol)
    assert bad.size == 0, f"{what}: {len(bad)} mismatches, worst {err.max():.4g}, first {bad[:3].tolist()}"


def test_fp8_linear_cfg1():
    """cfg1: quantise x (1x128) and W (128x128) on the GPU, GEMM, compare."""
    x = W.activation(256, 512, seed=0, outliers=False).to(DEV)
    w = W.weight(1344, 512, seed=100).to(DEV)
    xq, xs = check_act_quant(x)
    wq, ws = K.weight_quant(w)
    c = K.fp8_gemm(xq, xs, wq, ws)
    torch.cuda.synchronize()
    assert c.shape == (256, 1344) and c.dtype == torch.bfloat16
    assert_close(f32(c), gemm_oracle(xq, xs, wq, ws), "cfg1")
    # the FP8 linear approximates the bf16 one
    ref = (x.float() @ w.float().T).cpu().numpy()
    assert np.abs(f32(c) - ref).max() < 0.1 * np.abs(ref).max()


def test_fp8_gemm_exact_small_integers():
    rng = np.random.default_rng(20)
    M, N, Kd = 256, 320, 512
    ints = np.arange(-8, 9, dtype=np.float32)
    a = torch.from_numpy(F.e4m3_encode(rng.choice(ints, (M, Kd)))).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(F.e4m3_encode(rng.choice(ints, (N, Kd)))).view(torch.float8_e4m3fn).to(DEV)
    a_s = torch.ones(M, Kd // 128, device=DEV)
    b_s = torch.ones(-(-N // 128), Kd // 128, device=DEV)
    c = K.fp8_gemm(a, a_s, b, b_s)
    exact = F.e4m3_decode(codes(a)).astype(np.int64) @ F.e4m3_decode(codes(b)).astype(np.int64).T
    np.testing.assert_array_equal(f32(c), F.bf16_round(exact.astype(np.float32)))


def test_fp8_gemm_random_codes_and_scales():
    """Every byte pattern but NaN, distinct scale per (row, k-block) and per
    (128-col block, k-block): catches a transposed or shifted scale index."""
    rng = np.random.default_rng(21)
    M, N, Kd = 300, 400, 640
    ac = rng.integers(0, 256, (M, Kd), dtype=np.uint8)
    bc = rng.integers(0, 256, (N, Kd), dtype=np.uint8)
    ac[(ac & 0x7F) == 0x7F] = 0
    bc[(bc & 0x7F) == 0x7F] = 0
    a = torch.from_numpy(ac).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(bc).view(torch.float8_e4m3fn).to(DEV)
    a_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (M, Kd // 128)).astype(np.float32)).to(DEV)
    b_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (-(-N // 128), Kd // 128)).astype(np.float32)).to(DEV)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(DEV)
    assert_close(f32(K.fp8_gemm(a, a_s, b, b_s)), gemm_oracle(a, a_s, b, b_s), "nobias")
    assert_close(f32(K.fp8_gemm(a, a_s, b, b_s, bias)), gemm_oracle(a, a_s, b, b_s, bias), "bias")
    # per-row bias matrix, given as a strided view: a distinct value per (m, n)
    # catches a bias indexed by column only or with the wrong row stride
    bm = torch.from_numpy(rng.standard_normal((M, N + 24)).astype(np.float32)).to(DEV)[:, 5:5 + N]
    assert_close(f32(K.fp8_gemm(a, a_s, b, b_s, bm)), gemm_oracle(a, a_s, b, b_s, bm), "bias matrix")


@pytest.mark.parametrize("splits", [2, 3, 5, 7])
def test_fp8_gemm_split_k(splits):
    """K split over workgroups (fp32 partials + reduction): same oracle,
    ragged M/N, a K count that does not divide evenly, bias vector and
    per-row bias matrix."""
    rng = np.random.default_rng(40 + splits)
    M, N, Kd = 300, 400, 640
    ac = rng.integers(0, 256, (M, Kd), dtype=np.uint8)
    bc = rng.integers(0, 256, (N, Kd), dtype=np.uint8)
    ac[(ac & 0x7F) == 0x7F] = 0
    bc[(bc & 0x7F) == 0x7F] = 0
    a = torch.from_numpy(ac).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(bc).view(torch.float8_e4m3fn).to(DEV)
    a_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (M, Kd // 128)).astype(np.float32)).to(DEV)
    b_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (-(-N // 128), Kd // 128)).astype(np.float32)).to(DEV)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(DEV)
    bm = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(DEV)
    for bb, what in ((None, "nobias"), (bias, "bias"), (bm, "bias matrix")):
        got = K.fp8_gemm(a, a_s, b, b_s, bb, splits=splits)
        assert_close(f32(got), gemm_oracle(a, a_s, b, b_s, bb), f"splits={splits} {what}")
        one = K.fp8_gemm(a, a_s, b, b_s, bb, splits=1)
        assert np.abs(f32(got) - f32(one)).max() <= 2e-2 + 1e-2 * np.abs(f32(one)).max()


def _random_codes(rng, M, N, Kd):
    """Every e4m3 byte pattern but NaN, distinct scales per block."""
    ac = rng.integers(0, 256, (M, Kd), dtype=np.uint8)
    bc = rng.integers(0, 256, (N, Kd), dtype=np.uint8)
    ac[(ac & 0x7F) == 0x7F] = 0
    bc[(bc & 0x7F) == 0x7F] = 0
    a = torch.from_numpy(ac).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(bc).view(torch.float8_e4m3fn).to(DEV)
    a_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (M, Kd // 128)).astype(np.float32)).to(DEV)
    b_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (-(-N // 128), Kd // 128)).astype(np.float32)).to(DEV)
    return a, a_s, b, b_s


@pytest.mark.parametrize("M,N,Kd,variant", [(17, 250, 384, "r32c16"), (33, 96, 1024, "r32c16"),
                                            (128, 1280, 768, "r32c16"), (128, 31, 512, "r32c16"),
                                            (100, 4096, 768, "r32c32"), (128, 4090, 1024, "r32c32"),
                                            (128, 9216, 768, "r128c48"), (100, 8200, 256, "r128c48"),
                                            (128, 14000, 512, "r128c64"), (70, 12290, 768, "r128c64"),
                                            (128, 1024, 4096, "r16c16"), (40, 1000, 1536, "r16c16"),
                                            (128, 1536, 1536, None), (128, 768, 4608, None)])
def test_fp8_gemm_flat(M, N, Kd, variant):
    """The one-shot decode kernel (16 < M <= 128: every operand byte of a
    workgroup copied to LDS in one burst) in each of its geometries --
    32 x 16 and 32 x 32 (row x column) workgroups for K <= 1024, 128 x 48
    and 128 x 64 for wide N at K <= 768 (48 columns straddle the weights'
    128-row scale blocks), 16 x 16 for K <= 4096 -- and as split-K partials
    of 8 K blocks with the reduction (variant None: K = 1536 in 2 splits,
    the cfg5 down projection's K = 4608 in 5): ragged M and N (not
    multiples of 16, 32, 64 or 4), 2 to 36 K blocks, bias vector and per-row
    bias matrix, against the oracle."""
    assert K.flat_gemm_variant(M, N, Kd) == variant
    if variant is None:
        splits = K.default_gemm_splits(M, N, Kd)
        assert splits > 1 and K.flat_gemm_variant(M, N, Kd, kps=-(-(Kd // 128) // splits)) == "s32c32"
    rng = np.random.default_rng(M * 5 + N + Kd)
    a, a_s, b, b_s = _random_codes(rng, M, N, Kd)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(DEV)
    bm = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(DEV)
    for bb, what in ((None, "nobias"), (bias, "bias"), (bm, "bias matrix")):
        got = K.fp8_gemm(a, a_s, b, b_s, bb)
        assert_close(f32(got), gemm_oracle(a, a_s, b, b_s, bb), f"flat {M}x{N}x{Kd} {what}")


@pytest.mark.parametrize("M,N,Kd,variant", [(17, 250, 384, "r32c16"), (128, 768, 768, "r32c16"),
                                            (100, 4096, 768, "r32c32"), (128, 9216, 768, "r128c48"),
                                            (70, 12290, 768, "r128c64"), (40, 1000, 1536, "r16c16"),
                                            (128, 1024, 4096, "r16c16")])
def test_fp8_gemm_act_equals_act_quant_then_gemm(M, N, Kd, variant):
    """fp8_gemm_act (the act_quant of bf16 rows done inside the one-shot
    GEMM's workgroups) against act_quant followed by fp8_gemm in one split,
    bit for bit, in each one-shot geometry: ragged M (rows past M read the
    last row and are dropped), strided rows, outliers that set a group's
    scale, an all-zero group, bias vector or none; and the oracle's bar on
    the result.  FP8Linear.forward takes this path on these shapes."""
    assert K.flat_gemm_variant(M, N, Kd) == variant and K.fp8_gemm_act_supported(M, N, Kd)
    rng = np.random.default_rng(M * 7 + N + Kd)
    g = torch.Generator(device=DEV).manual_seed(M + N)
    wide = torch.randn(M, Kd + 64, generator=g, device=DEV).to(torch.bfloat16)
    wide[0, :128] = 0                      # one all-zero group
    wide[M // 2, 5] = 300.0                # an outlier sets its group's scale
    x = wide[:, :Kd]                       # rows with stride Kd + 64
    _, _, b, b_s = _random_codes(rng, M, N, Kd)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(DEV)
    print(f"fp8_gemm_act {M}x{N}x{Kd} {variant}", flush=True)
    for bb in (None, bias):
        got = K.fp8_gemm_act(x, b, b_s, bb)
        xq, xs = K.act_quant(x.contiguous(), 128)
        ref = K.fp8_gemm(xq, xs, b, b_s, bb, splits=1)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"{M}x{N}x{Kd} bias={bb is not None}"
        assert_close(f32(got), gemm_oracle(xq, xs, b, b_s, bb), f"fp8_gemm_act {M}x{N}x{Kd}")


def test_fp8_gemm_act_rejects_other_shapes():
    """Shapes outside the one-shot tilings (M <= 16, M > 128, long K) and a
    misaligned row stride are refused."""
    b = torch.zeros(256, 256, device=DEV, dtype=torch.float8_e4m3fn)
    b_s = torch.ones(2, 2, device=DEV)
    for M in (8, 200):
        assert not K.fp8_gemm_act_supported(M, 256, 256)
        with pytest.raises(ValueError, match="no one-shot tiling"):
            K.fp8_gemm_act(torch.zeros(M, 256, device=DEV, dtype=torch.bfloat16), b, b_s)
    x = torch.zeros(64, 260, device=DEV, dtype=torch.bfloat16)[:, 2:258]
    with pytest.raises(ValueError, match="row stride|aligned"):
        K.fp8_gemm_act(x, b, b_s)


@pytest.mark.parametrize("M,N,Kd", [(1, 768, 768), (5, 1282, 128), (16, 1280, 768), (13, 31, 512),
                                    (1, 1024, 4096), (7, 5632, 2048), (16, 96, 1536), (3, 250, 3072),
                                    (1, 200, 3200), (16, 96, 16384), (16, 1024, 4608), (9, 4096, 1024),
                                    (16, 4097, 2048), (2, 24, 256)])
def test_fp8_gemm_skinny(M, N, Kd):
    """The decode-batch kernel for M <= 16 (K blocks split over the waves of
    a workgroup: four, or 8 / 16 for 12 / 24+ K blocks; 16-column groups for
    N <= 4096, 32 otherwise): every byte pattern but NaN, distinct scales,
    ragged M and N (N not a multiple of 16, 32 or 4), 1 to 128 K blocks
    (fewer than and not a multiple of the waves; K = 16384 the longest K the
    dispatch sends here, (16, 1024, 4608) the cfg5 down projection at 16
    sequences), N on both sides of the 4096 column-group switch, bias vector
    and per-row bias matrix; against the oracle and the 128 x 128 tile
    kernel."""
    assert K.use_skinny_gemm(M, N, Kd)
    rng = np.random.default_rng(M * 7 + N + Kd)
    ac = rng.integers(0, 256, (M, Kd), dtype=np.uint8)
    bc = rng.integers(0, 256, (N, Kd), dtype=np.uint8)
    ac[(ac & 0x7F) == 0x7F] = 0
    bc[(bc & 0x7F) == 0x7F] = 0
    a = torch.from_numpy(ac).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(bc).view(torch.float8_e4m3fn).to(DEV)
    a_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (M, Kd // 128)).astype(np.float32)).to(DEV)
    b_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (-(-N // 128), Kd // 128)).astype(np.float32)).to(DEV)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(DEV)
    bm = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(DEV)
    for bb, what in ((None, "nobias"), (bias, "bias"), (bm, "bias matrix")):
        got = K.fp8_gemm(a, a_s, b, b_s, bb)
        assert_close(f32(got), gemm_oracle(a, a_s, b, b_s, bb), f"skinny {M}x{N}x{Kd} {what}")
        tile = K.fp8_gemm(a, a_s, b, b_s, bb, splits=1)
        assert np.abs(f32(got) - f32(tile)).max() <= 2e-2 + 1e-2 * np.abs(f32(tile)).max()


def test_fp8_gemm_skinny_exact_small_integers():
    """Small-integer codes with unit scales: every partial sum is an exact
    fp32 integer, so the wave-split sum is bit-exact in any order (the
    skinny kernel at M = 16, the one-shot kernel at M = 100)."""
    for M, N, Kd in ((16, 200, 1024), (100, 200, 1024)):
        _exact_small_integers(M, N, Kd)


def _exact_small_integers(M, N, Kd):
    rng = np.random.default_rng(22 + M)
    assert K.use_skinny_gemm(M, N, Kd) or K.flat_gemm_variant(M, N, Kd) is not None
    ints = np.arange(-8, 9, dtype=np.float32)
    a = torch.from_numpy(F.e4m3_encode(rng.choice(ints, (M, Kd)))).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(F.e4m3_encode(rng.choice(ints, (N, Kd)))).view(torch.float8_e4m3fn).to(DEV)
    a_s = torch.ones(M, Kd // 128, device=DEV)
    b_s = torch.ones(-(-N // 128), Kd // 128, device=DEV)
    c = K.fp8_gemm(a, a_s, b, b_s)
    exact = F.e4m3_decode(codes(a)).astype(np.int64) @ F.e4m3_decode(codes(b)).astype(np.int64).T
    np.testing.assert_array_equal(f32(c), F.bf16_round(exact.astype(np.float32)))


@pytest.mark.parametrize("M,N,Kd", [(4000, 4042, 1152), (4096, 4040, 640)])
def test_fp8_gemm_big_tiles_ragged(M, N, Kd):
    """Shapes with 256 tiles of 256x256 (the one-workgroup-per-CU kernel):
    partial last row and column tiles, N not a multiple of 8 (element-wise
    stores), 9 and 5 K blocks (a partial second scale chunk, a single
    partial chunk), bias vector and per-row bias matrix; sampled rows
    include both sides of every tile boundary near the edges."""
    rng = np.random.default_rng(M + N + Kd)
    ac = rng.integers(0, 256, (M, Kd), dtype=np.uint8)
    bc = rng.integers(0, 256, (N, Kd), dtype=np.uint8)
    ac[(ac & 0x7F) == 0x7F] = 0
    bc[(bc & 0x7F) == 0x7F] = 0
    a = torch.from_numpy(ac).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(bc).view(torch.float8_e4m3fn).to(DEV)
    a_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (M, Kd // 128)).astype(np.float32)).to(DEV)
    b_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (-(-N // 128), Kd // 128)).astype(np.float32)).to(DEV)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(DEV)
    bm = torch.from_numpy(rng.standard_normal((M, N)).astype(np.float32)).to(DEV)
    edge = [0, 1, 127, 128, 255, 256, 3839, 3840, M - 2, M - 1]
    rows = np.unique(np.concatenate([edge, rng.choice(M, 100, replace=False)]))
    for bb, what in ((None, "nobias"), (bias, "bias"), (bm, "bias matrix")):
        got = f32(K.fp8_gemm(a, a_s, b, b_s, bb))[rows]
        assert_close(got, gemm_oracle(a, a_s, b, b_s, bb, rows=rows), f"{M}x{N}x{Kd} {what}")


@pytest.mark.parametrize("M,N,Kd", [(8000, 2304, 1152), (4000, 4096, 256), (16384, 1024, 640)])
def test_fp8_gemm_persistent_tiles(M, N, Kd):
    """Shapes the persistent 256x256 kernel takes (N a multiple of 256, at
    least half a round of tiles): more tiles than workgroups, so a workgroup
    runs several tiles and copies each next tile's first K block during the
    last one (8000 x 2304: 288 tiles; 16384 x 1024: 256 tiles, one each);
    ragged M (the last row tile is partial and its stores fall outside the
    buffer range); 9, 2 and 5 K blocks (partial scale chunks, a single
    block past the first); vector bias.  Sampled rows include both sides of
    the tile boundaries near the edges."""
    rng = np.random.default_rng(M + N + Kd)
    ac = rng.integers(0, 256, (M, Kd), dtype=np.uint8)
    bc = rng.integers(0, 256, (N, Kd), dtype=np.uint8)
    ac[(ac & 0x7F) == 0x7F] = 0
    bc[(bc & 0x7F) == 0x7F] = 0
    a = torch.from_numpy(ac).view(torch.float8_e4m3fn).to(DEV)
    b = torch.from_numpy(bc).view(torch.float8_e4m3fn).to(DEV)
    a_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (M, Kd // 128)).astype(np.float32)).to(DEV)
    b_s = torch.from_numpy(rng.uniform(1e-3, 1e-2, (N // 128, Kd // 128)).astype(np.float32)).to(DEV)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(DEV)
    edge = [0, 1, 255, 256, 511, 512, M - 257, M - 256, M - 2, M - 1]
    rows = np.unique(np.concatenate([edge, rng.choice(M, 100, replace=False)]))
    for bb, what in ((None, "nobias"), (bias, "bias")):
        c = K.fp8_gemm(a, a_s, b, b_s, bb)
        torch.cuda.synchronize()
        assert_close(f32(c)[rows], gemm_oracle(a, a_s, b, b_s, bb, rows=rows), f"{M}x{N}x{Kd} {what}")
        # every element against the 128x128 tile kernel (split-K path, same
        # per-block products and folds: the same fp32 sums up to the order
        # of the split partials)
        ref = f32(K.fp8_gemm(a, a_s, b, b_s, bb, splits=2))
        assert np.isfinite(f32(c)).all()
        err = np.abs(f32(c) - ref)
        assert (err <= ATOL + RTOL * np.abs(ref)).all(), f"{what}: persistent vs split-K max err {err.max()}"


@pytest.mark.parametrize("M", [1, 16, 128, 4096])
@pytest.mark.parametrize("KN", W.GEMM_KN)
def test_fp8_gemm_cfg2_shapes(M, KN):
    Kd, N = KN
    x = W.activation(M, Kd, seed=30 + M).to(DEV)
    w = W.weight(N, Kd, seed=31).to(DEV)
    xq, xs = K.act_quant(x)
    wq, ws = K.weight_quant(w)
    c = K.fp8_gemm(xq, xs, wq, ws)
    torch.cuda.synchronize()
    rows = None if M <= 128 else np.random.default_rng(M).choice(M, 192, replace=False)
    ref = gemm_oracle(xq, xs, wq, ws, rows=rows)
    got = f32(c) if rows is None else f32(c)[rows]
    assert_close(got, ref, f"M={M} K={Kd} N={N}")


def test_fp8_gemm_persistent_half_tail_bit_identical():
    """A last round of at most half a round of 256x256 tiles runs as a second
    launch of 256 x 128 halves (four waves each).  M = 4096, N = 5632, K =
    2048: 352 tiles, the last 96 as 192 halves; the same rows of an M = 16384
    product (1408 tiles; those rows there in whole tiles of the first
    rounds) must be bit-identical, every byte pattern of e4m3 but NaN, with a
    bias vector; and the halves' rows against the oracle."""
    rng = np.random.default_rng(77)
    Kd, N = 2048, 5632
    a, a_s, b, b_s = _random_codes(rng, 16384, N, Kd)
    bias = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(DEV)
    print("half tail: M 4096 / 16384, K 2048, N 5632", flush=True)
    small = K.fp8_gemm(a[:4096].contiguous(), a_s[:4096].contiguous(), b, b_s, bias)
    big = K.fp8_gemm(a, a_s, b, b_s, bias)
    torch.cuda.synchronize()
    assert torch.equal(small.view(torch.int16), big[:4096].view(torch.int16)), "half tiles differ from whole tiles"
    rows = np.array([2048, 2300, 3071, 3072, 3500, 4095])  # rows of tail tiles
    assert_close(f32(small)[rows], gemm_oracle(a, a_s, b, b_s, bias, rows=rows), "half tail")


@pytest.mark.parametrize("KN", W.GEMM_KN)
def test_fp8_gemm_m16384_sampled_rows(KN):
    """The three cfg2 headline shapes at M = 16384 (the bench's launches):
    sampled rows against the oracle, and the whole output finite and within
    tolerance of the split-K 128x128 tile kernel on the same codes."""
    Kd, N = KN
    x = W.activation(16384, Kd, seed=40 + Kd).to(DEV)
    w = W.weight(N, Kd, seed=41).to(DEV)
    xq, xs = K.act_quant(x)
    wq, ws = K.weight_quant(w)
    c = K.fp8_gemm(xq, xs, wq, ws)
    torch.cuda.synchronize()
    rows = np.concatenate([[0, 255, 256, 16383], np.random.default_rng(3).choice(16384, 124, replace=False)])
    assert_close(f32(c)[rows], gemm_oracle(xq, xs, wq, ws, rows=rows), f"M=16384 K={Kd} N={N}")
    ref = f32(K.fp8_gemm(xq, xs, wq, ws, splits=2))
    got = f32(c)
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert (err <= ATOL + RTOL * np.abs(ref)).all(), f"vs split-K: max err {err.max()}"

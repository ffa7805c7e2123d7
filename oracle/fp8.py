"""CPU restatement of the block-wise FP8 path (numpy).  TEST INFRASTRUCTURE.

Arrays that hold bf16 data are carried as float32 arrays whose values are
exactly bf16-representable (``bf16_round`` produces them); FP8 codes are
uint8 arrays holding OCP ``float8_e4m3fn`` bit patterns.

Reference semantics (``/root/reference/model/attention/utils.py``):
  * group amax, clamped below at 1e-4 .................. :129-131
  * scale = amax * fp32(1/448)  (fp8_max_inv) .......... :101-104, :135
  * ue8m0 scale = 2**ceil(log2(amax * (1/448))) ........ :81-94, :133
  * y = e4m3fn(clamp(x / s, -448, 448)) (IEEE divide) .. :136-139
  * act_quant(x, block_size, scale_fmt) shapes ......... :148-172

Pinning (what checks each function, see tests/test_oracle_fp8.py):
  e4m3_encode   -- exhaustive against torch's CPU float8_e4m3fn cast over
                   every bf16 value in [-448, 448] and over 2^24 fp32 values;
                   decode(encode(decode(c))) == decode(c) for all 256 codes.
  act_quant     -- invariants: max |code| == 448 per group with amax >= 1e-4,
                   all-zero group -> s = fp32(1e-4)*fp32(1/448), codes 0;
                   ue8m0 scales are powers of two with s/2 < amax/448 <= s;
                   dequant error <= half an e4m3 ulp; brute-force per-element
                   python-float restatement on small inputs.
  weight_quant  -- same invariants over 128x128 blocks incl. ragged tails.
  weight_dequant-- bit-exact vs torch (fp32 product, RNE to bf16).
  fp8_gemm      -- float64 dequant(A) @ dequant(B)^T (textbook), exact on
                   small-integer codes with unit scales.
  fp8_index     -- scalar brute force on tiny inputs; all-negative dot
                   products give 0 (ReLU); linear in q_s and in k_s.
"""
from __future__ import annotations

import numpy as np

FP8_MAX = np.float32(448.0)
# The reference keeps 1/448 as a Python float and multiplies an fp32 amax by
# it inside the kernel (utils.py:101, :135): the constant is fp32(1/448).
FP8_MAX_INV = np.float32(1.0 / 448.0)
AMAX_FLOOR = np.float32(1e-4)  # utils.py:131


# ---------------------------------------------------------------------------
# bf16 helpers
# ---------------------------------------------------------------------------
def bf16_round(x) -> np.ndarray:
    """Round float32 values to the nearest bf16 (ties to even); returns float32.

    NaN stays NaN.  This is the rounding torch's ``.to(torch.bfloat16)`` does.
    """
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    b = x.view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) >> 16 << 16
    out = (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), x, out)


def bf16_bits(x) -> np.ndarray:
    """uint16 bit patterns of bf16-valued float32 data."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def bf16_from_bits(b) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


# ---------------------------------------------------------------------------
# OCP float8_e4m3fn codec (1 sign, 4 exponent bits with bias 7, 3 mantissa
# bits, no infinities, 0x7F/0xFF are NaN, max finite 448, subnormals m*2^-9)
# ---------------------------------------------------------------------------
def _e4m3_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            t[c] = np.nan
        elif e == 0:
            t[c] = s * m * 2.0 ** -9
        else:
            t[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


E4M3_VALUES = _e4m3_table()


def e4m3_decode(codes) -> np.ndarray:
    return E4M3_VALUES[np.asarray(codes, dtype=np.uint8)]


def e4m3_encode(x) -> np.ndarray:
    """float32 -> e4m3fn code, round-to-nearest-even.

    Finite inputs with |x| beyond the largest finite value are saturated to
    +-448 only if they round below 464 (the RNE midpoint between 448 and the
    NaN slot); callers clamp to +-448 first as the reference does, so that
    case never arises on the hot path.  NaN -> 0x7F | sign.
    """
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    bits = x.view(np.uint32)
    sign = ((bits >> 31) & 1).astype(np.uint8) << 7
    a = np.abs(x)
    ab = a.view(np.uint32).astype(np.int64)
    # normal range of e4m3 (|x| >= 2^-6): round the fp32 mantissa at bit 20
    rb = ab + 0x7FFFF + ((ab >> 20) & 1)
    exp = (rb >> 23) - 127 + 7
    man = (rb >> 20) & 0x7
    normal_code = (exp << 3) | man
    # subnormal range (|x| < 2^-6): code = RNE(|x| * 2^9) (exact scaling)
    sub_code = np.rint(a.astype(np.float64) * 512.0).astype(np.int64)
    code = np.where(a < np.float32(2.0 ** -6), sub_code, normal_code)
    # finite overflow: anything rounding past 448 becomes NaN (0x7F)
    code = np.where(code > 0x7E, 0x7F, code)
    code = np.where(np.isnan(x), 0x7F, code)
    return (code.astype(np.uint8) | sign).astype(np.uint8)


# ---------------------------------------------------------------------------
# scales
# ---------------------------------------------------------------------------
def scale_from_amax(amax, round_scale: bool = False) -> np.ndarray:
    """utils.py:129-135: clamp amax at 1e-4, then amax*fp32(1/448).

    round_scale (ue8m0, utils.py:81-94): 2^(exponent + (mantissa != 0)) of
    amax*(1/448), i.e. the smallest power of two >= that product.
    """
    amax = np.maximum(np.asarray(amax, dtype=np.float32), AMAX_FLOOR)
    s = (amax * FP8_MAX_INV).astype(np.float32)
    if round_scale:
        b = np.ascontiguousarray(s).view(np.uint32).astype(np.int64)
        e = ((b >> 23) & 0xFF) - 127 + ((b & 0x7FFFFF) != 0).astype(np.int64)
        s = ((e + 127) << 23).astype(np.uint32).view(np.float32)
    return s


def quantize_with_scale(x, s) -> np.ndarray:
    """utils.py:136-139: e4m3fn(clamp(x / s, -448, 448)), fp32 IEEE divide."""
    q = (np.asarray(x, dtype=np.float32) / np.asarray(s, dtype=np.float32)).astype(np.float32)
    q = np.clip(q, -FP8_MAX, FP8_MAX)  # NaN propagates, as T.clamp does
    return e4m3_encode(q)


# ---------------------------------------------------------------------------
# act_quant: 1 x block_size groups along the last dimension
# ---------------------------------------------------------------------------
def act_quant(x, block_size: int = 128, scale_fmt=None):
    """Restates ``act_quant`` (model/attention/utils.py:148-172) and its kernel
    (:97-145).  x: float32 array of bf16 values, last dim % block_size == 0.

    Returns (codes uint8 same shape as x, scales float32 [..., K/block_size]).
    Unlike the reference wrapper (which forwards no block size, :170-171,
    while its kernel hard-codes 128, :107) the group width here is
    ``block_size``.
    """
    x = np.asarray(x, dtype=np.float32)
    K = x.shape[-1]
    assert K % block_size == 0, f"Last dimension size must be divisible by block_size (block_size={block_size})"
    g = x.reshape(*x.shape[:-1], K // block_size, block_size)
    amax = np.abs(g).max(axis=-1) if g.size else np.zeros(g.shape[:-1], np.float32)
    s = scale_from_amax(amax, round_scale=scale_fmt is not None)
    y = quantize_with_scale(g, s[..., None]).reshape(x.shape)
    return y, s.astype(np.float32)


# ---------------------------------------------------------------------------
# 128 x 128 weight-block quantisation (not in the reference; defined by the
# per-(128x128) block scales, same scale formula as above)
# ---------------------------------------------------------------------------
def weight_quant(w, block_size: int = 128):
    """w: float32 [N, K] of bf16 values -> (codes uint8 [N,K],
    scales float32 [ceil(N/bs), ceil(K/bs)]).  Ragged tail blocks take their
    amax over their valid elements only."""
    w = np.asarray(w, dtype=np.float32)
    N, K = w.shape
    nb, kb = -(-N // block_size), -(-K // block_size)
    pad = np.zeros((nb * block_size, kb * block_size), np.float32)
    pad[:N, :K] = np.abs(w)
    amax = pad.reshape(nb, block_size, kb, block_size).max(axis=(1, 3))
    s = scale_from_amax(amax)
    s_full = np.repeat(np.repeat(s, block_size, 0), block_size, 1)[:N, :K]
    return quantize_with_scale(w, s_full), s.astype(np.float32)


def weight_dequant(codes, s, block_size: int = 128) -> np.ndarray:
    """bf16_RNE(fp32(code) * s[n // bs, k // bs]) -> float32 of bf16 values."""
    codes = np.asarray(codes, dtype=np.uint8)
    N, K = codes.shape
    s_full = np.repeat(np.repeat(np.asarray(s, np.float32), block_size, 0), block_size, 1)[:N, :K]
    return bf16_round((e4m3_decode(codes) * s_full).astype(np.float32))


# ---------------------------------------------------------------------------
# block-scaled FP8 GEMM: C[m, n] = sum_kb a_s[m,kb] b_s[n//128,kb] A_kb . B_kb
# ---------------------------------------------------------------------------
def fp8_gemm(a, a_s, b, b_s, bias=None, block_size: int = 128, accum=np.float64,
             round_bf16: bool = True) -> np.ndarray:
    """a: uint8 [M,K] codes, a_s float32 [M, K/bs]; b: uint8 [N,K] codes,
    b_s float32 [ceil(N/bs), K/bs].  Returns bf16 values (as float32) of
    ``sum_kb (a_s*b_s) * (A_kb @ B_kb^T) (+ bias)``.

    accum=np.float64: the textbook product of the dequantised operands (the
    parity oracle).  accum=np.float32: one fp32 matmul per K block with the
    scale product applied to the partial in an fp32 accumulator -- the same
    structure as the GPU kernel, used as the timed CPU baseline.
    round_bf16=False returns the unrounded sum (in ``accum``).
    """
    a = np.asarray(a, np.uint8)
    b = np.asarray(b, np.uint8)
    M, K = a.shape
    N = b.shape[0]
    assert K % block_size == 0
    kb = K // block_size
    A = e4m3_decode(a).astype(accum).reshape(M, kb, block_size)
    B = e4m3_decode(b).astype(accum).reshape(N, kb, block_size)
    bs_rows = np.repeat(np.asarray(b_s, np.float32), block_size, 0)[:N]  # [N, kb]
    acc = np.zeros((M, N), dtype=accum)
    for j in range(kb):
        part = A[:, j, :] @ B[:, j, :].T
        sc = np.asarray(a_s, np.float32)[:, j:j + 1].astype(accum) * bs_rows[None, :, j].astype(accum)
        if accum is np.float32:
            sc = sc.astype(np.float32)
        acc += part * sc
    if bias is not None:
        bias = np.asarray(bias, dtype=accum)
        acc = acc + (bias[None, :] if bias.ndim == 1 else bias)
    if not round_bf16:
        return acc
    return bf16_round(acc.astype(np.float32))


def fp8_index(q, q_s, k, k_s, accum=np.float64) -> np.ndarray:
    """o[b, m, n] = k_s[b, n] * sum_h relu(q[b, m, h] . k[b, n]) * q_s[b, m, h]
    (the indexer score of model/attention/utils.py:175-227: fp8 q.k per head,
    ReLU, head weights, head sum, key scale).  q: codes [B, M, H, D], q_s
    [B, M, H]; k: codes [B, N, D], k_s [B, N].  Returns float [B, M, N]."""
    qd = e4m3_decode(np.asarray(q)).astype(accum)
    kd = e4m3_decode(np.asarray(k)).astype(accum)
    logits = np.einsum("bmhd,bnd->bmhn", qd, kd)
    w = np.maximum(logits, 0) * np.asarray(q_s, accum)[..., None]
    return w.sum(axis=2) * np.asarray(k_s, accum)[:, None, :]

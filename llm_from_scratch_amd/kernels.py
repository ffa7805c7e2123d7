"""Operator surface of the block-wise FP8 and paged-KV path, on gfx950 kernels.

Same names, arguments and return values as the reference's operators:
  act_quant(x, block_size=128, scale_fmt=None) -> (y, s)
      model/attention/utils.py:148-172 (asserts kept word for word)
  weight_quant(x, block_size=128) -> (y, s)      128x128 block scales
  weight_dequant(x, s, block_size=128) -> y      bf16
  fp8_gemm(a, a_s, b, b_s, bias=None) -> c       bf16, fp32 accumulation
  store_kvcache(key, value, k_cache, v_cache, slot_mapping)
      KV slot write with the slot contract of engine/model_runner.py:226-230,
      :261, :303 (-1 = skip)
  paged_attention_decode(q, k_cache, v_cache, context_lens, block_tables,
                         scale=None) -> o
      GQA decode over block tables, math of model/attention/GQA.py:118-130
  flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                         max_seqlen_k, softmax_scale=None, causal=True,
                         block_table=None) -> o
      varlen causal prefill attention, the call engine/model_runner.py:291-292
      names
  sample_gumbel(logits, temperatures, seed, offset) -> tokens
      temperature + Gumbel-max sampling, utils/sampler.py:35-53
  fp8_index(q, q_s, k, k_s) -> index_score
      the DSA indexer score, model/attention/utils.py:175-250

Every call goes through the C ABI of liblfs_kernels.so on torch's current
stream; outputs are allocated here, as the reference wrappers do
(utils.py:168-169).  There is no CPU path: tensors must live on a GPU.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

from . import _lib

FP8 = torch.float8_e4m3fn


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _on_gpu(*ts: torch.Tensor) -> None:
    dev = ts[0].device
    for t in ts:
        if t.device.type != "cuda":
            raise ValueError(f"tensor on {t.device}: the FP8/paged-KV kernels run on the GPU only")
        if t.device != dev:
            raise ValueError(f"tensors on different devices: {t.device} vs {dev}")


def _dtype(t: torch.Tensor, dt: torch.dtype, name: str) -> None:
    if t.dtype != dt:
        raise TypeError(f"{name} must be {dt}, got {t.dtype}")


# ----------------------------------------------------------------- FP8 path --
def act_quant(x: torch.Tensor, block_size: int = 128, scale_fmt: Optional[str] = None
              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Block-wise activation quantisation (model/attention/utils.py:148-172).

    Per row, per ``block_size`` consecutive elements of the last dimension:
    s = max(amax, 1e-4) * fp32(1/448) (``scale_fmt`` set: rounded up to a
    power of two, the ue8m0 form), y = e4m3fn(clamp(x / s, -448, 448)).
    Returns (y float8_e4m3fn like x, s float32 [..., N // block_size]).
    ``block_size`` is honoured (32, 64 or 128), unlike the reference wrapper,
    whose kernel always used 128.
    """
    assert x.is_contiguous(), "Input tensor must be contiguous"
    assert x.size(-1) % block_size == 0, (
        f"Last dimension size must be divisible by block_size (block_size={block_size})"
    )
    _on_gpu(x)
    _dtype(x, torch.bfloat16, "x")
    N = x.size(-1)
    y = torch.empty_like(x, dtype=FP8)
    s = x.new_empty(*x.size()[:-1], N // block_size, dtype=torch.float32)
    M = x.numel() // N if N else 0
    rc = _lib.load().lfs_act_quant(_ptr(x), N, _ptr(y), _ptr(s), M, N, block_size,
                                   int(scale_fmt is not None), _stream(x))
    _lib.check(rc, "act_quant")
    return y, s


def weight_quant(x: torch.Tensor, block_size: int = 128) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-(block_size x block_size) quantisation of a [N, K] weight.

    Same scale formula as act_quant over 2-D blocks; ragged tail blocks use
    their valid elements.  Returns (y float8_e4m3fn [N, K],
    s float32 [ceil(N/bs), ceil(K/bs)]).
    """
    assert x.is_contiguous(), "Input tensor must be contiguous"
    assert x.dim() == 2, "Input tensor must have 2 dimensions"
    _on_gpu(x)
    _dtype(x, torch.bfloat16, "x")
    N, K = x.shape
    y = torch.empty_like(x, dtype=FP8)
    s = x.new_empty(math.ceil(N / block_size), math.ceil(K / block_size), dtype=torch.float32)
    rc = _lib.load().lfs_weight_quant(_ptr(x), _ptr(y), _ptr(s), N, K, block_size, _stream(x))
    _lib.check(rc, "weight_quant")
    return y, s


def weight_dequant(x: torch.Tensor, s: torch.Tensor, block_size: int = 128) -> torch.Tensor:
    """y = bf16(fp32(x) * s[n // bs, k // bs]) for a block-quantised weight."""
    assert x.is_contiguous() and s.is_contiguous(), "Input tensors must be contiguous"
    assert x.dim() == 2 and s.dim() == 2, "Input tensors must have 2 dimensions"
    _on_gpu(x, s)
    _dtype(x, FP8, "x")
    _dtype(s, torch.float32, "s")
    N, K = x.shape
    assert s.shape == (math.ceil(N / block_size), math.ceil(K / block_size)), "scale shape mismatch"
    y = torch.empty_like(x, dtype=torch.bfloat16)
    rc = _lib.load().lfs_weight_dequant(_ptr(x), _ptr(s), _ptr(y), N, K, block_size, _stream(x))
    _lib.check(rc, "weight_dequant")
    return y


def flat_gemm_variant(M: int, N: int, K: int, kps: Optional[int] = None) -> Optional[str]:
    """The one-shot GEMM fp8_gemm runs for 16 < M <= 128 (None: another
    kernel).  The same rule as flat_variant in csrc/fp8_gemm.hip: unsplit
    (``kps`` None) K <= 1024 with <= 512 workgroups of 32 rows x 16 (else 32)
    columns, K <= 768 with <= 256 workgroups of 128 x 48 (else 128 x 64), K
    <= 4096 with <= 512 workgroups of 16 x 16; split-K partials of at most 8
    K blocks each in <= 1024 workgroups of 32 x 32 ("s32c32")."""
    if M <= 16 or M > 128:
        return None
    kb = K // 128
    r32, c16, c32 = -(-M // 32), -(-N // 16), -(-N // 32)
    if kps is not None:
        return "s32c32" if kps <= 8 and r32 * c32 * -(-kb // kps) <= 1024 else None
    if kb <= 8 and r32 * c16 <= 512:
        return "r32c16"
    if kb <= 8 and r32 * c32 <= 512:
        return "r32c32"
    if kb <= 6 and -(-N // 48) <= 256:
        return "r128c48"
    if kb <= 6 and -(-N // 64) <= 256:
        return "r128c64"
    if kb <= 32 and -(-M // 16) * c16 <= 512:
        return "r16c16"
    return None


def default_gemm_splits(M: int, N: int, K: int) -> int:
    """K splits for fp8_gemm.  For 16 < M <= 128: 1 when the one-shot
    kernel covers the whole K (flat_gemm_variant), else blocks of 8 K blocks
    when its split partials fit (M = 128, K = 4608, N = 768: 5 splits, 6.3 us
    against 11.5 us for 6 tile-kernel splits).  Otherwise 1 when the 128x128
    output tiles alone give >= 192 workgroups or K has fewer than 12 blocks
    of 128.  Below that grid each tile-kernel workgroup already runs two K
    slices, and a call takes about 6.5 us plus 1.1 us per K block of a slice
    (measured back to back on MI355X at M = 128-512, K 2048 / 4096, N
    1536-8192), so splitting pays where it shortens long slices by more than
    the fp32 partials and their reduction cost: with >= 24 K blocks, max(4,
    K blocks / 6) splits (K = 4096: 16-22 % faster than unsplit at 12-64
    tiles); with 12-23 K blocks only for <= 16 tiles (4 splits, 15.4 -> 14.0
    us at M = 128, K = 2048, N = 1536), since from 24 tiles up the unsplit
    call is the fastest (N = 5632: 15.9 us against 18.2 at 2 splits).  At
    most ~256 workgroups and 32 MB of partials (M = 128, K = 4096, N = 8192:
    4 splits 22.0 us, unsplit 25.9)."""
    kt = K // 128
    if flat_gemm_variant(M, N, K) is not None:
        return 1
    if kt > 8 and flat_gemm_variant(M, N, K, kps=8) is not None:
        return -(-kt // 8)
    tiles = -(-M // 128) * -(-N // 128)
    if tiles >= 192 or kt < 12:
        return 1
    if kt >= 24:
        splits = max(4, kt // 6)
    elif tiles <= 16:
        splits = min(4, kt // 4)
    else:
        return 1
    splits = min(splits, max(1, 256 // tiles), max(1, (32 << 20) // max(1, 4 * M * N)))
    return max(1, splits)


SKINNY_MAX_M = 128  # the skinny kernel's row limit


def use_skinny_gemm(M: int, N: int, K: int) -> bool:
    """M <= 16 with K <= 16384 runs the skinny kernel: one 16-row tile, the
    K blocks split over 8 or 16 waves, and re-reading A costs little (M = 1,
    K = 4096, N = 1024: 5.0 us; split-K tiles 15-16 us).  Larger decode
    shapes (16 < M <= 128) run the one-shot kernel of flat_gemm_variant when
    it applies, which measured faster than the skinny kernel on every cfg5
    and cfg2 shape at M = 128 (the output projection, N 768 / K 768: 4.3
    against 6.6 us)."""
    return 0 < M <= 16 and K <= 16384


def fp8_gemm(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
             bias: Optional[torch.Tensor] = None, splits: Optional[int] = None) -> torch.Tensor:
    """c = a @ b^T with 1x128 activation scales and 128x128 weight scales.

    a: e4m3fn [..., K], a_s: fp32 [..., K/128]; b: e4m3fn [N, K] (nn.Linear
    weight layout), b_s: fp32 [ceil(N/128), K/128]; bias: None, fp32 [N], or
    an fp32 per-row bias matrix [..., N] (rows with unit stride in N).
    The scale products are applied to each 128-wide K-block partial in an
    fp32 accumulator, the bias is added in fp32, and the result is rounded
    once to bf16 [..., N].  ``splits`` > 1 splits the K blocks over that many
    workgroups per output tile (fp32 partials, then one reduction).  By
    default M <= 16 with K <= 16384 runs the skinny kernel (the K blocks
    split across the waves of one workgroup per 16 or 32 output columns),
    16 < M <= 128 the one-shot kernel where flat_gemm_variant applies (every
    operand byte of a workgroup copied to LDS in one burst), other shapes
    that cannot fill the GPU are split, and the rest run the tile kernels.
    """
    assert a.is_contiguous() and b.is_contiguous(), "Input tensors must be contiguous"
    assert a_s.is_contiguous() and b_s.is_contiguous(), "Scaling factor tensors must be contiguous"
    _on_gpu(a, a_s, b, b_s)
    _dtype(a, FP8, "a")
    _dtype(b, FP8, "b")
    _dtype(a_s, torch.float32, "a_s")
    _dtype(b_s, torch.float32, "b_s")
    K = a.size(-1)
    M = a.numel() // K if K else 0
    N = b.size(0)
    assert b.dim() == 2 and b.size(1) == K, "b must be [N, K]"
    assert K % 128 == 0, "K must be a multiple of 128"
    assert a_s.shape == (*a.shape[:-1], K // 128), "a_s must be [..., K/128]"
    assert b_s.shape == (math.ceil(N / 128), K // 128), "b_s must be [ceil(N/128), K/128]"
    bias_ld = 0
    if bias is not None:
        _on_gpu(a, bias)
        _dtype(bias, torch.float32, "bias")
        if bias.dim() == 1:
            assert bias.is_contiguous() and bias.shape == (N,), "bias must be fp32 [N]"
        else:
            bias = bias.reshape(-1, bias.size(-1)) if bias.dim() > 2 else bias
            assert bias.shape == (M, N) and bias.stride(1) == 1, "bias matrix must be fp32 [..., N]"
            bias_ld = bias.stride(0) if M > 1 else N
    c = a.new_empty(*a.shape[:-1], N, dtype=torch.bfloat16)
    L = _lib.load()
    if splits is None and use_skinny_gemm(M, N, K):
        rc = L.lfs_fp8_gemm_skinny(_ptr(a), _ptr(a_s), _ptr(b), _ptr(b_s), _ptr(bias), bias_ld, _ptr(c), M, N, K,
                                   _stream(a))
        _lib.check(rc, "fp8_gemm")
        return c
    if splits is None:
        splits = default_gemm_splits(M, N, K)
    need = int(L.lfs_fp8_gemm_workspace_bytes(M, N, K, splits)) if splits > 1 else 0
    if need:
        ws = torch.empty(need // 4, dtype=torch.float32, device=a.device)
        rc = L.lfs_fp8_gemm_splitk(_ptr(a), _ptr(a_s), _ptr(b), _ptr(b_s), _ptr(bias), bias_ld, _ptr(c),
                                   M, N, K, splits, _ptr(ws), need, _stream(a))
    else:
        rc = L.lfs_fp8_gemm(_ptr(a), _ptr(a_s), _ptr(b), _ptr(b_s), _ptr(bias), bias_ld, _ptr(c),
                            M, N, K, _stream(a))
    _lib.check(rc, "fp8_gemm")
    return c


def fp8_gemm_act_supported(M: int, N: int, K: int) -> bool:
    """Whether fp8_gemm_act takes the shape: the one-shot tilings of
    fp8_gemm (16 < M <= 128, small K and N)."""
    return bool(_lib.load().lfs_fp8_gemm_act_supported(M, N, K))


def fp8_gemm_act(x: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
                 bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp8_gemm(*act_quant(x, 128), b, b_s, bias, splits=1) in one launch,
    bit for bit: the act_quant codes and scales of x are computed inside the
    GEMM's workgroups.  x: bf16 [..., K] (rows may be strided, K contiguous);
    only the shapes fp8_gemm_act_supported accepts."""
    assert x.stride(-1) == 1, "x must be contiguous along K"
    _on_gpu(x, b, b_s)
    _dtype(x, torch.bfloat16, "x")
    _dtype(b, FP8, "b")
    _dtype(b_s, torch.float32, "b_s")
    K = x.size(-1)
    x2 = x.reshape(-1, K)
    M, N = x2.size(0), b.size(0)
    assert b.dim() == 2 and b.size(1) == K and b.is_contiguous(), "b must be contiguous [N, K]"
    assert b_s.shape == (math.ceil(N / 128), K // 128) and b_s.is_contiguous(), "b_s must be [ceil(N/128), K/128]"
    if bias is not None:
        _dtype(bias, torch.float32, "bias")
        assert bias.is_contiguous() and bias.shape == (N,), "bias must be fp32 [N]"
    c = x.new_empty(*x.shape[:-1], N, dtype=torch.bfloat16)
    rc = _lib.load().lfs_fp8_gemm_act(_ptr(x2), x2.stride(0), _ptr(b), _ptr(b_s), _ptr(bias), 0, _ptr(c), M, N, K,
                                      _stream(x))
    _lib.check(rc, "fp8_gemm_act")
    return c


# ------------------------------------------------------------- paged KV path --
def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """k_cache.view(-1, Hkv, D)[slot_mapping[t]] = key[t] for slot != -1.

    key/value: bf16 [T, Hkv, D] (heads and dims contiguous, any token stride);
    caches: bf16 [num_blocks, block_size, Hkv, D] contiguous; slot_mapping:
    int64 [T].  Slots outside the pool are skipped like -1.
    """
    N, num_heads, head_dim = key.shape
    D = num_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.is_contiguous() and v_cache.is_contiguous()
    assert k_cache.dim() == 4 and k_cache.shape[2:] == (num_heads, head_dim)
    assert v_cache.shape == k_cache.shape and value.shape == key.shape
    assert slot_mapping.numel() == N and slot_mapping.is_contiguous()
    _on_gpu(key, value, k_cache, v_cache, slot_mapping)
    for t, n in ((key, "key"), (value, "value"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _dtype(t, torch.bfloat16, n)
    _dtype(slot_mapping, torch.int64, "slot_mapping")
    num_slots = k_cache.shape[0] * k_cache.shape[1]
    rc = _lib.load().lfs_store_kvcache(_ptr(key), key.stride(0), _ptr(value), value.stride(0),
                                       _ptr(k_cache), _ptr(v_cache), _ptr(slot_mapping), N,
                                       num_heads, head_dim, num_slots, _stream(key))
    _lib.check(rc, "store_kvcache")


BALANCED_MAX_BATCH = 8192  # the balanced split scans the batch's tile counts in LDS


PAIRS_MAX_CONTEXT = 8192  # longest table (tokens) the single-launch decode is the default for
PAIR_MAX_BATCH = 256  # the paired order ranks the batch in one workgroup


def _cu_count() -> int:
    if torch.cuda.is_available():
        return torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    return 256


def default_blocks_per_split(batch: int, num_kv_heads: int, max_blocks: int, block_size: int,
                             cus: Optional[int] = None, quant_values: int = 0) -> int:
    """Split of the decode context (shapes only, so the choice is capturable).

    -2 selects the single launch in the paired order: one workgroup per
    (sequence, kv head), the sequences ranked by context length inside the
    kernel so that each CU runs a long and a short one at once (the
    workgroups w and w + CUs of a grid of at most two per CU share a CU).
    It is the default when B * Hkv is more than one and at most two
    workgroups per CU, B <= 256, the table holds at most PAIRS_MAX_CONTEXT
    tokens and a quantised output (quant_values = G * D, 0 for none) has
    whole 128-value groups per kv head.  Measured on MI355X at the cfg5
    attention shape (B 128, GQA 12/4, D 64, contexts U[256, 2048]): 36.4 us
    kernel time against 43.5 us for one workgroup per pair of kv heads.

    -1 selects the single launch: one workgroup per (sequence, pair of kv
    heads), whose waves walk interleaved tiles and merge through LDS (no
    second launch, no workspace).  A workgroup streams at most ~30 GB/s, so
    it is the default only when Hkv is even, the B * Hkv / 2 workgroups
    cover every CU (at most four rounds) and the table holds at most
    PAIRS_MAX_CONTEXT tokens.  Measured on MI355X at the cfg5 attention
    shape (B 128, GQA 12/4, D 64, act_quant fused): contexts U[256, 2048]
    46.1 against 47.5 us balanced, all 2048 tokens 54.8 against 60.3 us; at
    B 64 the balanced split wins (35.1 against 42.9 us).

    0 selects the balanced split: a fixed grid of one 4-wave workgroup per
    CU, each taking an equal share of the (sequence, kv-head group, tile)
    work, whatever the context lengths, then a merge launch.  Measured on
    MI355X: cfg4 (B 256, lengths log-uniform to 32k) 1169 us against 1523 us
    for the best fixed chunking; cfg3 44.3 us against 49.7 us.

    Above BALANCED_MAX_BATCH sequences, fixed chunks of the returned number
    of blocks, one wave per (sequence, kv head, chunk): with fewer than 1024
    (sequence, kv head) pairs 512-token chunks (cfg3: 49 us against 66 us at
    256 tokens); with more, chunks grow until the grid has at most 32768
    potential waves (cfg4: 2000 / 1826 / 1683 / 1634 us at 1 / 2 / 4 / 8
    blocks per chunk)."""
    cus = _cu_count() if cus is None else cus
    units = batch * num_kv_heads
    if (batch <= PAIR_MAX_BATCH and cus < units <= 2 * cus and quant_values % 128 == 0
            and max_blocks * block_size <= PAIRS_MAX_CONTEXT):
        return -2
    groups = batch * num_kv_heads // 2
    if (num_kv_heads % 2 == 0 and cus <= groups <= 4 * cus
            and max_blocks * block_size <= PAIRS_MAX_CONTEXT):
        return -1
    if batch <= BALANCED_MAX_BATCH:
        return 0
    base = max(1, 256 // max(block_size, 1))
    pairs = batch * num_kv_heads
    if pairs < 1024:
        bps = 2 * base
    else:
        bps = base
        while pairs * -(-max_blocks // bps) > 32768 and bps < max_blocks:
            bps *= 2
    return max(1, min(bps, max(max_blocks, 1)))


def paged_decode_workspace_bytes(batch: int, num_q_heads: int, head_dim: int, max_blocks: int,
                                 blocks_per_split: int) -> int:
    return int(_lib.load().lfs_paged_decode_workspace_bytes(batch, num_q_heads, head_dim,
                                                            max_blocks, blocks_per_split))


def paged_attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           context_lens: torch.Tensor, block_tables: torch.Tensor,
                           scale: Optional[float] = None, blocks_per_split: Optional[int] = None,
                           workspace: Optional[torch.Tensor] = None, quant: bool = False):
    """One decode step of GQA attention over a paged KV pool.

    q: bf16 [B, Hq, D]; caches bf16 [num_blocks, block_size, Hkv, D];
    context_lens int64 [B] (0 = padding row, output zeros); block_tables
    int32 [B, max_blocks] padded with -1.  scale defaults to 1/sqrt(D) as
    SDPA (model/attention/GQA.py:130).  Returns bf16 [B, Hq, D].
    ``blocks_per_split`` -1 runs one launch with a workgroup per (sequence,
    kv-head pair), -2 one launch with a workgroup per (sequence, kv head) in
    the paired order, 0 shares the context tiles evenly over a fixed grid, n > 0
    splits every context into chunks of n blocks (default_blocks_per_split
    picks one from the shapes).  Either way the grid depends only on the
    shapes, so the call can be captured in a HIP graph (pass a
    preallocated ``workspace`` of ``paged_decode_workspace_bytes`` bytes to
    keep the capture free of allocations).  With ``quant`` the merge also quantises each output row
    for the next FP8 linear and the call returns (o, codes e4m3fn
    [B, Hq*D], scales fp32 [B, Hq*D/128]), the codes equal to
    act_quant(o.view(B, -1)) bit for bit.
    """
    assert q.dim() == 3 and q.is_contiguous(), "q must be contiguous [B, Hq, D]"
    assert k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.shape == v_cache.shape
    assert k_cache.dim() == 4, "caches must be [num_blocks, block_size, Hkv, D]"
    assert block_tables.dim() == 2 and block_tables.stride(1) == 1, "block_tables must be [B, max_blocks]"
    assert context_lens.is_contiguous() and context_lens.numel() == q.size(0)
    _on_gpu(q, k_cache, v_cache, context_lens, block_tables)
    for t, n in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _dtype(t, torch.bfloat16, n)
    _dtype(context_lens, torch.int64, "context_lens")
    _dtype(block_tables, torch.int32, "block_tables")
    B, Hq, D = q.shape
    NB, BS, Hkv, Dk = k_cache.shape
    assert Dk == D, "head_dim mismatch between q and the caches"
    assert block_tables.size(0) == B
    max_blocks = block_tables.size(1)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if blocks_per_split is None:
        bps = default_blocks_per_split(B, Hkv, max_blocks, BS, quant_values=(Hq // Hkv) * D if quant else 0)
    else:
        bps = blocks_per_split
    need = paged_decode_workspace_bytes(B, Hq, D, max_blocks, bps)
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=q.device)
    o = torch.empty_like(q)
    oq = os_ = None
    if quant:
        oq = torch.empty(B, Hq * D, dtype=FP8, device=q.device)
        os_ = torch.empty(B, Hq * D // 128, dtype=torch.float32, device=q.device)
    rc = _lib.load().lfs_paged_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(context_lens),
                                      _ptr(block_tables), block_tables.stride(0), _ptr(o),
                                      _ptr(workspace), workspace.numel() * workspace.element_size(),
                                      B, Hq, Hkv, D, BS, NB, max_blocks, float(scale), bps,
                                      _ptr(oq), _ptr(os_), _stream(q))
    _lib.check(rc, "paged_attention_decode")
    return (o, oq, os_) if quant else o


def paged_attention_decode_rope(qkv: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                                cos_sin: torch.Tensor, positions: torch.Tensor, num_q_heads: int,
                                num_kv_heads: int, eps: float, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                slot_mapping: Optional[torch.Tensor], context_lens: torch.Tensor,
                                block_tables: torch.Tensor, scale: Optional[float] = None, quant: bool = False,
                                q_rot: Optional[torch.Tensor] = None):
    """qk_norm_rope_store then paged_attention_decode(blocks_per_split=-1)
    for one new token per sequence, in one launch (lfs_paged_decode_rope).

    qkv: bf16 [B, (Hq + 2 Hkv) * D] (rows may be strided), the fused QKV
    projection of each sequence's newest token; its q and k are normalised
    and rotated with qk_norm_rope_store's arithmetic (same bits), its k and v
    written to the caches at slot_mapping (None: no write).  The attention
    covers context_lens[b] tokens, the newest from the row itself.  Returns
    what paged_attention_decode returns (with ``quant`` the output's FP8
    codes and scales too); ``q_rot`` (bf16 [B, Hq, D]) optionally receives
    the rotated q.  Results equal the unfused pair up to fp32 summation
    order.  use_fused_decode_rope says whether a shape is supported."""
    assert qkv.dim() == 2 and qkv.stride(1) == 1
    B = qkv.size(0)
    D = cos_sin.size(1)
    Hq, Hkv = num_q_heads, num_kv_heads
    assert qkv.size(1) == (Hq + 2 * Hkv) * D, "qkv width mismatch"
    assert k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.shape == v_cache.shape
    assert k_cache.dim() == 4 and k_cache.shape[2:] == (Hkv, D), "caches must be [NB, BS, Hkv, D]"
    assert block_tables.dim() == 2 and block_tables.stride(1) == 1 and block_tables.size(0) == B
    assert context_lens.is_contiguous() and context_lens.numel() == B
    _on_gpu(qkv, q_weight, k_weight, cos_sin, positions, k_cache, v_cache, context_lens, block_tables)
    _dtype(qkv, torch.bfloat16, "qkv")
    for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        _dtype(t, torch.bfloat16, n)
    for t, n in ((q_weight, "q_weight"), (k_weight, "k_weight"), (cos_sin, "cos_sin")):
        _dtype(t, torch.float32, n)
        assert t.is_contiguous(), f"{n} must be contiguous"
    assert q_weight.numel() == Hq * D and k_weight.numel() == Hkv * D
    _dtype(positions, torch.int64, "positions")
    _dtype(context_lens, torch.int64, "context_lens")
    _dtype(block_tables, torch.int32, "block_tables")
    if slot_mapping is not None:
        _on_gpu(slot_mapping)
        _dtype(slot_mapping, torch.int64, "slot_mapping")
        assert slot_mapping.numel() == B and slot_mapping.is_contiguous()
    NB, BS = k_cache.shape[:2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    o = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=qkv.device)
    oq = os_ = None
    if quant:
        oq = torch.empty(B, Hq * D, dtype=FP8, device=qkv.device)
        os_ = torch.empty(B, Hq * D // 128, dtype=torch.float32, device=qkv.device)
    if q_rot is not None:
        assert q_rot.shape == (B, Hq, D) and q_rot.dtype == torch.bfloat16 and q_rot.is_contiguous()
    rc = _lib.load().lfs_paged_decode_rope(
        _ptr(qkv), qkv.stride(0), _ptr(q_weight), _ptr(k_weight), _ptr(cos_sin), cos_sin.size(0),
        _ptr(positions), _ptr(slot_mapping), float(eps), _ptr(q_rot), _ptr(k_cache), _ptr(v_cache),
        _ptr(context_lens), _ptr(block_tables), block_tables.stride(0), _ptr(o), B, Hq, Hkv, D, BS, NB,
        block_tables.size(1), float(scale), _ptr(oq), _ptr(os_), _stream(qkv))
    _lib.check(rc, "paged_attention_decode_rope")
    return (o, oq, os_) if quant else o


def decode_rope_paired(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, max_blocks: int,
                       block_size: int) -> bool:
    """Whether paged_attention_decode_rope without the quantised output
    runs the paired order (blocks_per_split -2): the rule
    lfs_paged_decode_rope applies when q_out is NULL."""
    return (use_fused_decode_rope(batch, num_q_heads, num_kv_heads, head_dim, max_blocks, block_size, quant=False)
            and default_blocks_per_split(batch, num_kv_heads, max_blocks, block_size) == -2)


def use_fused_decode_rope(batch: int, num_q_heads: int, num_kv_heads: int, head_dim: int, max_blocks: int,
                          block_size: int, quant: bool = True) -> bool:
    """Whether the decode step runs paged_attention_decode_rope: when the
    default split is a single launch (default_blocks_per_split -1 or -2)
    and the shape fits the fused prologue ((Hq + Hkv) * D / 16 <= 256; with
    the quantised output an even Hkv or G * D % 128 == 0)."""
    G = num_q_heads // num_kv_heads
    bps = default_blocks_per_split(batch, num_kv_heads, max_blocks, block_size,
                                   quant_values=G * head_dim if quant else 0)
    if bps not in (-1, -2):
        return False
    if head_dim not in (64, 128) or (num_q_heads + num_kv_heads) * head_dim // 16 > 256:
        return False
    return not quant or num_kv_heads % 2 == 0 or (G * head_dim) % 128 == 0


def paged_attention_decode_noalloc(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                                   context_lens: torch.Tensor, block_tables: torch.Tensor,
                                   scale: Optional[float] = None, blocks_per_split: Optional[int] = None,
                                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """paged_attention_decode with the split workspace taken from the
    library's static device array (lfs_paged_decode_noalloc): the C call
    allocates nothing, so with a preallocated ``out`` the whole call
    allocates nothing.  Raises ValueError when the shape needs more than
    _lib.DECODE_SCRATCH_BYTES of workspace.  Calls that overlap on one GPU
    share the array and race."""
    assert q.dim() == 3 and q.is_contiguous(), "q must be contiguous [B, Hq, D]"
    assert k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.shape == v_cache.shape
    assert k_cache.dim() == 4, "caches must be [num_blocks, block_size, Hkv, D]"
    assert block_tables.dim() == 2 and block_tables.stride(1) == 1, "block_tables must be [B, max_blocks]"
    assert context_lens.is_contiguous() and context_lens.numel() == q.size(0)
    _on_gpu(q, k_cache, v_cache, context_lens, block_tables)
    for t, n in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _dtype(t, torch.bfloat16, n)
    _dtype(context_lens, torch.int64, "context_lens")
    _dtype(block_tables, torch.int32, "block_tables")
    B, Hq, D = q.shape
    NB, BS, Hkv, Dk = k_cache.shape
    assert Dk == D, "head_dim mismatch between q and the caches"
    assert block_tables.size(0) == B
    max_blocks = block_tables.size(1)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    bps = default_blocks_per_split(B, Hkv, max_blocks, BS) if blocks_per_split is None else blocks_per_split
    if out is None:
        out = torch.empty_like(q)
    assert out.shape == q.shape and out.dtype == torch.bfloat16 and out.is_contiguous()
    rc = _lib.load().lfs_paged_decode_noalloc(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(context_lens),
                                              _ptr(block_tables), block_tables.stride(0), _ptr(out),
                                              B, Hq, Hkv, D, BS, NB, max_blocks, float(scale), bps,
                                              None, None, _stream(q))
    _lib.check(rc, "paged_attention_decode_noalloc")
    return out


def flash_attn_varlen_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                           max_seqlen_q: int, max_seqlen_k: int, softmax_scale: Optional[float] = None,
                           causal: bool = True, block_table: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Varlen causal prefill attention, the call engine/model_runner.py:291-292
    of the reference names for its prefill step (same argument meaning).

    q: bf16 [total_q, Hq, D]; cu_seqlens_q / cu_seqlens_k: int32 [B + 1].
    Without ``block_table``, k and v are bf16 [total_k, Hkv, D] (key t of
    sequence i is row cu_seqlens_k[i] + t); with it (int32 [B, max_blocks],
    a prefix-cache hit) they are the paged caches [num_blocks, block_size,
    Hkv, D].  Queries of sequence i sit at the last lq positions of its lk
    keys and attend to keys up to their own position.  softmax_scale
    defaults to 1/sqrt(D).  Returns bf16 [total_q, Hq, D]."""
    assert causal, "only causal prefill attention is provided"
    assert q.dim() == 3 and q.is_contiguous(), "q must be contiguous [total_q, Hq, D]"
    assert k.is_contiguous() and v.is_contiguous() and k.shape == v.shape
    _on_gpu(q, k, v, cu_seqlens_q, cu_seqlens_k)
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _dtype(t, torch.bfloat16, n)
    _dtype(cu_seqlens_q, torch.int32, "cu_seqlens_q")
    _dtype(cu_seqlens_k, torch.int32, "cu_seqlens_k")
    assert cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous()
    assert cu_seqlens_q.numel() == cu_seqlens_k.numel() >= 1
    B = cu_seqlens_q.numel() - 1
    _, Hq, D = q.shape
    if block_table is not None:
        assert k.dim() == 4, "with block_table, k and v are the paged caches [NB, BS, Hkv, D]"
        _on_gpu(block_table)
        _dtype(block_table, torch.int32, "block_table")
        assert block_table.dim() == 2 and block_table.stride(1) == 1 and block_table.size(0) == B
        NB, BS, Hkv, Dk = k.shape
        bt_ptr, bt_stride, num_slots = _ptr(block_table), block_table.stride(0), NB * BS
    else:
        assert k.dim() == 3, "k and v must be [total_k, Hkv, D]"
        _, Hkv, Dk = k.shape
        bt_ptr, bt_stride, BS, num_slots = None, 0, 0, k.size(0)
    assert Dk == D, "head_dim mismatch between q and k"
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    o = torch.empty_like(q)
    rc = _lib.load().lfs_prefill_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(cu_seqlens_q), _ptr(cu_seqlens_k),
                                           bt_ptr, bt_stride, BS, num_slots, _ptr(o), B, Hq, Hkv, D,
                                           int(max_seqlen_q), float(softmax_scale), _stream(q))
    _lib.check(rc, "flash_attn_varlen_func")
    return o


def fp8_index(q: torch.Tensor, q_s: torch.Tensor, k: torch.Tensor, k_s: torch.Tensor) -> torch.Tensor:
    """Index score of the DSA lightning indexer (model/attention/utils.py:
    230-250): fp8 q @ fp8 k -> fp32 logits, relu(logits) * q_s, sum over
    heads, * k_s.

    q: e4m3fn [b, m, h, d] contiguous; q_s: fp32 [b, m, h] (or [b, m, h, 1]);
    k: e4m3fn [b, n, d] (rows contiguous; a slice of a longer FP8 K cache
    along n is accepted without a copy); k_s: fp32 [b, n].  d in {32, 64,
    128}, h <= 128.  Returns fp32 [b, m, n]."""
    assert q.dim() == 4 and q.is_contiguous(), "q must be contiguous [b, m, h, d]"
    if q_s.dim() == 4:
        assert q_s.size(-1) == 1, "q_s must be [b, m, h] (one weight per head)"
        q_s = q_s.squeeze(-1)
    q_s = q_s.contiguous()
    assert k.dim() == 3 and k.stride(2) == 1 and k.stride(1) == k.size(2), "k rows must be contiguous [b, n, d]"
    assert k_s.dim() == 2 and k_s.stride(1) == 1, "k_s must be [b, n]"
    _on_gpu(q, q_s, k, k_s)
    _dtype(q, FP8, "q")
    _dtype(k, FP8, "k")
    _dtype(q_s, torch.float32, "q_s")
    _dtype(k_s, torch.float32, "k_s")
    b, m, h, d = q.shape
    n = k.size(1)
    assert k.shape == (b, n, d) and q_s.shape == (b, m, h) and k_s.shape == (b, n)
    o = torch.empty(b, m, n, dtype=torch.float32, device=q.device)
    rc = _lib.load().lfs_fp8_index(_ptr(q), _ptr(q_s), _ptr(k), _ptr(k_s), _ptr(o), b, m, n, h, d,
                                   k.stride(0), k_s.stride(0), _stream(q))
    _lib.check(rc, "fp8_index")
    return o


def sample_gumbel(logits: torch.Tensor, temperatures: torch.Tensor, seed: int, offset: int,
                  return_noise: bool = False):
    """Temperature + Gumbel-max sampling (utils/sampler.py:35-53:
    argmax(softmax(logits / T) / Exp(1) noise), noise clamped at 1e-10).

    logits: bf16 [B, V] (unit column stride); temperatures: fp32 [B].  The
    noise of element (b, i) is fixed by (seed, offset, b, i) through
    Philox4x32-10; advance ``offset`` by ceil(V / 4) per call for fresh
    noise.  Returns int64 [B] (and the fp32 [B, V] noise when
    ``return_noise``)."""
    assert logits.dim() == 2 and logits.stride(1) == 1, "logits must be [B, V] with unit column stride"
    _on_gpu(logits, temperatures)
    _dtype(logits, torch.bfloat16, "logits")
    _dtype(temperatures, torch.float32, "temperatures")
    B, V = logits.shape
    if logits.stride(0) < V:  # broadcast rows (an expanded view): give each row its own copy
        logits = logits.contiguous()
    temperatures = temperatures.contiguous()
    assert temperatures.shape == (B,)
    out = torch.empty(B, dtype=torch.int64, device=logits.device)
    noise = torch.empty(B, V, dtype=torch.float32, device=logits.device) if return_noise else None
    L = _lib.load()
    # rows cut into slices when the batch alone leaves CUs idle (same picks)
    need = int(L.lfs_sample_gumbel_workspace_bytes(B, V)) if B > 0 else 0
    ws = torch.empty(max(need, 8), dtype=torch.uint8, device=logits.device)
    rc = L.lfs_sample_gumbel_split(_ptr(logits), logits.stride(0), _ptr(temperatures), B, V,
                                   int(seed) & ((1 << 64) - 1), int(offset) & ((1 << 64) - 1), _ptr(out),
                                   _ptr(noise) if noise is not None else None, _ptr(ws), ws.numel(), _stream(logits))
    _lib.check(rc, "sample_gumbel")
    return (out, noise) if return_noise else out


# ------------------------------------------------- fused decode-step rows --
def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
                residual: Optional[torch.Tensor] = None, out: bool = True, quant: bool = False):
    """RMSNorm with fused residual add (model/utils.py:53-67) in one launch.

    x (and residual): bf16 [T, d] contiguous; weight fp32 [d].  Returns
    (out, residual_out, q, q_scale): out = bf16(weight * r * rsqrt(mean(r^2)
    + eps)) with r = x (+ residual); residual_out = bf16(r) when a residual
    is given, else x; q, q_scale = act_quant(out, 128) when ``quant``.
    """
    assert x.dim() == 2 and x.is_contiguous(), "x must be contiguous [T, d]"
    T, d = x.shape
    _on_gpu(x, weight)
    _dtype(x, torch.bfloat16, "x")
    _dtype(weight, torch.float32, "weight")
    assert weight.is_contiguous() and weight.shape == (d,)
    res_out = None
    if residual is not None:
        _on_gpu(x, residual)
        _dtype(residual, torch.bfloat16, "residual")
        assert residual.shape == x.shape and residual.is_contiguous()
        res_out = torch.empty_like(x)
    y = torch.empty_like(x) if out else None
    q = qs = None
    if quant:
        q = torch.empty(T, d, dtype=FP8, device=x.device)
        qs = torch.empty(T, d // 128, dtype=torch.float32, device=x.device)
    rc = _lib.load().lfs_add_rmsnorm(_ptr(x), _ptr(residual), _ptr(weight), _ptr(y), _ptr(res_out),
                                     _ptr(q), _ptr(qs), T, d, float(eps), _stream(x))
    _lib.check(rc, "add_rmsnorm")
    return y, (res_out if residual is not None else x), q, qs


def splitk_used(K: int, splits: int) -> int:
    """Number of fp32 partials a split-K GEMM over K writes for ``splits``
    requested splits (consecutive runs of ceil((K/128) / splits) K blocks)."""
    kt = K // 128
    kps = -(-kt // max(1, splits))
    return -(-kt // kps)


def fp8_gemm_splitk_partials(a: torch.Tensor, a_s: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
                             splits: int) -> torch.Tensor:
    """The split-K partial sums of fp8_gemm(a, a_s, b, b_s) without the
    reduction: fp32 [n, M, N], n = splitk_used(K, splits) >= 2 (no bias).
    Summing them in order with the bias and rounding to bf16 gives
    fp8_gemm(..., splits=splits) bit for bit; add_rmsnorm_partials does that
    as part of the next add & norm."""
    assert a.is_contiguous() and b.is_contiguous(), "Input tensors must be contiguous"
    assert a_s.is_contiguous() and b_s.is_contiguous(), "Scaling factor tensors must be contiguous"
    _on_gpu(a, a_s, b, b_s)
    _dtype(a, FP8, "a")
    _dtype(b, FP8, "b")
    K = a.size(-1)
    M = a.numel() // K
    N = b.size(0)
    n = splitk_used(K, splits)
    assert n >= 2, "fp8_gemm_splitk_partials needs at least two K splits"
    parts = torch.empty(n, M, N, dtype=torch.float32, device=a.device)
    rc = _lib.load().lfs_fp8_gemm_splitk_partials(_ptr(a), _ptr(a_s), _ptr(b), _ptr(b_s), M, N, K, splits,
                                                  _ptr(parts), parts.numel() * 4, _stream(a))
    _lib.check(rc, "fp8_gemm_splitk_partials")
    return parts


def add_rmsnorm_partials(parts: torch.Tensor, bias: Optional[torch.Tensor], weight: torch.Tensor, eps: float,
                         residual: Optional[torch.Tensor] = None, out: bool = True, quant: bool = False):
    """add_rmsnorm whose x is bf16(sum_s parts[s] + bias), the reduction
    fp8_gemm's split-K would perform (parts: fp32 [n, T, d] from
    fp8_gemm_splitk_partials; bias None, fp32 [d] or [T, d]); the same
    returns as add_rmsnorm, bit-identical to reducing first."""
    assert parts.dim() == 3 and parts.is_contiguous() and parts.dtype == torch.float32
    n, T, d = parts.shape
    _on_gpu(parts, weight)
    _dtype(weight, torch.float32, "weight")
    assert weight.is_contiguous() and weight.shape == (d,)
    bias_ld = 0
    if bias is not None:
        _on_gpu(parts, bias)
        _dtype(bias, torch.float32, "bias")
        assert bias.stride(-1) == 1 and bias.size(-1) == d
        bias_ld = 0 if bias.dim() == 1 else bias.stride(0)
    res_out = None
    if residual is not None:
        _dtype(residual, torch.bfloat16, "residual")
        assert residual.shape == (T, d) and residual.is_contiguous()
        res_out = torch.empty_like(residual)
    y = torch.empty(T, d, dtype=torch.bfloat16, device=parts.device) if out else None
    q = qs = None
    if quant:
        q = torch.empty(T, d, dtype=FP8, device=parts.device)
        qs = torch.empty(T, d // 128, dtype=torch.float32, device=parts.device)
    rc = _lib.load().lfs_add_rmsnorm_partials(_ptr(parts), n, _ptr(bias), bias_ld, _ptr(residual), _ptr(weight),
                                              _ptr(y), _ptr(res_out), _ptr(q), _ptr(qs), T, d, float(eps),
                                              _stream(parts))
    _lib.check(rc, "add_rmsnorm_partials")
    return y, res_out, q, qs


def qk_norm_rope_store(qkv: torch.Tensor, q_weight: torch.Tensor, k_weight: torch.Tensor,
                       cos_sin: torch.Tensor, positions: torch.Tensor, num_q_heads: int,
                       num_kv_heads: int, eps: float, k_cache: Optional[torch.Tensor] = None,
                       v_cache: Optional[torch.Tensor] = None,
                       slot_mapping: Optional[torch.Tensor] = None) -> torch.Tensor:
    """q_norm / k_norm (fp32 RMSNorm over Hq*D and Hkv*D), half-split RoPE
    (model/attention/utils.py:34-45) and the KV slot write, one launch.

    qkv: bf16 [T, (Hq + 2 Hkv) * D] (rows may be strided); cos_sin: fp32
    [max_pos, D] = cat(cos, sin); positions int64 [T]; caches bf16
    [NB, BS, Hkv, D] and slot_mapping int64 [T] (-1 = skip), or None.
    Returns q: bf16 [T, Hq, D].
    """
    assert qkv.dim() == 2 and qkv.stride(1) == 1
    T = qkv.size(0)
    D = cos_sin.size(1)
    assert qkv.size(1) == (num_q_heads + 2 * num_kv_heads) * D, "qkv width mismatch"
    _on_gpu(qkv, q_weight, k_weight, cos_sin, positions)
    _dtype(qkv, torch.bfloat16, "qkv")
    for t, n in ((q_weight, "q_weight"), (k_weight, "k_weight"), (cos_sin, "cos_sin")):
        _dtype(t, torch.float32, n)
        assert t.is_contiguous(), f"{n} must be contiguous"
    _dtype(positions, torch.int64, "positions")
    assert q_weight.numel() == num_q_heads * D and k_weight.numel() == num_kv_heads * D
    num_slots = 0
    if slot_mapping is not None:
        _on_gpu(qkv, k_cache, v_cache, slot_mapping)
        _dtype(slot_mapping, torch.int64, "slot_mapping")
        for t, n in ((k_cache, "k_cache"), (v_cache, "v_cache")):
            _dtype(t, torch.bfloat16, n)
            assert t.is_contiguous() and t.dim() == 4 and t.shape[2:] == (num_kv_heads, D), \
                f"{n} must be [NB, BS, Hkv, D]"
        assert slot_mapping.numel() == T and slot_mapping.is_contiguous()
        num_slots = k_cache.shape[0] * k_cache.shape[1]
    q = torch.empty(T, num_q_heads, D, dtype=torch.bfloat16, device=qkv.device)
    rc = _lib.load().lfs_qk_norm_rope_store(
        _ptr(qkv), qkv.stride(0), _ptr(q_weight), _ptr(k_weight), _ptr(cos_sin), _ptr(positions),
        _ptr(slot_mapping), _ptr(q), _ptr(k_cache), _ptr(v_cache), T, num_q_heads, num_kv_heads, D,
        num_slots, cos_sin.size(0), float(eps), _stream(qkv))
    _lib.check(rc, "qk_norm_rope_store")
    return q


def moe_route(h: torch.Tensor, gate_weight: torch.Tensor, expert_bias: torch.Tensor,
              down_bias: Optional[torch.Tensor], top_k: int, num_shared: int, dense: bool = True,
              return_topk: bool = False):
    """MoE gate (model/architecture/moe.py:45-90).

    h: bf16 [T, d]; gate_weight bf16 [E, d]; expert_bias fp32 [E];
    down_bias fp32 [E + S, d] or None.  Returns (weights fp32 [T, E + S] --
    the renormalised top-k sigmoid scores, 0 for unpicked experts, 1 for the
    S shared experts -- and bias fp32 [T, d] = weights @ down_bias, None
    without down_bias); with ``dense=False`` both are None.  With
    ``return_topk`` also (topk_idx int64 [T, top_k], topk_weight fp32
    [T, top_k]), the gate's index form in pick order.
    """
    assert h.dim() == 2 and h.is_contiguous() and gate_weight.is_contiguous()
    assert dense or return_topk, "moe_route: nothing to return"
    T, d = h.shape
    E = gate_weight.size(0)
    _on_gpu(h, gate_weight, expert_bias)
    _dtype(h, torch.bfloat16, "h")
    _dtype(gate_weight, torch.bfloat16, "gate_weight")
    _dtype(expert_bias, torch.float32, "expert_bias")
    assert gate_weight.shape == (E, d) and expert_bias.shape == (E,)
    if down_bias is not None:
        _on_gpu(h, down_bias)
        _dtype(down_bias, torch.float32, "down_bias")
        assert down_bias.shape == (E + num_shared, d) and down_bias.is_contiguous()
    w = torch.empty(T, E + num_shared, dtype=torch.float32, device=h.device) if dense else None
    bias = torch.empty(T, d, dtype=torch.float32, device=h.device) if dense and down_bias is not None else None
    idx = torch.empty(T, top_k, dtype=torch.int64, device=h.device) if return_topk else None
    wt = torch.empty(T, top_k, dtype=torch.float32, device=h.device) if return_topk else None
    rc = _lib.load().lfs_moe_route(_ptr(h), _ptr(gate_weight), _ptr(expert_bias), _ptr(down_bias),
                                   _ptr(w), _ptr(bias), T, d, E, num_shared, top_k, _ptr(idx), _ptr(wt),
                                   _stream(h))
    _lib.check(rc, "moe_route")
    if return_topk:
        return w, bias, idx, wt
    return w, bias


def add_rmsnorm_route(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: Optional[torch.Tensor],
                      gate_weight: torch.Tensor, expert_bias: torch.Tensor, down_bias: Optional[torch.Tensor],
                      top_k: int, num_shared: int, out: bool = False):
    """The decode step's ffn_norm and MoE gate in one launch: the results of
    add_rmsnorm(x, weight, eps, residual, out, quant=True) followed by
    moe_route(normalised rows, gate_weight, expert_bias, down_bias, top_k,
    num_shared), bit for bit.  Returns (out or None, residual_out, q,
    q_scale, weights fp32 [T, E + S], bias fp32 [T, d] or None)."""
    assert x.dim() == 2 and x.is_contiguous(), "x must be contiguous [T, d]"
    assert gate_weight.is_contiguous()
    T, d = x.shape
    E = gate_weight.size(0)
    _on_gpu(x, weight, gate_weight, expert_bias)
    _dtype(x, torch.bfloat16, "x")
    _dtype(weight, torch.float32, "weight")
    _dtype(gate_weight, torch.bfloat16, "gate_weight")
    _dtype(expert_bias, torch.float32, "expert_bias")
    assert weight.is_contiguous() and weight.shape == (d,)
    assert gate_weight.shape == (E, d) and expert_bias.shape == (E,)
    res_out = None
    if residual is not None:
        _on_gpu(x, residual)
        _dtype(residual, torch.bfloat16, "residual")
        assert residual.shape == x.shape and residual.is_contiguous()
        res_out = torch.empty_like(x)
    if down_bias is not None:
        _on_gpu(x, down_bias)
        _dtype(down_bias, torch.float32, "down_bias")
        assert down_bias.shape == (E + num_shared, d) and down_bias.is_contiguous()
    y = torch.empty_like(x) if out else None
    q = torch.empty(T, d, dtype=FP8, device=x.device)
    qs = torch.empty(T, d // 128, dtype=torch.float32, device=x.device)
    w = torch.empty(T, E + num_shared, dtype=torch.float32, device=x.device)
    bias = torch.empty(T, d, dtype=torch.float32, device=x.device) if down_bias is not None else None
    rc = _lib.load().lfs_add_rmsnorm_route(_ptr(x), _ptr(residual), _ptr(weight), _ptr(y), _ptr(res_out),
                                           _ptr(q), _ptr(qs), T, d, float(eps), _ptr(gate_weight),
                                           _ptr(expert_bias), _ptr(down_bias), _ptr(w), _ptr(bias), E,
                                           num_shared, top_k, _stream(x))
    _lib.check(rc, "add_rmsnorm_route")
    return y, (res_out if residual is not None else x), q, qs, w, bias


def swiglu_quant(h13: torch.Tensor, route_weights: torch.Tensor):
    """silu(w1 x) * (w3 x) with bf16 roundings (model/architecture/mlp.py:
    60-67), quantised per 128 group with each group's scale multiplied by the
    routing weight of its expert.

    h13: bf16 [T, E, 2, F] (w1 rows then w3 rows per expert); route_weights
    fp32 [T, E].  Returns (q e4m3fn [T, E*F], scales fp32 [T, E*F/128]).
    """
    assert h13.dim() == 4 and h13.size(2) == 2 and h13.is_contiguous()
    T, E, _, F = h13.shape
    _on_gpu(h13, route_weights)
    _dtype(h13, torch.bfloat16, "h13")
    _dtype(route_weights, torch.float32, "route_weights")
    assert route_weights.shape == (T, E) and route_weights.is_contiguous()
    assert F % 128 == 0, "d_ff must be a multiple of 128"
    q = torch.empty(T, E * F, dtype=FP8, device=h13.device)
    qs = torch.empty(T, E * F // 128, dtype=torch.float32, device=h13.device)
    rc = _lib.load().lfs_swiglu_quant(_ptr(h13), _ptr(route_weights), _ptr(q), _ptr(qs), T, E, F,
                                      _stream(h13))
    _lib.check(rc, "swiglu_quant")
    return q, qs


# ------------------------------------------------------------ MoE dispatch --
class MoeRows:
    """Result of moe_align: rows grouped by expert in 128-row tiles.

    row_token int32 [P] (token of each row, -1 padding), row_weight fp32 [P]
    (0 padding), tile_expert int32 [P / 128] (-1 past the last segment),
    entry_row int32 [T, top_k + S] (row of each (token, pick), -1 if
    dropped); P = num_tiles * 128."""

    def __init__(self, row_token, row_weight, tile_expert, entry_row):
        self.row_token, self.row_weight = row_token, row_weight
        self.tile_expert, self.entry_row = tile_expert, entry_row

    @property
    def num_rows(self) -> int:
        return self.row_token.numel()


def moe_align_tiles(T: int, top_k: int, num_experts: int, num_shared: int) -> int:
    """128-row tiles moe_align may fill (its output size; fixed per T)."""
    return int(_lib.load().lfs_moe_align_tiles(T, top_k, num_experts, num_shared))


def moe_align(topk_idx: torch.Tensor, topk_weight: torch.Tensor, num_experts: int,
              num_shared: int = 0) -> MoeRows:
    """Group a batch's (token, pick) entries by expert -- the argsort +
    bincount + offsets of MoE.moe_infer (model/architecture/moe.py:298-307)
    on the GPU, with no host sync and an output size fixed by T.

    topk_idx int64 [T, k], topk_weight fp32 [T, k] (the gate's outputs);
    the S shared experts (indices E .. E+S-1, weight 1) are appended to
    every token.  Each expert's rows keep the entries' flat order."""
    assert topk_idx.dim() == 2 and topk_idx.is_contiguous() and topk_weight.is_contiguous()
    _on_gpu(topk_idx, topk_weight)
    _dtype(topk_idx, torch.int64, "topk_idx")
    _dtype(topk_weight, torch.float32, "topk_weight")
    T, k = topk_idx.shape
    assert topk_weight.shape == (T, k)
    tiles = moe_align_tiles(T, k, num_experts, num_shared)
    dev = topk_idx.device
    row_token = torch.empty(tiles * 128, dtype=torch.int32, device=dev)
    row_weight = torch.empty(tiles * 128, dtype=torch.float32, device=dev)
    tile_expert = torch.empty(tiles, dtype=torch.int32, device=dev)
    entry_row = torch.empty(T, k + num_shared, dtype=torch.int32, device=dev)
    L = _lib.load()
    ws = torch.empty(int(L.lfs_moe_align_workspace_bytes(T, k, num_experts, num_shared)) // 4, dtype=torch.int32,
                     device=dev)
    rc = L.lfs_moe_align(_ptr(topk_idx), _ptr(topk_weight), T, k, num_experts, num_shared, _ptr(row_token),
                         _ptr(row_weight), _ptr(tile_expert), tiles, _ptr(entry_row), _ptr(ws), ws.numel() * 4,
                         _stream(topk_idx))
    _lib.check(rc, "moe_align")
    return MoeRows(row_token, row_weight, tile_expert, entry_row)


def fp8_grouped_gemm(a: torch.Tensor, a_s: torch.Tensor, row_index: Optional[torch.Tensor],
                     tile_expert: torch.Tensor, b: torch.Tensor, b_s: torch.Tensor,
                     bias: Optional[torch.Tensor] = None, out_dtype: torch.dtype = torch.bfloat16
                     ) -> torch.Tensor:
    """Per-expert block-scaled FP8 GEMMs over 128-row tiles (the expert MLP
    calls of MoE.moe_infer, model/architecture/moe.py:318-330, batched).

    a e4m3fn [A, K], a_s fp32 [A, K/128]; tile_expert int32 [tiles]; row m
    of the output (tile m // 128) is a[row_index[m]] (row_index int32
    [tiles*128], -1 = padding) or a[m] (row_index None) times expert
    e = tile_expert[m // 128]'s weights b[e] (e4m3fn [E, N, K], any strides
    with unit K stride, e.g. a permuted view of a matrix stacked along K),
    scales b_s[e] (fp32 [E, ceil(N/128), K/128], unit last stride), plus
    bias[e] (fp32 [E, N]) for a bf16 output.  Returns [tiles*128, N] in
    out_dtype (bfloat16, or float32 without bias); rows of tiles with
    e < 0 are left unwritten."""
    _on_gpu(a, a_s, tile_expert, b, b_s)
    _dtype(a, FP8, "a")
    _dtype(b, FP8, "b")
    _dtype(a_s, torch.float32, "a_s")
    _dtype(b_s, torch.float32, "b_s")
    _dtype(tile_expert, torch.int32, "tile_expert")
    assert a.dim() == 2 and a.is_contiguous() and a_s.is_contiguous(), "a, a_s must be contiguous [A, K]"
    A, K = a.shape
    assert K % 128 == 0 and a_s.shape == (A, K // 128)
    assert b.dim() == 3 and b.size(2) == K and b.stride(2) == 1, "b must be [E, N, K] with unit K stride"
    E, N, _ = b.shape
    assert b_s.dim() == 3 and b_s.shape == (E, math.ceil(N / 128), K // 128) and b_s.stride(2) == 1
    assert tile_expert.dim() == 1 and tile_expert.is_contiguous()
    tiles = tile_expert.numel()
    if row_index is not None:
        _on_gpu(a, row_index)
        _dtype(row_index, torch.int32, "row_index")
        assert row_index.is_contiguous() and row_index.numel() == tiles * 128
    else:
        assert A >= tiles * 128, "without row_index, a needs tiles*128 rows"
    assert out_dtype in (torch.bfloat16, torch.float32)
    bias_es = 0
    if bias is not None:
        assert out_dtype == torch.bfloat16, "the fp32 output takes no bias"
        _on_gpu(a, bias)
        _dtype(bias, torch.float32, "bias")
        assert bias.shape == (E, N) and bias.stride(1) == 1
        bias_es = bias.stride(0)
    c = torch.empty(tiles * 128, N, dtype=out_dtype, device=a.device)
    is_f32 = out_dtype == torch.float32
    rc = _lib.load().lfs_fp8_grouped_gemm(
        _ptr(a), _ptr(a_s), A, _ptr(row_index), _ptr(tile_expert), tiles, _ptr(b), _ptr(b_s), b.stride(0),
        b.stride(1), b_s.stride(0), b_s.stride(1), _ptr(bias), bias_es, None if is_f32 else _ptr(c),
        _ptr(c) if is_f32 else None, N, K, _stream(a))
    _lib.check(rc, "fp8_grouped_gemm")
    return c


def moe_combine(out: torch.Tensor, entry_row: torch.Tensor, topk_idx: torch.Tensor, topk_weight: torch.Tensor,
                num_experts: int, num_shared: int = 0, down_bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y[t] = bf16(sum_j out[entry_row[t, j]] + sum_j w_tj * down_bias[e_tj])
    over the token's picks then its shared experts, fp32 in that order: the
    scatter_add_ of MoE.moe_infer (model/architecture/moe.py:332-339) plus
    the shared-expert add (:272-273).  out: bf16 or fp32 [rows, d] (routing
    weights already applied); down_bias fp32 [E + S, d] or None."""
    _on_gpu(out, entry_row, topk_idx, topk_weight)
    assert out.dtype in (torch.bfloat16, torch.float32), "out must be bf16 or fp32"
    _dtype(entry_row, torch.int32, "entry_row")
    assert out.dim() == 2 and out.stride(1) == 1 and entry_row.is_contiguous()
    T, k = topk_idx.shape
    assert entry_row.shape == (T, k + num_shared)
    d = out.size(1)
    if down_bias is not None:
        _on_gpu(out, down_bias)
        _dtype(down_bias, torch.float32, "down_bias")
        assert down_bias.shape == (num_experts + num_shared, d) and down_bias.is_contiguous()
    y = torch.empty(T, d, dtype=torch.bfloat16, device=out.device)
    rc = _lib.load().lfs_moe_combine(_ptr(out), int(out.dtype == torch.float32), out.stride(0), _ptr(entry_row),
                                     _ptr(topk_idx), _ptr(topk_weight), T, k, num_experts, num_shared,
                                     _ptr(down_bias), d, _ptr(y), _stream(out))
    _lib.check(rc, "moe_combine")
    return y


def _seg_args(expert_output: torch.Tensor, weights: torch.Tensor, idx: torch.Tensor):
    assert expert_output.dim() == 2 and expert_output.stride(1) == 1, "expert_output must be [n, d] rows"
    assert expert_output.dtype in (torch.bfloat16, torch.float32), "expert_output must be bf16 or fp32"
    assert weights.dtype in (torch.bfloat16, torch.float32), "weights must be bf16 or fp32"
    _on_gpu(expert_output, weights, idx)
    _dtype(idx, torch.int64, "token indices")
    weights = weights.reshape(-1).contiguous()
    idx = idx.reshape(-1).contiguous()
    n = expert_output.size(0)
    assert weights.numel() == n and idx.numel() == n
    return weights, idx, n


def segment_reduce_weighted(expert_output: torch.Tensor, sorted_weights: torch.Tensor,
                            sorted_token_idx: torch.Tensor, num_tokens: int, top_k: int) -> torch.Tensor:
    """model/architecture/moe_kernels.py:70-125: y[t] = sum of
    expert_output[p] * sorted_weights[p] over the segment of p with
    sorted_token_idx[p] == t (sorted_token_idx non-decreasing), fp32
    accumulation, returned in expert_output's dtype [num_tokens, d].
    ``top_k`` is accepted for the signature; every entry of a segment is
    summed."""
    w, idx, n = _seg_args(expert_output, sorted_weights, sorted_token_idx)
    d = expert_output.size(1)
    y = torch.empty(num_tokens, d, dtype=expert_output.dtype, device=expert_output.device)
    rc = _lib.load().lfs_segment_reduce_weighted(
        _ptr(expert_output), int(expert_output.dtype == torch.float32), expert_output.stride(0), _ptr(w),
        int(w.dtype == torch.float32), _ptr(idx), n, num_tokens, d, _ptr(y), _stream(expert_output))
    _lib.check(rc, "segment_reduce_weighted")
    return y


def fused_scatter_add_weighted(expert_output: torch.Tensor, sorted_token_idx: torch.Tensor,
                               sorted_weights: torch.Tensor, num_tokens: int, top_k: int = 2) -> torch.Tensor:
    """model/architecture/moe_kernels.py:128-171: y[t] = sum over entries i
    with sorted_token_idx[i] == t (any order) of expert_output[i] *
    sorted_weights[i], fp32 accumulation in increasing i, returned in
    expert_output's dtype [num_tokens, d].  ``top_k`` is accepted for the
    signature."""
    w, idx, n = _seg_args(expert_output, sorted_weights, sorted_token_idx)
    d = expert_output.size(1)
    L = _lib.load()
    ws = torch.empty(max(1, int(L.lfs_scatter_add_weighted_workspace_bytes(n, num_tokens)) // 4),
                     dtype=torch.int32, device=expert_output.device)
    y = torch.empty(num_tokens, d, dtype=expert_output.dtype, device=expert_output.device)
    rc = L.lfs_scatter_add_weighted(_ptr(expert_output), int(expert_output.dtype == torch.float32),
                                    expert_output.stride(0), _ptr(w), int(w.dtype == torch.float32), _ptr(idx), n,
                                    num_tokens, d, _ptr(y), _ptr(ws), ws.numel() * 4, _stream(expert_output))
    _lib.check(rc, "fused_scatter_add_weighted")
    return y

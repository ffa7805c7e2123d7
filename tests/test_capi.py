"""The C-ABI library loads and exports every symbol include/lfs_kernels.h
declares; host-side argument checks fail with negative codes before any
launch (no GPU work is done here)."""
import ctypes
import re
from pathlib import Path

import pytest

from llm_from_scratch_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "lfs_kernels.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lfs_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.fail("liblfs_kernels.so is not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_and_binding_agree():
    assert declared_symbols() == sorted(_lib.SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in declared_symbols():
        assert hasattr(raw, name), name
    assert lib.lfs_abi_version() == _lib.ABI_VERSION


def test_argument_errors_are_reported_without_launch(lib):
    # block_size 100 is rejected on the host
    rc = lib.lfs_act_quant(None, 128, None, None, 4, 128, 100, 0, None)
    assert rc == -1 and b"block_size" in lib.lfs_last_error()
    rc = lib.lfs_act_quant(None, 256, None, None, 4, 200, 128, 0, None)
    assert rc == -1 and b"divisible" in lib.lfs_last_error()
    rc = lib.lfs_fp8_gemm(None, None, None, None, None, 0, None, 4, 4, 100, None)
    assert rc == -1 and b"multiple of 128" in lib.lfs_last_error()
    rc = lib.lfs_paged_decode(None, None, None, None, None, 4, None, None, 0, 2, 16, 4, 96, 256, 8, 4,
                              0.1, 1, None, None, None)
    assert rc == -1 and b"head_dim" in lib.lfs_last_error()
    rc = lib.lfs_paged_decode(None, None, None, None, None, 4, None, None, 0, 2, 12, 5, 64, 256, 8, 4,
                              0.1, 1, None, None, None)
    assert rc == -1 and b"multiple of num_kv_heads" in lib.lfs_last_error()
    rc = lib.lfs_paged_decode(16, 16, 16, 16, 16, 4, 16, 16, 1 << 20, 2, 12, 4, 64, 256, 8, 4,
                              0.1, 1, 16, None, None)
    assert rc == -1 and b"go together" in lib.lfs_last_error()
    # the balanced split (blocks_per_split 0) is limited to 8192 sequences
    rc = lib.lfs_paged_decode(16, 16, 16, 16, 16, 4, 16, 16, 1 << 20, 8193, 12, 4, 64, 256, 8, 4,
                              0.1, 0, None, None, None)
    assert rc == -1 and b"balanced split" in lib.lfs_last_error()
    with pytest.raises(ValueError, match="block_size"):
        _lib.check(lib.lfs_weight_quant(None, None, None, 8, 8, 7, None), "weight_quant")
    # split-K needs its workspace (non-null dummy pointers: the check comes first)
    rc = lib.lfs_fp8_gemm_splitk(16, 16, 16, 16, None, 0, 16, 8, 8, 512, 4, None, 0, None)
    assert rc == -1 and b"workspace" in lib.lfs_last_error()
    rc = lib.lfs_fp8_gemm(16, 16, 16, 16, 16, 4, 16, 8, 8, 128, None)
    assert rc == -1 and b"bias_ld" in lib.lfs_last_error()
    rc = lib.lfs_fp8_gemm_skinny(16, 16, 16, 16, None, 0, 16, 129, 8, 128, None)
    assert rc == -1 and b"<= 128" in lib.lfs_last_error()
    rc = lib.lfs_fp8_gemm_skinny(16, 16, 16, 16, None, 0, 16, 8, 8, 100, None)
    assert rc == -1 and b"multiple of 128" in lib.lfs_last_error()
    rc = lib.lfs_add_rmsnorm(None, None, None, None, None, None, None, 4, 100, 1e-5, None)
    assert rc == -1 and b"multiple of 8" in lib.lfs_last_error()
    rc = lib.lfs_add_rmsnorm(None, None, None, None, None, 16, 16, 4, 200, 1e-5, None)
    assert rc == -1 and b"128" in lib.lfs_last_error()
    rc = lib.lfs_qk_norm_rope_store(None, 1280, None, None, None, None, None, None, None, None, 4, 12, 4, 72,
                                    0, 4096, 1e-6, None)
    assert rc == -1 and b"head_dim" in lib.lfs_last_error()
    rc = lib.lfs_moe_route(None, None, None, None, None, None, 4, 768, 8, 1, 9, None, None, None)
    assert rc == -1 and b"top_k" in lib.lfs_last_error()
    rc = lib.lfs_moe_route(16, 16, 16, None, 16, 16, 4, 768, 8, 1, 2, None, None, None)
    assert rc == -1 and b"down_bias" in lib.lfs_last_error()
    rc = lib.lfs_swiglu_quant(None, None, None, None, 4, 9, 500, None)
    assert rc == -1 and b"d_ff" in lib.lfs_last_error()
    # MoE dispatch: capacity too small, too many experts, fp32 output with a bias, bad K
    rc = lib.lfs_moe_align(16, 16, 100, 2, 8, 1, 16, 16, 16, 3, 16, 16, 1 << 20, None)
    assert rc == -1 and b"tiles needed" in lib.lfs_last_error()
    rc = lib.lfs_moe_align(16, 16, 100, 2, 64, 1, 16, 16, 16, 1000, 16, 16, 1 << 20, None)
    assert rc == -1 and b"at most 64 experts" in lib.lfs_last_error()
    rc = lib.lfs_moe_align(16, 16, 100, 2, 8, 1, 16, 16, 16, 20, 16, 16, 8, None)
    assert rc == -1 and b"workspace" in lib.lfs_last_error()
    rc = lib.lfs_fp8_grouped_gemm(16, 16, 8, None, 16, 1, 16, 16, 0, 256, 0, 2, 16, 0, None, 16, 128, 256, None)
    assert rc == -1 and b"no bias" in lib.lfs_last_error()
    rc = lib.lfs_fp8_grouped_gemm(16, 16, 8, None, 16, 1, 16, 16, 0, 256, 0, 2, None, 0, 16, None, 128, 200, None)
    assert rc == -1 and b"multiple of 128" in lib.lfs_last_error()
    rc = lib.lfs_moe_combine(16, 1, 104, 16, 16, 16, 4, 2, 8, 1, None, 100, 16, None)
    assert rc == -1 and b"multiple of 8" in lib.lfs_last_error()
    rc = lib.lfs_scatter_add_weighted(16, 0, 8, 16, 1, 16, 10, 5, 8, 16, None, 0, None)
    assert rc == -1 and b"workspace" in lib.lfs_last_error()


def test_moe_capacity_helpers(lib):
    # 100 tokens x (2 picks + 1 shared) over 9 experts: (300 + 9*127 + 127) // 128
    assert lib.lfs_moe_align_tiles(100, 2, 8, 1) == (300 + 9 * 127 + 127) // 128
    assert lib.lfs_moe_align_tiles(0, 2, 8, 1) == 0
    # 3000 entries -> 3 chunks of 1024, 9 experts
    assert lib.lfs_moe_align_workspace_bytes(1000, 2, 8, 1) == 4 * (3 * 9 + 2 * 9 + 1)
    assert lib.lfs_scatter_add_weighted_workspace_bytes(10, 5) == 4 * (3 * 5 + 1 + 10)


def test_gemm_workspace_bytes(lib):
    # K = 5 blocks over 3 splits -> 2 blocks per split -> 3 partial tiles
    assert lib.lfs_fp8_gemm_workspace_bytes(10, 20, 640, 3) == 3 * 10 * 20 * 4
    # 4 blocks over 3 splits -> 2 per split -> 2 partials
    assert lib.lfs_fp8_gemm_workspace_bytes(10, 20, 512, 3) == 2 * 10 * 20 * 4
    assert lib.lfs_fp8_gemm_workspace_bytes(10, 20, 128, 8) == 0
    assert lib.lfs_fp8_gemm_workspace_bytes(10, 20, 512, 1) == 0


def test_empty_shapes_are_no_ops(lib):
    assert lib.lfs_act_quant(None, 128, None, None, 0, 128, 128, 0, None) == 0
    assert lib.lfs_fp8_gemm(None, None, None, None, None, 0, None, 0, 64, 128, None) == 0
    assert lib.lfs_store_kvcache(None, 0, None, 0, None, None, None, 0, 4, 64, 0, None) == 0


def test_workspace_bytes(lib):
    # 4 bytes * B * splits * Hq * (D + 2)
    assert lib.lfs_paged_decode_workspace_bytes(64, 16, 64, 16, 1) == 4 * 64 * 16 * 16 * 66
    assert lib.lfs_paged_decode_workspace_bytes(3, 8, 128, 10, 4) == 4 * 3 * 3 * 8 * 130
    assert lib.lfs_paged_decode_workspace_bytes(3, 8, 128, 10, -1) == 0  # single launch: none
    assert lib.lfs_paged_decode_workspace_bytes(3, 8, 128, 10, -2) == 0  # paired single launch: none
    assert lib.lfs_paged_decode_workspace_bytes(3, 8, 128, 10, -3) == -1
    # balanced split (0): (8 * CUs + 2 * B) * Hq partial rows of D + 2 floats, then B + 1 ints
    v = lib.lfs_paged_decode_workspace_bytes(3, 8, 128, 10, 0)
    rows, rem = divmod(v - 4 * 4, 4 * 8 * 130)
    assert rem == 0 and rows - 6 > 0 and (rows - 6) % 8 == 0


def test_default_decode_split_rule():
    """The decode mode is chosen from shapes only (capturable): the paired
    single launch (-2) when B <= 256, the B * Hkv workgroups are more than
    one and at most two per CU, the table holds <= 8192 tokens and a
    quantised output has whole 128-value groups per kv head; else the
    single launch (-1) when Hkv is even, the B * Hkv / 2 workgroups cover
    every CU (at most four rounds) and the table holds <= 8192 tokens; else
    the balanced split (0) up to 8192 sequences, else fixed chunks."""
    from llm_from_scratch_amd import kernels as K
    assert K.default_blocks_per_split(128, 4, 16, 256, cus=256) == -2   # cfg5 attention shape, no act_quant
    assert K.default_blocks_per_split(128, 4, 16, 256, cus=256, quant_values=192) == -1  # cfg5 step (G*D 192)
    assert K.default_blocks_per_split(128, 4, 16, 256, cus=256, quant_values=256) == -2
    assert K.default_blocks_per_split(300, 1, 16, 256, cus=256) != -2   # more than 256 sequences
    assert K.default_blocks_per_split(128, 4, 64, 256, cus=256) != -2   # tables past 8192 tokens
    assert K.default_blocks_per_split(64, 4, 16, 256, cus=256) == 0     # cfg3: 128 workgroups
    assert K.default_blocks_per_split(256, 8, 128, 256, cus=256) == 0   # cfg4: tables of 32768 tokens
    assert K.default_blocks_per_split(128, 3, 16, 256, cus=256) == -2   # odd Hkv: one head per workgroup
    assert K.default_blocks_per_split(128, 3, 16, 256, cus=256, quant_values=192) == 0  # odd Hkv, G*D 192
    assert K.default_blocks_per_split(1024, 4, 16, 256, cus=256) == 0   # more than four rounds
    assert K.default_blocks_per_split(8200, 1, 4, 16, cus=256) > 0      # above the balanced limit


def test_decode_gemm_dispatch_rule():
    """Which GEMM kernel a decode-sized call gets (shapes only): the skinny
    kernel for M <= 16, the one-shot kernel for the cfg5 step's M = 128
    projections and the split partials of its down projection, the tile
    kernel for lm_head's 32000 columns."""
    from llm_from_scratch_amd import kernels as K
    assert K.use_skinny_gemm(16, 1024, 4096) and not K.use_skinny_gemm(17, 1024, 4096)
    assert K.flat_gemm_variant(128, 1280, 768) == "r32c16"     # fused QKV
    assert K.flat_gemm_variant(128, 768, 768) == "r32c16"      # output projection
    assert K.flat_gemm_variant(128, 9216, 768) == "r128c48"    # stacked w13
    assert K.flat_gemm_variant(128, 14000, 512) == "r128c64"
    assert K.flat_gemm_variant(128, 32000, 768) is None        # lm_head
    assert K.flat_gemm_variant(128, 768, 4608) is None         # down projection: split instead
    assert K.default_gemm_splits(128, 768, 4608) == 5
    assert K.flat_gemm_variant(128, 768, 4608, kps=8) == "s32c32"
    assert K.default_gemm_splits(128, 9216, 768) == 1

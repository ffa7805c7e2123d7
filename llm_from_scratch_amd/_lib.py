"""ctypes binding of the gfx950 kernel library (C ABI in include/lfs_kernels.h).

There is no fallback: if ``liblfs_kernels.so`` is missing or does not load,
every operator raises.  torch is imported before the library is opened so the
library binds to the HIP runtime torch already loaded (one runtime per
process).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "liblfs_kernels.so"
ABI_VERSION = 15
# size of the library's static paged-decode workspace (LFS_DECODE_SCRATCH_BYTES)
DECODE_SCRATCH_BYTES = 64 << 20

_c_i64, _c_i32, _c_p, _c_f = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_float

# name -> (restype, argtypes); must match include/lfs_kernels.h
SIGNATURES = {
    "lfs_abi_version": (ctypes.c_int, []),
    "lfs_last_error": (ctypes.c_char_p, []),
    "lfs_act_quant": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_i32, _c_p]),
    "lfs_weight_quant": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_p]),
    "lfs_weight_dequant": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i32, _c_p]),
    "lfs_fp8_gemm": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                    _c_p]),
    "lfs_fp8_gemm_act_supported": (ctypes.c_int, [_c_i64, _c_i64, _c_i64]),
    "lfs_fp8_gemm_act": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                        _c_p]),
    "lfs_fp8_gemm_workspace_bytes": (ctypes.c_int64, [_c_i64, _c_i64, _c_i64, _c_i32]),
    "lfs_fp8_gemm_splitk": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                           _c_i32, _c_p, _c_i64, _c_p]),
    "lfs_fp8_gemm_skinny": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i64, _c_i64,
                                           _c_p]),
    "lfs_store_kvcache": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i32,
                                         _c_i32, _c_i64, _c_p]),
    "lfs_paged_decode_workspace_bytes": (ctypes.c_int64, [_c_i64, _c_i32, _c_i32, _c_i32, _c_i32]),
    "lfs_paged_decode": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64,
                                        _c_i32, _c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_f, _c_i32,
                                        _c_p, _c_p, _c_p]),
    "lfs_paged_decode_rope": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_f, _c_p, _c_p,
                                             _c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i32, _c_i32, _c_i32,
                                             _c_i32, _c_i64, _c_i32, _c_f, _c_p, _c_p, _c_p]),
    "lfs_paged_decode_noalloc": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_i32, _c_i32,
                                                _c_i32, _c_i32, _c_i64, _c_i32, _c_f, _c_i32, _c_p, _c_p, _c_p]),
    "lfs_add_rmsnorm": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_f, _c_p]),
    "lfs_add_rmsnorm_partials": (ctypes.c_int, [_c_p, _c_i32, _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                                _c_i64, _c_i32, _c_f, _c_p]),
    "lfs_fp8_gemm_splitk_partials": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_i64, _c_i32, _c_p,
                                                    _c_i64, _c_p]),
    "lfs_qk_norm_rope_store": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                              _c_i64, _c_i32, _c_i32, _c_i32, _c_i64, _c_i64, _c_f, _c_p]),
    "lfs_add_rmsnorm_route": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_f,
                                             _c_p, _c_p, _c_p, _c_p, _c_p, _c_i32, _c_i32, _c_i32, _c_p]),
    "lfs_moe_route": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32,
                                     _c_i32, _c_p, _c_p, _c_p]),
    "lfs_swiglu_quant": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_p]),
    "lfs_fp8_index": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i64,
                                     _c_i64, _c_p]),
    "lfs_sample_gumbel": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i32, ctypes.c_uint64, ctypes.c_uint64,
                                         _c_p, _c_p, _c_p]),
    "lfs_sample_gumbel_workspace_bytes": (ctypes.c_int64, [_c_i64, _c_i32]),
    "lfs_sample_gumbel_split": (ctypes.c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_i32, ctypes.c_uint64, ctypes.c_uint64,
                                               _c_p, _c_p, _c_p, _c_i64, _c_p]),
    "lfs_prefill_attention": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i64, _c_p,
                                             _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_f, _c_p]),
    "lfs_moe_align_tiles": (ctypes.c_int64, [_c_i64, _c_i32, _c_i32, _c_i32]),
    "lfs_moe_align": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32, _c_p, _c_p, _c_p, _c_i64, _c_p,
                                     _c_p, _c_i64, _c_p]),
    "lfs_moe_align_workspace_bytes": (ctypes.c_int64, [_c_i64, _c_i32, _c_i32, _c_i32]),
    "lfs_fp8_grouped_gemm": (ctypes.c_int, [_c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64,
                                            _c_i64, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_p]),
    "lfs_moe_combine": (ctypes.c_int, [_c_p, _c_i32, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_i32, _c_i32, _c_i32,
                                       _c_p, _c_i32, _c_p, _c_p]),
    "lfs_segment_reduce_weighted": (ctypes.c_int, [_c_p, _c_i32, _c_i64, _c_p, _c_i32, _c_p, _c_i64, _c_i64,
                                                   _c_i32, _c_p, _c_p]),
    "lfs_scatter_add_weighted_workspace_bytes": (ctypes.c_int64, [_c_i64, _c_i64]),
    "lfs_scatter_add_weighted": (ctypes.c_int, [_c_p, _c_i32, _c_i64, _c_p, _c_i32, _c_p, _c_i64, _c_i64, _c_i32,
                                                _c_p, _c_p, _c_i64, _c_p]),
}

_LIB = None


class KernelLibraryError(RuntimeError):
    pass


def load(path: Path | str | None = None):
    """Open the library once and attach the ctypes signatures."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    import torch  # noqa: F401  (bind to torch's HIP runtime)

    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise KernelLibraryError(
            f"{p} is not built: run `python -m llm_from_scratch_amd.build` (there is no CPU fallback)")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.lfs_abi_version() != ABI_VERSION:
        raise KernelLibraryError(f"ABI version {lib.lfs_abi_version()} != expected {ABI_VERSION}")
    if path is None:
        _LIB = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().lfs_last_error().decode(errors="replace")
        if rc < 0:
            raise ValueError(f"{what}: {msg}")
        raise KernelLibraryError(f"{what}: {msg} (hipError {rc})")

"""Build the gfx950 kernel library ``liblfs_kernels.so`` in-tree with hipcc.

    python -m llm_from_scratch_amd.build

Cross-compiles on a machine without a GPU.  The library has a plain C ABI
(include/lfs_kernels.h) and is loaded with ctypes; it links the HIP runtime
by soname, so inside a process that imported torch it binds to the runtime
torch already loaded.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
LIB_PATH = PKG_DIR / "liblfs_kernels.so"
SOURCES = ["capi.hip", "quant.hip", "fp8_gemm.hip", "paged_kv.hip", "fused.hip", "prefill.hip", "sampler.hip", "indexer.hip", "moe.hip"]
# benchmark instrument (the decode's read ceiling), a library of its own that
# nothing in the package loads: only bench.py does
PROBE_PATH = PKG_DIR / "liblfs_probe.so"
PROBE_SOURCES = ["probe.hip"]

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "--offload-arch=gfx950",
    "-fPIC",
    "-shared",
    # no packed fp32 (v_pk_*_f32) instructions in any generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in VGPRs: the accumulators are scaled by VALU FMAs, which
    # cannot read AGPRs (an AGPR result costs one v_accvgpr_read per element)
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # IEEE fp32 divide (act_quant's x / s must be correctly rounded)
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-fast-math",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the gfx950 kernel library cannot be built")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    if verbose and res.stderr.strip():
        print(res.stderr, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source into LIB_PATH, and the benchmark probe into
    PROBE_PATH (always recompiles): one object per source, compiled in
    parallel, then one shared-library link per library."""
    flags = [f for f in HIPCC_FLAGS if f != "-shared"]
    libs = ((LIB_PATH, SOURCES), (PROBE_PATH, PROBE_SOURCES))
    with tempfile.TemporaryDirectory(prefix="lfs_build_") as d:
        objs = {lib: [str(Path(d) / (s.rsplit(".", 1)[0] + ".o")) for s in srcs] for lib, srcs in libs}
        cmds = [[hipcc(), *flags, f"-I{REPO / 'include'}", "-c", str(CSRC / s), "-o", o]
                for lib, srcs in libs for s, o in zip(srcs, objs[lib])]
        n = jobs or max(1, min(len(cmds), os.cpu_count() or 1, 8))
        with ThreadPoolExecutor(max_workers=n) as ex:
            for f in [ex.submit(_run, c, verbose) for c in cmds]:
                f.result()
        for lib, _ in libs:
            tmp = lib.with_suffix(".so.tmp")
            _run([hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", *objs[lib], "-o", str(tmp)], verbose)
            os.replace(tmp, lib)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))

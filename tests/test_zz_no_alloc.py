"""lfs_paged_decode_noalloc (the decode with the library's static workspace)
against lfs_paged_decode with a caller-owned workspace, through the C ABI.

Both run the same kernels over the same inputs, so the outputs must be
bit-identical.  Two calls in a row, the second on a smaller batch, check
that the static array's leftover contents from the first call do not leak
into the second; a shape whose workspace exceeds the array is rejected.
"""
import os
import subprocess
import sys
import textwrap

import numpy as np
import pytest
import torch

from llm_from_scratch_amd import _lib
from llm_from_scratch_amd import kernels as K
from llm_from_scratch_amd import workloads as W

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(batch, seed):
    case = W.paged_case("cfg3", seed=seed, batch=batch)
    kc, vc = W.fill_pool(case, seed=seed, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(seed + 7)
    q = torch.randn(case.batch, case.num_q_heads, case.head_dim, generator=g, device=DEV).to(torch.bfloat16)
    cl = torch.from_numpy(case.context_lens).to(DEV)
    bt = torch.from_numpy(case.block_tables).to(DEV)
    return case, q, kc, vc, cl, bt


@pytest.mark.parametrize("bps", [0, 2])
def test_noalloc_matches_workspace_entry_point(bps):
    # first call: the full cfg3 batch; second: a smaller batch whose partial
    # rows land where the first call left its own
    for batch, seed in ((64, 2), (9, 5)):
        case, q, kc, vc, cl, bt = _inputs(batch, seed)
        print(f"noalloc: batch {batch} seed {seed} blocks_per_split {bps}", flush=True)
        ref = K.paged_attention_decode(q, kc, vc, cl, bt, case.scale, bps)
        got = K.paged_attention_decode_noalloc(q, kc, vc, cl, bt, case.scale, bps)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"batch {batch}: outputs differ"
        assert np.isfinite(got.float().cpu().numpy()).all()


def test_noalloc_rejects_shape_beyond_scratch():
    # B 4096 x Hq 64 x D 128 needs (8*CUs + 2*B)*Hq*(D+2)*4 bytes > 64 MiB
    B, Hq, Hkv, D, NB, BS = 4096, 64, 8, 128, 4, 16
    need = K.paged_decode_workspace_bytes(B, Hq, D, 1, 0)
    assert need > _lib.DECODE_SCRATCH_BYTES
    q = torch.zeros(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    kc = torch.zeros(NB, BS, Hkv, D, dtype=torch.bfloat16, device=DEV)
    cl = torch.ones(B, dtype=torch.int64, device=DEV)
    bt = torch.zeros(B, 1, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError, match="static scratch"):
        K.paged_attention_decode_noalloc(q, kc, kc, cl, bt, None, 0)


_CAPTURE_CHILD = textwrap.dedent("""
    import sys, torch
    sys.path.insert(0, sys.argv[1])
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd import workloads as W
    case = W.paged_case("cfg3", seed=3, batch=24)
    kc, vc = W.fill_pool(case, seed=3, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(10)
    q = torch.randn(case.batch, case.num_q_heads, case.head_dim, generator=g, device="cuda").to(torch.bfloat16)
    cl = torch.from_numpy(case.context_lens).to("cuda")
    bt = torch.from_numpy(case.block_tables).to("cuda")
    out = torch.empty_like(q)
    torch.cuda.synchronize()
    print("child: capturing the process's first noalloc call", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        K.paged_attention_decode_noalloc(q, kc, vc, cl, bt, case.scale, 0, out=out)
    ref = K.paged_attention_decode(q, kc, vc, cl, bt, case.scale, 0)
    for r in range(2):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"replay {r} differs"
        _ = (q.float() * 2).sum().item()  # eager work between the replays
    print("child: OK", flush=True)
""")


def test_noalloc_first_call_under_graph_capture():
    """In a fresh process the first lfs_paged_decode_noalloc call (and so the
    first lookup of the static array's device address) happens inside a
    torch.cuda.graph capture; two replays, with eager work between them, are
    bit-identical to lfs_paged_decode with a caller-owned workspace."""
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("noalloc: graph capture in a child process", flush=True)
    res = subprocess.run([sys.executable, "-c", _CAPTURE_CHILD, repo], capture_output=True, text=True,
                         timeout=300)
    assert res.returncode == 0 and "child: OK" in res.stdout, res.stdout[-2000:] + res.stderr[-3000:]

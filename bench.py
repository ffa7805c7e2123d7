"""Benchmark of the block-wise FP8 GEMM and paged-KV decode path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu] [--no-extra]

Prints ONE JSON line.  Headline (``value``): fp8_gemm TFLOP/s over the
cfg2 sweep's compute-bound shapes, one step = the six GEMMs
M in {4096, 16384} x (K, N) in {(1024,4096), (4096,1024), (2048,5632)} with
1x128 activation / 128x128 weight scales, inputs already quantised and
resident in HBM.  ``roofline`` prices the GEMM against the dense FP8 MFMA
peak (5.0 PFLOP/s); each launch is bracketed by HIP events on the stream it
runs on.  ``roofline_decode`` prices the paged decode of cfg3 (the other half
of the metric) against 8 TB/s.  ``paged_decode`` (cfg3, cfg3_4k, cfg4),
``act_quant`` (every cfg2 (M, K)), ``store_kvcache`` and the decode-sized
GEMMs report HBM GB/s against 8 TB/s with the 256 MB last-level cache
flushed before every timed call.  ``traffic`` and ``kernel_us`` figures come
from the rocprofv3 summaries under profiles/, used only when the kernel
source they were measured on is the one built (sha256 recorded there).
``cpu_baseline`` times the CPU restatements on all host cores (1 warm-up,
median of 5; 3 for cfg4 and cfg5): the numpy oracle's blockwise fp32 GEMM on
the three M=4096 shapes (the headline ``value``), plus act_quant, paged
decode (cfg3, a 16-sequence cfg4 subset), store_kvcache, the cfg1 FP8
linear and the cfg5 decode step (32 of its 128 sequences) in torch CPU ops.
"""
from __future__ import annotations

import argparse
import hashlib
import json
import math
import os
import re
import sys
import time

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
METRIC = "FP8 block-GEMM TFLOP/s & paged-decode HBM GB/s (% of MI355X roofline)"
REPO = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(REPO, "llm_from_scratch_amd", "csrc")
PROFILES = os.path.join(REPO, "profiles")


def source_sha(name: str) -> str:
    with open(os.path.join(CSRC, name), "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()[:16]


def profile_figures(md: str, key: str, source: str) -> dict:
    """Figures a rocprofv3 summary under profiles/ records for `key`, in a
    line ``<!-- bench key=... source=<file> sha=<16 hex> name=value ... -->``.
    Returned only if that sha is the current source's, so a kernel change
    makes them null until the PMC runs are repeated."""
    path = os.path.join(PROFILES, md)
    try:
        text = open(path).read()
    except OSError:
        return {"stale": "no profile " + md}
    for m in re.finditer(r"<!-- bench (.*?) -->", text):
        kv = dict(item.split("=", 1) for item in m.group(1).split())
        if kv.get("key") != key:
            continue
        if kv.get("sha") != source_sha(source):
            return {"stale": f"{md}: measured on {source} sha {kv.get('sha')}, built {source_sha(source)}"}
        return {k: float(v) for k, v in kv.items() if k not in ("key", "source", "sha")}
    return {"stale": f"{md}: no entry {key}"}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def timed_launches(fns, reps, flush=None):
    """Run each fn `reps` times, bracketing every launch with events on the
    current stream; returns per-fn mean kernel-time in seconds."""
    stream = torch.cuda.current_stream()
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(reps)] for _ in fns]
    for r in range(reps):
        for i, fn in enumerate(fns):
            if flush is not None:
                flush()
            evs[i][r][0].record(stream)
            fn()
            evs[i][r][1].record(stream)
    torch.cuda.synchronize()
    return [sum(a.elapsed_time(b) for a, b in e) / reps / 1e3 for e in evs]


def gemm_setup(device):
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd import workloads as W
    cases = []
    for M in (4096, 16384):
        for Kd, N in W.GEMM_KN:
            x = W.activation(M, Kd, seed=1 + M + Kd, device=device)
            w = W.weight(N, Kd, seed=31 + Kd, device=device)
            xq, xs = K.act_quant(x)
            wq, ws = K.weight_quant(w)
            del x, w
            cases.append(dict(M=M, K=Kd, N=N, a=xq, a_s=xs, b=wq, b_s=ws,
                              flops=2.0 * M * N * Kd,
                              bytes=M * Kd + N * Kd + 4 * (xs.numel() + ws.numel()) + 2 * M * N))
    return cases


def bench_gemm(cases, steps, warmup):
    """Warm up, then time exactly `steps` steps between two synchronizes
    (the whole-job wall time: the launches back to back, nothing between
    them); then the same `steps` steps again with every launch bracketed by
    HIP events on its stream (per-launch kernel time for the roofline --
    an event record is a packet in the queue between two kernels, so that
    pass is not the one the wall time is taken from)."""
    from llm_from_scratch_amd import kernels as K
    fns = [lambda c=c: K.fp8_gemm(c["a"], c["a_s"], c["b"], c["b_s"]) for c in cases]
    for _ in range(warmup):
        for f in fns:
            f()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for r in range(steps):
        for f in fns:
            f()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    stream = torch.cuda.current_stream()
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(steps)] for _ in fns]
    for r in range(steps):
        for i, f in enumerate(fns):
            evs[i][r][0].record(stream)
            f()
            evs[i][r][1].record(stream)
    torch.cuda.synchronize()
    per = [sum(a.elapsed_time(b) for a, b in e) / steps / 1e3 for e in evs]
    return wall, per


def bench_vendor_gemm(device, reps):
    """Context for the headline, not a parity path: the vendor library's
    FP8 GEMM (torch._scaled_mm -> hipBLASLt) on the same six shapes and the
    same e4m3fn codes with one scale per tensor -- it has no per-128-block
    scale fold, the block-scaled GEMM's main extra cost."""
    from llm_from_scratch_amd import workloads as W
    rows = []
    tot_fl = tot_t = 0.0
    one = torch.ones((), dtype=torch.float32, device=device)
    for M in (4096, 16384):
        for Kd, N in W.GEMM_KN:
            a = torch.randn(M, Kd, device=device).to(torch.float8_e4m3fn)
            b = torch.randn(N, Kd, device=device).to(torch.float8_e4m3fn)
            f = lambda: torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
            f()
            torch.cuda.synchronize()
            ts = []
            for _ in range(reps):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                f()
                e1.record()
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1) / 1e3)
            t = sorted(ts)[len(ts) // 2]
            fl = 2.0 * M * N * Kd
            rows.append({"M": M, "K": Kd, "N": N, "us": t * 1e6, "TFLOP/s": fl / t / 1e12})
            tot_fl += fl
            tot_t += t
            del a, b
    return {"library": "hipBLASLt via torch._scaled_mm, per-tensor scales (no block scales)",
            "TFLOP/s": tot_fl / tot_t / 1e12, "frac": tot_fl / tot_t / 1e12 / FP8_PEAK_TFLOPS, "shapes": rows}


def bench_act_quant(device, reps, flush_buf):
    """act_quant over every cfg2 activation shape (M in {1, 16, 128, 4096,
    16384} x K in {1024, 4096, 2048}), the 512 MB flush before every call
    (16384 x 4096 is 134 MB and would sit in the Infinity Cache).
    Algorithmic bytes: 2 read + 1 written per element + 4 per 128-group."""
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd import workloads as W
    out = []
    for M in W.GEMM_M:
        for Kd in sorted({kd for kd, _ in W.GEMM_KN}):
            x = W.activation(M, Kd, seed=77 + M + Kd, device=device)
            K.act_quant(x)
            t = timed_launches([lambda: K.act_quant(x)], reps, flush=lambda: flush_buf.add_(1))[0]
            nbytes = 3 * M * Kd + 4 * M * Kd // 128
            out.append({"shape": [M, Kd], "us": t * 1e6, "GB/s": nbytes / t / 1e9,
                        "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "bytes": nbytes})
            del x
    prof = profile_figures("act_quant_16384x4096.md", "act_quant_16384x4096", "quant.hip")
    for o in out:
        if o["shape"] == [16384, 4096]:
            o["kernel_us_rocprof"] = prof.get("kernel_us", prof.get("stale"))
    return out


def bench_cfg1(device, reps):
    """cfg1 latency: one FP8 linear (act_quant of x [256, 512], fp8_gemm with
    the 128x128-quantised W [1344, 512]), inputs resident, no flush."""
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd import workloads as W
    x = W.activation(256, 512, seed=0, outliers=False, device=device)
    wq, ws = K.weight_quant(W.weight(1344, 512, seed=100, device=device))

    def fn():
        xq, xs = K.act_quant(x)
        return K.fp8_gemm(xq, xs, wq, ws)

    fn()
    t = timed_launches([fn], reps)[0]
    fl = 2.0 * 256 * 1344 * 512
    return {"shape": {"M": 256, "K": 512, "N": 1344}, "us": t * 1e6, "TFLOP/s": fl / t / 1e12,
            "launches": 2}


def bench_store_kvcache(device, reps, flush_buf):
    """store_kvcache of one decode step: cfg3 (64 tokens, 4 kv heads x 64)
    and cfg4 (256 tokens, 8 x 128) into the full pools at the decode slots.
    Algorithmic bytes: K and V rows read and written, slots read."""
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd import workloads as W
    out = []
    for name, seed in (("cfg3", 2), ("cfg4", 3)):
        case = W.paged_case(name, seed=seed)
        shape = (case.num_blocks, case.block_size, case.num_kv_heads, case.head_dim)
        kc = torch.empty(shape, dtype=torch.bfloat16, device=device)
        vc = torch.empty(shape, dtype=torch.bfloat16, device=device)
        g = torch.Generator(device=device).manual_seed(6)
        T = case.batch
        k = torch.randn(T, case.num_kv_heads, case.head_dim, generator=g, device=device).to(torch.bfloat16)
        v = torch.randn(T, case.num_kv_heads, case.head_dim, generator=g, device=device).to(torch.bfloat16)
        slots = torch.from_numpy(case.slot_mapping).to(device)
        fn = lambda: K.store_kvcache(k, v, kc, vc, slots)  # noqa: E731
        fn()
        t = timed_launches([fn], reps, flush=lambda: flush_buf.add_(1))[0]
        nbytes = 2 * (T * case.num_kv_heads * case.head_dim * 2) * 2 + 8 * T
        out.append({"config": name, "tokens": T, "us": t * 1e6, "GB/s": nbytes / t / 1e9,
                    "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "bytes": nbytes, "bound": "latency"})
        del kc, vc
        torch.cuda.empty_cache()
    return out


BF16_PEAK_TFLOPS = 2500.0


def bench_gemm_small(device, reps, flush_buf):
    """cfg2's decode-sized GEMMs (M in {1, 16, 128}): HBM/latency-bound, so
    reported as algorithmic bytes (A + B + scales read, C written) per second
    against the 8 TB/s roofline.  A call moves 0.5-12 MB in a few
    microseconds, about what the dispatch gap inside a HIP-event window
    around one call adds, so the calls run back to back as in a decode
    step: R >= 64 calls over R copies of the weights (more than 512 MB
    together, so the 256 MB Infinity Cache holds none of them when it is
    read again), captured in one HIP graph so that host dispatch does not
    pace them; events around a replay, per-call time = window / R (median of
    3 replays).  ``us_single`` is the event window around one eager call
    after a 512 MB cache-evicting write (launch gap included).  Default
    dispatch of kernels.fp8_gemm."""
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd import workloads as W
    out = []
    for M in (1, 16, 128):
        for Kd, N in W.GEMM_KN:
            x = W.activation(M, Kd, seed=1 + M + Kd, device=device)
            w = W.weight(N, Kd, seed=31 + Kd, device=device)
            xq, xs = K.act_quant(x)
            wq, ws = K.weight_quant(w)
            del w
            wbytes = wq.numel() + 4 * ws.numel()
            R = max(64, -(-(512 << 20) // wbytes))
            wqs = [wq.clone() for _ in range(R)]
            wss = [ws.clone() for _ in range(R)]
            fns = [lambda i=i: K.fp8_gemm(xq, xs, wqs[i], wss[i]) for i in range(R)]
            for f in fns[:4]:
                f()
            t1 = timed_launches([fns[0]], reps, flush=lambda: flush_buf.add_(1))[0]
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):
                for f in fns:
                    f()
            graph.replay()
            torch.cuda.synchronize()
            ts = []
            for _ in range(3):
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                graph.replay()
                e1.record()
                torch.cuda.synchronize()
                ts.append(e0.elapsed_time(e1) / 1e3 / R)
            del graph
            t = sorted(ts)[1]
            nbytes = M * Kd + N * Kd + 4 * (xs.numel() + ws.numel()) + 2 * M * N
            out.append({"M": M, "K": Kd, "N": N, "us": t * 1e6, "GB/s": nbytes / t / 1e9,
                        "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "TFLOP/s": 2.0 * M * N * Kd / t / 1e12,
                        "calls_back_to_back": R, "us_single": t1 * 1e6})
            del wqs, wss
            torch.cuda.empty_cache()
    return out


def bench_prefill(device, reps):
    """Varlen causal prefill attention at the cfg5 attention geometry (GQA
    12/4, D = 64): 16 whole prompts of 2048 tokens (keys just stored,
    contiguous), and 16 prompts of 2048 keys of which the first 1536 come
    from the prefix cache (paged keys, block 256, 512 new queries each).
    Algorithmic flop = 4 * D * Hq * (attended query-key pairs)."""
    from llm_from_scratch_amd import kernels as K
    Hq, Hkv, D, B, L, BS = 12, 4, 64, 16, 2048, 256
    g = torch.Generator(device=device).manual_seed(9)
    rnd = lambda *s: torch.randn(*s, generator=g, device=device).to(torch.bfloat16)
    res = []
    # whole prompts
    cu = torch.arange(0, (B + 1) * L, L, dtype=torch.int32, device=device)
    q, k, v = rnd(B * L, Hq, D), rnd(B * L, Hkv, D), rnd(B * L, Hkv, D)
    fn = lambda: K.flash_attn_varlen_func(q, k, v, cu, cu, L, L)  # noqa: E731
    fn()  # the first launch loads the kernel
    torch.cuda.synchronize()
    t = timed_launches([fn], reps)[0]
    pairs = B * L * (L + 1) // 2
    fl = 4 * D * Hq * pairs
    res.append({"case": f"{B} prompts x {L} tokens, contiguous keys", "us": t * 1e6, "TFLOP/s": fl / t / 1e12,
                "frac": fl / t / 1e12 / BF16_PEAK_TFLOPS, "flop": fl})
    del q, k, v
    # cached prefix: 1536 cached + 512 new tokens per sequence, keys from the pool
    lq = 512
    nb = L // BS
    kc, vc = rnd(B * nb, BS, Hkv, D), rnd(B * nb, BS, Hkv, D)
    bt = torch.randperm(B * nb, generator=g, device=device).to(torch.int32).view(B, nb).contiguous()
    cu_q = torch.arange(0, (B + 1) * lq, lq, dtype=torch.int32, device=device)
    q = rnd(B * lq, Hq, D)
    fn = lambda: K.flash_attn_varlen_func(q, kc, vc, cu_q, cu, lq, L, block_table=bt)  # noqa: E731
    fn()
    torch.cuda.synchronize()
    t = timed_launches([fn], reps)[0]
    pairs = B * (lq * (L - lq) + lq * (lq + 1) // 2)
    fl = 4 * D * Hq * pairs
    res.append({"case": f"{B} prompts x {L} keys, {L - lq} from the prefix cache (paged, block {BS})",
                "us": t * 1e6, "TFLOP/s": fl / t / 1e12, "frac": fl / t / 1e12 / BF16_PEAK_TFLOPS, "flop": fl})
    return res


def bench_indexer(device, reps):
    """DSA indexer score, fp8_index (model/attention/utils.py:175-250), at the
    lightning-indexer shape of 64 heads x 128 dims: one sequence of 4096
    queries against 4096 cached keys.  Algorithmic flop = 2*B*M*N*H*D (the
    q.k products; ReLU, weights and sums add 3*B*M*N*H)."""
    from llm_from_scratch_amd import kernels as K
    B, M, N, H, D = 1, 4096, 4096, 64, 128
    g = torch.Generator(device=device).manual_seed(10)
    q = (torch.randn(B, M, H, D, generator=g, device=device) * 16).to(torch.float8_e4m3fn)
    k = (torch.randn(B, N, D, generator=g, device=device) * 16).to(torch.float8_e4m3fn)
    qs = torch.rand(B, M, H, generator=g, device=device)
    ks = torch.rand(B, N, generator=g, device=device)
    fn = lambda: K.fp8_index(q, qs, k, ks)  # noqa: E731
    fn()  # the first launch loads the kernel
    torch.cuda.synchronize()
    t = timed_launches([fn], reps)[0]
    fl = 2 * B * M * N * H * D
    return {"shape": {"B": B, "M": M, "N": N, "H": H, "D": D}, "us": t * 1e6, "TFLOP/s": fl / t / 1e12,
            "frac": fl / t / 1e12 / FP8_PEAK_TFLOPS, "flop": fl}


def bench_moe(device, reps):
    """The MoE layer of cfg5 (d 768, d_ff 512, 8 routed experts top-2 + 1
    shared, random nn.Linear-init weights) over a prefill batch of 16384
    tokens, dispatched grouped (moe_route -> moe_align -> grouped w13 GEMM
    -> swiglu_quant -> grouped w2 GEMM -> moe_combine) and dense (every
    expert over every token).  Algorithmic flop = 2 * T * (top_k + S) *
    3 * d * d_ff (the picked experts' three projections)."""
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd.decode_model import DecodeModel, DecodeModelConfig
    cfg = DecodeModelConfig(vocab_size=256, num_layers=1, max_model_length=64)
    model = DecodeModel(cfg, device=device, seed=11)
    f = model.layers[0].ffn
    T = 16384
    g = torch.Generator(device=device).manual_seed(12)
    h = torch.randn(T, cfg.d_model, generator=g, device=device).to(torch.bfloat16)
    hq, hs = K.act_quant(h)
    kk = cfg.num_experts_per_tok + cfg.n_shared_experts
    fl = 2.0 * T * kk * 3 * cfg.d_model * cfg.d_ff
    out = {"tokens": T, "experts": [cfg.n_routed_experts, cfg.num_experts_per_tok, cfg.n_shared_experts],
           "d_model": cfg.d_model, "d_ff": cfg.d_ff, "flop": fl}
    with torch.no_grad():
        for mode in ("grouped", "dense"):
            f.dispatch = mode
            fn = lambda: f(h, hq, hs)  # noqa: E731
            fn()
            torch.cuda.synchronize()
            t = timed_launches([fn], reps)[0]
            out[mode] = {"us": t * 1e6, "TFLOP/s": fl / t / 1e12, "frac": fl / t / 1e12 / FP8_PEAK_TFLOPS}
    del model, f
    torch.cuda.empty_cache()
    return out


def _probe_lib():
    """The benchmark's read-ceiling library (llm_from_scratch_amd/csrc/
    probe.hip, built next to the kernel library), or None if absent."""
    import ctypes
    path = os.path.join(REPO, "llm_from_scratch_amd", "liblfs_probe.so")
    if not os.path.exists(path):
        return None
    lib = ctypes.CDLL(path)
    lib.lfs_probe_read_chunks.restype = ctypes.c_int
    lib.lfs_probe_read_chunks.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32,
                                          ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    return lib


def _decode_read_chunks(case, kc, vc, device):
    """4 KB chunks (absolute address, bytes) of every K and V row the decode
    reads: per (sequence, block) the block's valid rows, contiguous in the
    pool (rows of Hkv * D * 2 bytes)."""
    BS = case.block_size
    row = case.num_kv_heads * case.head_dim * 2
    lens = case.context_lens.astype(np.int64)
    nblk = -(-lens // BS)
    seq = np.repeat(np.arange(len(lens)), nblk)
    idx = np.arange(int(nblk.sum())) - np.repeat(np.cumsum(nblk) - nblk, nblk)
    blk = case.block_tables[seq, idx].astype(np.int64)
    seg_bytes = np.minimum(BS, lens[seq] - idx * BS) * row
    seg_off = blk * BS * row
    nch = -(-seg_bytes // 4096)
    cseg = np.repeat(np.arange(len(seg_bytes)), nch)
    cidx = np.arange(int(nch.sum())) - np.repeat(np.cumsum(nch) - nch, nch)
    off = seg_off[cseg] + cidx * 4096
    nbytes = np.minimum(4096, seg_bytes[cseg] - cidx * 4096).astype(np.uint32)
    addr = np.concatenate([kc.data_ptr() + off, vc.data_ptr() + off]).astype(np.uint64)
    nbytes = np.concatenate([nbytes, nbytes])
    return (torch.from_numpy(addr.view(np.int64)).to(device), torch.from_numpy(nbytes.view(np.int32)).to(device),
            int(nbytes.astype(np.int64).sum()))


def bench_read_rate(device, reps, flush_buf):
    """How fast workgroups of 256 threads stream from HBM as their number
    grows (the probe of liblfs_probe.so over a plain 512 MB buffer, 256 KB
    per workgroup, 16 loads of 16 bytes in flight per thread, cache flushed
    before every call): per-workgroup and whole-chip GB/s at 32 .. 2048
    workgroups (1/8 .. 8 per CU)."""
    probe = _probe_lib()
    if probe is None:
        return {"error": "liblfs_probe.so not built"}
    buf = torch.empty(512 << 20, dtype=torch.uint8, device=device)
    per_group = 256 << 10
    out = []
    for groups in (32, 64, 128, 256, 512, 1024, 2048):
        n = groups * per_group // 4096
        if n * 4096 > buf.numel():
            break
        addr = torch.from_numpy((buf.data_ptr() + np.arange(n, dtype=np.int64) * 4096).view(np.int64)).to(device)
        nb = torch.full((n,), 4096, dtype=torch.int32, device=device)
        sink = torch.empty(groups * 256, dtype=torch.float32, device=device)

        def read():
            rc = probe.lfs_probe_read_chunks(addr.data_ptr(), nb.data_ptr(), n, groups, 16, sink.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream)
            assert rc == 0, f"read probe: {rc}"

        read()
        torch.cuda.synchronize()
        t = timed_launches([read], reps, flush=lambda: flush_buf.add_(1))[0]
        out.append({"workgroups": groups, "bytes": n * 4096, "us": t * 1e6, "GB/s": n * 4096 / t / 1e9,
                    "GB/s per workgroup": per_group / t / 1e9})
    del buf
    torch.cuda.empty_cache()
    return out


def bench_decode(name, device, reps, flush_buf):
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd import workloads as W
    case = W.paged_case(name, seed=3 if name == "cfg4" else 2)
    kc, vc = W.fill_pool(case, seed=2, device=device, only_referenced=(name == "cfg4"))
    g = torch.Generator(device=device).manual_seed(5)
    q = torch.randn(case.batch, case.num_q_heads, case.head_dim, generator=g, device=device,
                    dtype=torch.bfloat16)
    cl = torch.from_numpy(case.context_lens).to(device)
    bt = torch.from_numpy(case.block_tables).to(device)
    bps = K.default_blocks_per_split(case.batch, case.num_kv_heads, bt.shape[1], case.block_size)
    ws = torch.empty(K.paged_decode_workspace_bytes(case.batch, case.num_q_heads, case.head_dim,
                                                    bt.shape[1], bps), dtype=torch.uint8, device=device)
    fn = lambda: K.paged_attention_decode(q, kc, vc, cl, bt, case.scale, bps, ws)  # noqa: E731
    fn()
    torch.cuda.synchronize()
    t = timed_launches([fn], reps, flush=lambda: flush_buf.add_(1))[0]
    nbytes = case.kv_bytes()
    out = {"config": name, "batch": case.batch, "heads": [case.num_q_heads, case.num_kv_heads],
           "head_dim": case.head_dim, "tokens": int(case.context_lens.sum()), "us": t * 1e6,
           "GB/s": nbytes / t / 1e9, "frac": nbytes / t / 1e9 / HBM_PEAK_GBS, "bytes": nbytes,
           "blocks_per_split": bps}
    # the read ceiling at this size: the same K / V bytes read once with
    # nothing computed (liblfs_probe.so), timed the same way
    probe = _probe_lib()
    if probe is not None:
        addr, nb, read_bytes = _decode_read_chunks(case, kc, vc, device)
        n = addr.numel()
        groups = max(1024, -(-n // 1024))
        sink = torch.empty(groups * 256, dtype=torch.float32, device=device)

        def read():
            rc = probe.lfs_probe_read_chunks(addr.data_ptr(), nb.data_ptr(), n, groups, 16, sink.data_ptr(),
                                             torch.cuda.current_stream().cuda_stream)
            assert rc == 0, f"read probe: {rc}"

        read()
        torch.cuda.synchronize()
        tr = timed_launches([read], reps, flush=lambda: flush_buf.add_(1))[0]
        out["read_ceiling"] = {"us": tr * 1e6, "bytes": read_bytes, "GB/s": read_bytes / tr / 1e9,
                               "frac": read_bytes / tr / 1e9 / HBM_PEAK_GBS, "decode_vs_read": tr / t}
    # split + merge kernel time and fabric bytes of the same call from the
    # rocprofv3 summary (the event window also holds the launch gap)
    prof = profile_figures("paged_decode_cfg3_cfg4.md", "paged_decode_" + name, "paged_kv.hip")
    if "stale" in prof:
        out["rocprof"] = prof
    else:
        out["kernel_us_rocprof"] = prof["kernel_us"]
        out["kernel_frac"] = nbytes / (prof["kernel_us"] * 1e-6) / 1e9 / HBM_PEAK_GBS
        out["traffic"] = prof.get("traffic")
    del kc, vc
    torch.cuda.empty_cache()
    return out


def bench_decode_step(device, reps):
    """cfg5: one graph-captured decode step (12-layer GQA + MoE model, FP8
    linears, paged KV) for 128 sequences with contexts U{256..2048}, plus
    lm_head and Gumbel-max sampling.  Synthetic KV (random pool contents),
    random-init weights."""
    from llm_from_scratch_amd.decode_model import DecodeModel, DecodeModelConfig
    from llm_from_scratch_amd.engine import ModelRunner, Sequence
    from llm_from_scratch_amd.fp8_linear import FP8Linear
    cfg = DecodeModelConfig()
    BS, B = 256, 128
    rng = np.random.default_rng(4)
    lens = rng.integers(256, 2049, B)
    nblk = (lens + BS - 1) // BS
    total = int(nblk.sum())
    Sequence.block_size = BS
    model = DecodeModel(cfg, device=device, seed=4)
    runner = ModelRunner(model, cfg.runner_config(block_size=BS, num_kv_blocks=total, max_num_seqs=B))
    runner.kv_cache.normal_(generator=torch.Generator(device=device).manual_seed(4))
    perm = rng.permutation(total)
    seqs, off = [], 0
    for L, n in zip(lens, nblk):
        s = Sequence(rng.integers(0, cfg.vocab_size, int(L)).tolist())
        s.block_table = perm[off:off + n].tolist()
        off += n
        seqs.append(s)
    ids, pos = runner.prepare_decode(seqs)
    temps = runner.prepare_sample(seqs)
    runner.run_model(ids, pos, False)  # fills the static graph inputs
    graph = runner.graphs[B]
    gen = torch.Generator(device=device).manual_seed(0)

    def step():
        graph.replay()
        return runner.sampler(runner.graph_logits(B), temps, gen)

    for _ in range(3):
        step()
    t = timed_launches([step], reps)[0]
    w_bytes = sum(m.weight.numel() + 4 * m.weight_scale.numel() + (4 * m.bias.numel() if m.bias is not None else 0)
                  for m in model.modules() if isinstance(m, FP8Linear))
    kv = int(lens.sum()) * cfg.num_layers * cfg.num_kv_heads * cfg.head_dim * 2 * 2
    nbytes = w_bytes + kv
    out = {"config": "cfg5", "batch": B, "context_tokens": int(lens.sum()), "ms": t * 1e3,
           "tokens/s": B / t, "bytes": nbytes, "weight_bytes": w_bytes, "kv_bytes": kv,
           "GB/s": nbytes / t / 1e9, "frac": nbytes / t / 1e9 / HBM_PEAK_GBS,
           "graph_kernels_note": "decode step captured in one HIP graph; lm_head + sampler eager"}
    del runner, model
    torch.cuda.empty_cache()
    return out


def _median_time(fn, runs: int, warmup: int = 1) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def _cpu_act_quant(x):
    """act_quant in torch CPU ops, the formula of oracle.fp8.act_quant
    (model/attention/utils.py:129-139): amax per 128-group, clamp 1e-4,
    times fp32(1/448), IEEE divide, clamp +-448, RNE cast to e4m3fn."""
    g = x.float().view(x.shape[0], -1, 128)
    s = g.abs().amax(-1).clamp_min(1e-4) * torch.tensor(1.0 / 448.0, dtype=torch.float32)
    y = (g / s[..., None]).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return y.view(x.shape), s


def _cpu_decode(q, kc, vc, lens, bt, scale, BS):
    """Paged GQA decode in torch CPU fp32: gather each sequence's K/V rows
    through its block table, softmax(scale q K^T) V per kv head (the math of
    oracle.paged_kv.paged_decode, model/attention/GQA.py:118-130)."""
    B, Hq, D = q.shape
    Hkv = kc.shape[2]
    G = Hq // Hkv
    o = torch.zeros(B, Hq, D)
    for b in range(B):
        L = int(lens[b])
        nb = -(-L // BS)
        blocks = torch.from_numpy(bt[b, :nb].astype(np.int64))
        Kb = kc[blocks].reshape(-1, Hkv, D)[:L].float().permute(1, 2, 0)  # [Hkv, D, L]
        Vb = vc[blocks].reshape(-1, Hkv, D)[:L].float().permute(1, 0, 2)  # [Hkv, L, D]
        qh = q[b].float().view(Hkv, G, D)
        p = torch.softmax(torch.matmul(qh, Kb) * scale, dim=-1)
        o[b] = torch.matmul(p, Vb).reshape(Hq, D)
    return o


def _compact_case(name, seed, nseq=None):
    """cfg3 / cfg4 metadata with the pool compacted to the referenced blocks
    (tables remapped), K/V ~N(0,1) bf16 on the host."""
    from llm_from_scratch_amd import workloads as W
    case = W.paged_case(name, seed=seed)
    lens = case.context_lens[:nseq] if nseq else case.context_lens
    bt = case.block_tables[:len(lens)]
    used = np.unique(bt[bt >= 0])
    remap = np.full(case.num_blocks, -1, np.int64)
    remap[used] = np.arange(len(used))
    bt_c = np.where(bt >= 0, remap[np.maximum(bt, 0)], -1)
    g = torch.Generator().manual_seed(seed)
    shape = (len(used), case.block_size, case.num_kv_heads, case.head_dim)
    kc = torch.randn(shape, generator=g).to(torch.bfloat16)
    vc = torch.randn(shape, generator=g).to(torch.bfloat16)
    q = torch.randn(len(lens), case.num_q_heads, case.head_dim, generator=g).to(torch.bfloat16)
    return case, lens, bt_c, kc, vc, q


def _cfg5_cpu_weights(dims, seed):
    """Random weights of the cfg5 model in the reference's state-dict layout
    (the names oracle.model reads), fp32 on the host.  Every projection
    weight is an FP8 weight: random finite e4m3fn codes times one scale per
    128x128 block (1 / (448 sqrt(fan_in)) times a random factor in [0.5, 1]),
    decoded exactly and stored transposed for x @ W; biases uniform in
    +-1/sqrt(fan_in), norms in [0.5, 1.5], the gate bf16-valued, the expert
    bias in +-0.5."""
    g = torch.Generator().manual_seed(seed)
    d, Fd, V, E = dims.d_model, dims.d_ff, dims.vocab_size, dims.n_routed_experts
    kv = dims.num_kv_heads * dims.head_dim
    w = {}

    def uni(name, shape, lo, hi):
        w[name] = lo + (hi - lo) * torch.rand(shape, generator=g)

    def lin(name, n_out, n_in):
        # random bytes read as e4m3fn codes (the two NaN codes count as 0)
        codes = torch.empty(n_out * n_in // 4, dtype=torch.int32).random_(generator=g).view(torch.uint8)
        vals = torch.nan_to_num_(codes.view(torch.float8_e4m3fn).float(), nan=0.0).view(n_out, n_in)
        sc = (0.5 + 0.5 * torch.rand(-(-n_out // 128), n_in // 128, generator=g)) / (448.0 * math.sqrt(n_in))
        sc = sc.repeat_interleave(128, 0)[:n_out].repeat_interleave(128, 1)
        w[name + ".weight"] = (vals * sc).t().contiguous()
        uni(name + ".bias", (n_out,), -1 / math.sqrt(n_in), 1 / math.sqrt(n_in))

    def mlp(name):
        lin(name + ".w1", Fd, d)
        lin(name + ".w3", Fd, d)
        lin(name + ".w2", d, Fd)

    uni("token_embeddings.weight", (V, d), -math.sqrt(3.0), math.sqrt(3.0))
    for i in range(dims.num_layers):
        p = f"layers.{i}."
        lin(p + "att.q_proj", d, d)
        lin(p + "att.k_proj", kv, d)
        lin(p + "att.v_proj", kv, d)
        lin(p + "att.output_proj", d, d)
        uni(p + "att.q_norm.weight", (d,), 0.5, 1.5)
        uni(p + "att.k_norm.weight", (kv,), 0.5, 1.5)
        for e in range(E):
            mlp(p + f"ffn.experts.{e}")
        mlp(p + "ffn.shared_expert")
        uni(p + "ffn.gate.weight", (E, d), -1 / math.sqrt(d), 1 / math.sqrt(d))
        w[p + "ffn.gate.weight"] = w[p + "ffn.gate.weight"].to(torch.bfloat16).float()
        uni(p + "ffn.gate.expert_bias", (E,), -0.5, 0.5)
        uni(p + "att_norm.weight", (d,), 0.5, 1.5)
        uni(p + "ffn_norm.weight", (d,), 0.5, 1.5)
    uni("final_norm.weight", (d,), 0.5, 1.5)
    lin("lm_head", V, d)
    return w


def _cpu_fp8_linear(w):
    """The FP8 linear in torch CPU ops: dequant(act_quant(x)) @ dequant(W)^T
    + b, rounded to bf16 (the product FP8Linear's arithmetic up to fp32
    summation order)."""
    def linear(p, x):
        xq, xs = _cpu_act_quant(x.to(torch.bfloat16))
        xd = (xq.float().view(x.shape[0], -1, 128) * xs[..., None]).view(x.shape[0], -1)
        y = xd @ w[p + ".weight"]
        b = w.get(p + ".bias")
        return (y if b is None else y + b).to(torch.bfloat16)
    return linear


def _cpu_decode_step_baseline(nseq, runs):
    """cfg5 decode step on the host: oracle/model.py's decoder block
    (model/transformer.py:90-118, 162-183) with the FP8-emulating linear,
    each layer storing the new token's K/V at its slot and attending over the
    sequence's context in torch CPU fp32 (paged, compacted pool per layer),
    then final norm, lm_head and Gumbel-max sampling (utils/sampler.py:35-53)
    -- for the first `nseq` sequences of the GPU line's batch (same length
    draw), random weights and KV."""
    from oracle import model as om
    dims = om.ModelDims(32000, 768, 12, 12, 4, 512, 8, 2, 1)
    w = _cfg5_cpu_weights(dims, seed=4)
    BS, Hkv, D, Hq = 256, dims.num_kv_heads, dims.head_dim, dims.num_heads
    G = Hq // Hkv
    rng = np.random.default_rng(4)
    lens = rng.integers(256, 2049, 128)[:nseq]  # the draw of bench_decode_step
    nblk = -(-lens // BS)
    total = int(nblk.sum())
    perm = rng.permutation(total)
    bt = np.full((nseq, 16), -1, np.int64)
    off = 0
    for b in range(nseq):
        bt[b, :nblk[b]] = perm[off:off + nblk[b]]
        off += nblk[b]
    g = torch.Generator().manual_seed(4)
    shape = (total, BS, Hkv, D)
    base = torch.randn(shape, generator=g).to(torch.bfloat16)  # every layer's K and V pool starts as a copy
    pools = [(base.clone(), base.clone()) for _ in range(dims.num_layers)]
    tokens = torch.from_numpy(rng.integers(0, dims.vocab_size, nseq))
    pos = torch.from_numpy(lens - 1)
    slots = torch.from_numpy(bt[np.arange(nseq), (lens - 1) // BS] * BS + (lens - 1) % BS)
    blocks = [torch.from_numpy(bt[b, :nblk[b]]) for b in range(nseq)]
    linear = _cpu_fp8_linear(w)
    scale = 1.0 / math.sqrt(D)

    def step():
        x = w["token_embeddings.weight"][tokens].to(torch.bfloat16)
        residual = None
        for i in range(dims.num_layers):
            kc, vc = pools[i]

            def attend(q, k, v):
                kc.view(-1, Hkv, D)[slots] = k
                vc.view(-1, Hkv, D)[slots] = v
                o = torch.empty(nseq, Hq, D)
                for b in range(nseq):
                    L = int(lens[b])
                    kb = kc[blocks[b]].reshape(-1, Hkv, D)[:L].float().permute(1, 2, 0)
                    vb = vc[blocks[b]].reshape(-1, Hkv, D)[:L].float().permute(1, 0, 2)
                    p = torch.softmax(torch.matmul(q[b].float().view(Hkv, G, D), kb) * scale, dim=-1)
                    o[b] = torch.matmul(p, vb).reshape(Hq, D)
                return o.view(nseq, -1)
            x, residual = om.block(w, i, x, residual, pos, dims, linear, attend)
        h, _ = om.rms_norm(x, w["final_norm.weight"], dims.rms_eps, residual)
        probs = torch.softmax(linear("lm_head", h).float(), -1)
        return (probs / torch.empty_like(probs).exponential_(1).clamp_min(1e-10)).argmax(-1)

    t = _median_time(step, runs)
    return {"config": "cfg5", "sample": f"first {nseq} of the 128 sequences ({int(lens.sum())} context tokens), "
                                        f"random weights and KV, median of {runs}",
            "batch": nseq, "ms": t * 1e3, "tokens/s": nseq / t}


def _cpu_cfg1_baseline(runs):
    """cfg1 FP8 linear on the host: act_quant (torch CPU ops) of x [256, 512]
    then the numpy oracle's blockwise fp32 fp8_gemm with W [1344, 512]
    (128x128 scales) -- the latency the GPU line cfg1_linear reports."""
    from oracle import fp8 as F
    from llm_from_scratch_amd import workloads as W
    x = torch.randn(256, 512, generator=torch.Generator().manual_seed(0)).to(torch.bfloat16)
    b, b_s = F.weight_quant(W.weight(1344, 512, seed=0).float().numpy())

    def fn():
        xq, xs = _cpu_act_quant(x)
        return F.fp8_gemm(xq.view(torch.uint8).numpy(), xs.numpy(), b, b_s, accum=np.float32)

    t = _median_time(fn, runs)
    return {"shape": {"M": 256, "K": 512, "N": 1344}, "us": t * 1e6,
            "TFLOP/s": 2.0 * 256 * 512 * 1344 / t / 1e12, "runs": runs}


def cpu_baseline(device):
    """CPU restatements on all host cores (1 warm-up, median of 5; 3 for
    cfg4 and the cfg5 step): the headline is the numpy oracle's blockwise
    fp32 GEMM on the three cfg2 M=4096 shapes; act_quant, paged decode and
    store_kvcache run the same formulas in torch CPU ops; cfg1 is act_quant
    plus the oracle's GEMM at 256x512x1344; decode_step is the cfg5 step
    (oracle/model.py's blocks with FP8-emulating linears, paged attention,
    lm_head, Gumbel-max) on the first 32 of its 128 sequences.  The act_quant
    codes and the decode output are checked against the GPU on the same
    inputs (bit-exact codes; decode within the 1e-2 / 2e-2 bar)."""
    from threadpoolctl import threadpool_limits
    from oracle import fp8 as F
    from llm_from_scratch_amd import kernels as K
    from llm_from_scratch_amd import workloads as W
    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    t_start = time.perf_counter()
    out = {"unit": "TFLOP/s", "cores": cores, "kind": "port"}
    flops, secs = 0.0, 0.0
    with threadpool_limits(cores):
        for Kd, N in W.GEMM_KN:
            M = 4096
            a, a_s = F.act_quant(W.activation(M, Kd, seed=1 + M + Kd).float().numpy())
            b, b_s = F.weight_quant(W.weight(N, Kd, seed=31 + Kd).float().numpy())
            secs += _median_time(lambda: F.fp8_gemm(a, a_s, b, b_s, accum=np.float32), 5)
            flops += 2.0 * M * N * Kd
    out["value"] = flops / secs / 1e12
    out["gemm_s_per_step"] = secs

    # act_quant: 2048 x 4096 rows of the cfg2 activation (1/8 of the GPU line's 16384 rows)
    x = W.activation(2048, 4096, seed=78)
    t = _median_time(lambda: _cpu_act_quant(x), 5)
    nbytes = 3 * x.numel() + 4 * x.numel() // 128
    yc, sc = _cpu_act_quant(x)
    yg, sg = K.act_quant(x.to(device))
    same = bool(torch.equal(yc.view(torch.uint8), yg.view(torch.uint8).cpu()) and torch.equal(sc, sg.cpu()))
    out["act_quant"] = {"sample": "2048x4096 (GPU line: up to 16384x4096)", "GB/s": nbytes / t / 1e9,
                        "s": t, "codes_equal_gpu": same}

    # paged decode: cfg3 whole batch; cfg4 its first 16 sequences (compacted pools)
    out["paged_decode"] = []
    for name, seed, nseq, runs in (("cfg3", 2, None, 5), ("cfg4", 3, 16, 3)):
        case, lens, bt, kc, vc, q = _compact_case(name, seed, nseq)
        t = _median_time(lambda: _cpu_decode(q, kc, vc, lens, bt, case.scale, case.block_size), runs)
        nbytes = int(lens.sum()) * case.num_kv_heads * case.head_dim * 2 * 2 + \
            2 * len(lens) * case.num_q_heads * case.head_dim * 2 + 4 * bt.size + 8 * len(lens)
        ref = _cpu_decode(q, kc, vc, lens, bt, case.scale, case.block_size)
        dev_bt = torch.from_numpy(bt.astype(np.int32)).to(device)
        got = K.paged_attention_decode(q.to(device), kc.to(device), vc.to(device),
                                       torch.from_numpy(lens.astype(np.int64)).to(device), dev_bt, case.scale)
        err = (got.float().cpu() - ref).abs()
        ok = bool((err <= 2e-2 + 1e-2 * ref.abs()).all())
        out["paged_decode"].append({"config": name, "sample": f"{len(lens)} sequences, {int(lens.sum())} tokens",
                                    "GB/s": nbytes / t / 1e9, "s": t, "runs": runs, "matches_gpu": ok})
        del kc, vc

    # store_kvcache: cfg3's 64 decode slots into the compacted cfg3 pool (index_copy_)
    case, lens, bt, kc, vc, q = _compact_case("cfg3", 2)
    slots = torch.from_numpy((bt[np.arange(len(lens)), (lens - 1) // case.block_size] * case.block_size
                              + (lens - 1) % case.block_size).astype(np.int64))
    kf, vf = kc.view(-1, case.num_kv_heads, case.head_dim), vc.view(-1, case.num_kv_heads, case.head_dim)
    kn, vn = q[:, :case.num_kv_heads].contiguous(), q[:, case.num_kv_heads:2 * case.num_kv_heads].contiguous()

    def store():
        for _ in range(100):
            kf.index_copy_(0, slots, kn)
            vf.index_copy_(0, slots, vn)

    t = _median_time(store, 5) / 100
    nbytes = 2 * kn.numel() * 2 * 2 + 8 * len(slots)
    out["store_kvcache"] = {"config": "cfg3", "tokens": len(slots), "us": t * 1e6, "GB/s": nbytes / t / 1e9}
    out["cfg1"] = _cpu_cfg1_baseline(5)
    out["decode_step"] = _cpu_decode_step_baseline(32, 3)
    out["sample"] = ("GEMM: numpy oracle fp8_gemm (blockwise fp32) on cfg2 M=4096 x 3 (K,N), median of 5; "
                     f"{time.perf_counter() - t_start:.1f} s of CPU baselines in total")
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-extra", action="store_true", help="skip decode / act_quant lines")
    ap.add_argument("--extras",
                    default="vendor,cfg1,act_quant,gemm_small,store_kvcache,cfg3,cfg3_4k,cfg4,prefill,indexer,moe,cfg5",
                    help="comma list of extra lines: vendor (hipBLASLt per-tensor FP8 GEMM on the headline "
                         "shapes, for context), cfg1 (FP8 linear latency), act_quant (every cfg2 "
                         "shape), gemm_small (cfg2 M <= 128), store_kvcache, cfg3, cfg3_4k, cfg4 (paged "
                         "decode), prefill (varlen prefill attention), indexer (DSA fp8_index), moe (MoE "
                         "layer, grouped vs dense dispatch), cfg5 (decode step); not in the default list: "
                         "read_rate (HBM read rate per workgroup at 32-2048 workgroups)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run 4 plain device copies of 256 MiB (a known-traffic kernel for "
                         "scaling FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    dev = "cuda:0"
    torch.cuda.set_device(0)
    extras = set() if args.no_extra else set(e for e in args.extras.split(",") if e)
    if args.copy_calibration:
        src = torch.empty(256 * 1024 * 1024, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    log("bench: setting up fp8_gemm inputs")
    cases = gemm_setup(dev)
    log("bench: timing fp8_gemm")
    wall, per = bench_gemm(cases, args.steps, args.warmup)
    total_flops = sum(c["flops"] for c in cases)
    kern_time = sum(per)
    achieved = total_flops / kern_time / 1e12
    shapes = [{"M": c["M"], "K": c["K"], "N": c["N"], "us": t * 1e6,
               "TFLOP/s": c["flops"] / t / 1e12, "frac": c["flops"] / t / 1e12 / FP8_PEAK_TFLOPS}
              for c, t in zip(cases, per)]
    alg_bytes = sum(c["bytes"] for c in cases) / len(cases)
    # fabric bytes per launch (average over the six launches) from the PMC
    # runs summarised in profiles/, if measured on the kernel source built
    gprof = profile_figures("fp8_gemm_cfg2_sweep.md", "fp8_gemm_cfg2", "fp8_gemm.hip")
    del cases
    torch.cuda.empty_cache()
    out = {
        "metric": METRIC,
        "value": total_flops / wall / 1e12,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": wall * 1e3,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3",
        "data": "synthetic",
        "config": {"workload": "cfg2 fp8_gemm sweep: M in {4096,16384} x (K,N) in "
                               "{(1024,4096),(4096,1024),(2048,5632)}, 1x128 act / 128x128 weight "
                               "e4m3fn scales, bf16 out",
                   "launches_per_step": len(per)},
        "roofline": {"bound": "mfma", "kernel": "fp8_gemm", "achieved": achieved,
                     "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": achieved / FP8_PEAK_TFLOPS,
                     "traffic": gprof.get("traffic"),
                     "algorithmic_bytes": alg_bytes},
        "gemm_shapes": shapes,
    }
    if "stale" in gprof:
        out["roofline"]["traffic_note"] = gprof["stale"]
    else:
        out["roofline"]["kernel_us_rocprof"] = gprof.get("kernel_us")
    try:
        decode = [n for n in ("cfg3", "cfg3_4k", "cfg4") if n in extras]
        flushed = decode or extras & {"act_quant", "gemm_small", "store_kvcache", "read_rate"}
        if flushed:
            flush_buf = torch.empty(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev).zero_()
        if "vendor" in extras:
            log("bench: vendor FP8 GEMM (per-tensor scales)")
            try:
                out["vendor_fp8_gemm"] = bench_vendor_gemm(dev, 20)
            except Exception as e:  # noqa: BLE001 -- a missing vendor kernel is reported, not fatal
                out["vendor_fp8_gemm"] = {"error": repr(e)[:300]}
        if "cfg1" in extras:
            log("bench: cfg1 FP8 linear latency")
            out["cfg1_linear"] = bench_cfg1(dev, 20)
        if "act_quant" in extras:
            log("bench: act_quant")
            out["act_quant"] = bench_act_quant(dev, 20, flush_buf)
        if "gemm_small" in extras:
            log("bench: fp8_gemm at M <= 128")
            out["gemm_small"] = bench_gemm_small(dev, 20, flush_buf)
        if "read_rate" in extras:
            log("bench: HBM read rate per workgroup")
            out["read_rate"] = bench_read_rate(dev, 10, flush_buf)
        if "store_kvcache" in extras:
            log("bench: store_kvcache")
            out["store_kvcache"] = bench_store_kvcache(dev, 20, flush_buf)
        if decode:
            out["paged_decode"] = []
            for name in decode:
                log(f"bench: paged decode {name}")
                out["paged_decode"].append(bench_decode(name, dev, 20, flush_buf))
            c3 = [d for d in out["paged_decode"] if d["config"] == "cfg3"]
            if c3:  # the decode half of the metric: cfg3 against 8 TB/s
                d = c3[0]
                out["roofline_decode"] = {"bound": "hbm", "kernel": "paged_decode (split + merge)",
                                          "workload": "cfg3", "achieved": d["GB/s"], "peak": HBM_PEAK_GBS,
                                          "unit": "GB/s", "frac": d["frac"], "traffic": d.get("traffic"),
                                          "algorithmic_bytes": d["bytes"],
                                          "kernel_us_rocprof": d.get("kernel_us_rocprof"),
                                          "kernel_frac": d.get("kernel_frac")}
        if flushed:
            del flush_buf
            torch.cuda.empty_cache()
        if "indexer" in extras:
            log("bench: fp8_index")
            out["fp8_index"] = bench_indexer(dev, 10)
        if "moe" in extras:
            log("bench: MoE layer (grouped / dense dispatch)")
            out["moe_layer"] = bench_moe(dev, 10)
        if "prefill" in extras:
            log("bench: prefill attention")
            out["prefill_attention"] = bench_prefill(dev, 10)
        if "cfg5" in extras:
            log("bench: cfg5 decode step")
            out["decode_step"] = bench_decode_step(dev, 20)
    except Exception as e:  # report, keep the headline line
        out["extra_error"] = repr(e)
    if not args.no_cpu:
        log("bench: cpu baseline")
        out["cpu_baseline"] = cpu_baseline(dev)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()

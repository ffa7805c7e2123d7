"""MoE expert dispatch (HIP) against the CPU oracle.

Bars: moe_align bit-exact (integer layout and copied weights);
fp8_grouped_gemm within 1e-2 relative / 2e-2 absolute of the float64 oracle
(bf16 output) or 1e-4 relative to the row's largest value (fp32 output:
the activation codes span the whole e4m3 range, and products up to 2e5
summed inside the MFMA do not round like a sequential fp32 sum), and
bit-identical to fp8_gemm on the gathered rows (both run the same MFMA and
fold sequence per 128x128 tile); moe_combine within one bf16 rounding of the
float64 sum; segment_reduce_weighted / fused_scatter_add_weighted within one
rounding of the output dtype; the grouped MoE layer within 1e-2 of the
dense-dispatch layer, and as close as it, row by row, to the fp32 torch
restatement of moe_infer (99% of rows within 1e-2).
Cases: cfg5's 8 experts top-2 + 1 shared, 64 experts top-6, token counts
across tile edges (1, 127, 128, 129, 1000), dropped (-1 / out-of-range)
picks, strided per-expert weight views, bf16 and fp32 inputs.
"""
import numpy as np
import pytest
import torch

from llm_from_scratch_amd import kernels as K
from oracle import fp8 as F
from oracle import moe as MO

pytestmark = pytest.mark.gpu
DEV = "cuda"


def picks(rng, T, E, k, bad=0):
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int64)
    w = rng.uniform(0.05, 1.0, (T, k)).astype(np.float32)
    for _ in range(bad):
        idx[rng.integers(T), rng.integers(k)] = rng.choice([-1, E, E + 7])
    return idx, w


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV)


def fp8(x):
    return dev(x).view(torch.float8_e4m3fn)


@pytest.mark.parametrize("T,E,k,S,bad", [(1, 8, 2, 1, 0), (127, 8, 2, 1, 0), (129, 8, 2, 1, 4),
                                         (1000, 8, 2, 1, 0), (3000, 64, 6, 0, 9), (128, 4, 1, 2, 0)])
def test_moe_align_exact(T, E, k, S, bad):
    rng = np.random.default_rng(T + E)
    idx, w = picks(rng, T, E, k, bad)
    rows = K.moe_align(dev(idx), dev(w), E, S)
    rt, rw, te, er = MO.moe_align(idx, w, E, S)
    np.testing.assert_array_equal(rows.tile_expert.cpu().numpy(), te)
    np.testing.assert_array_equal(rows.row_token.cpu().numpy(), rt)
    np.testing.assert_array_equal(rows.row_weight.cpu().numpy(), rw)
    np.testing.assert_array_equal(rows.entry_row.cpu().numpy(), er)


def expert_stack(rng, E, N, Kd):
    """Per-expert weights quantised 128x128 like FP8Linear, stacked [E, N, K]."""
    w = rng.standard_normal((E, N, Kd)).astype(np.float32) * 0.05
    q, s = zip(*(F.weight_quant(w[e]) for e in range(E)))
    return np.stack(q), np.stack(s)


def test_grouped_gemm_gather_bias_and_fp32():
    rng = np.random.default_rng(5)
    T, E, k, S, N, Kd = 300, 6, 2, 1, 320, 384
    idx, w = picks(rng, T, E, k)
    x = rng.standard_normal((T, Kd)).astype(np.float32)
    xq, xs = F.act_quant(x)
    bq, bs = expert_stack(rng, E + S, N, Kd)
    bias = rng.standard_normal((E + S, N)).astype(np.float32)
    rows = K.moe_align(dev(idx), dev(w), E, S)
    rt, _, te, _ = MO.moe_align(idx, w, E, S)
    c = K.fp8_grouped_gemm(fp8(xq), dev(xs), rows.row_token, rows.tile_expert, fp8(bq), dev(bs), dev(bias))
    ref = MO.grouped_gemm(xq, xs, rt, te, bq, bs, bias, round_bf16=False)
    used = np.repeat(te >= 0, 128)
    got = c.float().cpu().numpy()[used]
    err = np.abs(got - ref[used])
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref[used])), f"bf16 out: worst {err.max():.3g}"
    c32 = K.fp8_grouped_gemm(fp8(xq), dev(xs), rows.row_token, rows.tile_expert, fp8(bq), dev(bs),
                             out_dtype=torch.float32)
    ref32 = MO.grouped_gemm(xq, xs, rt, te, bq, bs, round_bf16=False)[used]
    got32 = c32.cpu().numpy()[used]
    scale = np.abs(ref32).max(1, keepdims=True) + 1e-30
    assert np.all(np.abs(got32 - ref32) <= 1e-4 * scale), "fp32 out"
    # bit-identical to the dense tile kernel on the gathered rows of each used
    # tile (129 rows, so that the dense call takes the 128 x 128 tile kernel
    # and not the one-shot kernel of M <= 128, which sums K in another order)
    for i in np.nonzero(te >= 0)[0][:4]:
        src = np.maximum(rt[i * 128:(i + 1) * 128], 0)
        src = np.concatenate([src, src[:1]])
        e = te[i]
        dense = K.fp8_gemm(fp8(xq[src]), dev(xs[src]), fp8(bq[e]), dev(bs[e]), dev(bias[e]), splits=1)[:128]
        assert torch.equal(dense, c[i * 128:(i + 1) * 128]), f"tile {i} differs from fp8_gemm"


def test_grouped_gemm_k_stacked_view():
    """The down projection's layout: experts stacked along K of one
    [N, E*F] matrix, viewed [E, N, F] (strides F, E*F, 1); identity rows."""
    rng = np.random.default_rng(6)
    E, N, Fd, tiles = 4, 256, 256, 3
    wfull = rng.standard_normal((N, E * Fd)).astype(np.float32) * 0.05
    wq, ws = F.weight_quant(wfull)
    a = rng.standard_normal((tiles * 128, Fd)).astype(np.float32)
    aq, as_ = F.act_quant(a)
    te = np.array([3, 0, 2], np.int32)
    bview = fp8(wq).view(N, E, Fd).permute(1, 0, 2)
    sview = dev(ws).view(N // 128, E, Fd // 128).permute(1, 0, 2)
    c = K.fp8_grouped_gemm(fp8(aq), dev(as_), None, dev(te), bview, sview, out_dtype=torch.float32)
    for i, e in enumerate(te):
        ref = F.fp8_gemm(aq[i * 128:(i + 1) * 128], as_[i * 128:(i + 1) * 128], wq[:, e * Fd:(e + 1) * Fd],
                         ws[:, e * Fd // 128:(e + 1) * Fd // 128], round_bf16=False)
        got = c[i * 128:(i + 1) * 128].cpu().numpy()
        assert np.all(np.abs(got - ref) <= 1e-4 * (np.abs(ref).max(1, keepdims=True) + 1e-30)), f"tile {i}"


@pytest.mark.parametrize("rows_dtype", [torch.float32, torch.bfloat16])
def test_moe_combine(rows_dtype):
    rng = np.random.default_rng(7)
    T, E, k, S, d = 300, 8, 2, 1, 768
    idx, w = picks(rng, T, E, k, bad=3)
    rows = K.moe_align(dev(idx), dev(w), E, S)
    _, _, _, er = MO.moe_align(idx, w, E, S)
    out = dev(rng.standard_normal((rows.num_rows, d)).astype(np.float32)).to(rows_dtype)
    b2 = rng.standard_normal((E + S, d)).astype(np.float32)
    y = K.moe_combine(out, rows.entry_row, dev(idx), dev(w), E, S, dev(b2)).float().cpu().numpy()
    ref = MO.moe_combine(out.double().cpu().numpy(), er, idx, w, E, S, b2)
    # one bf16 rounding of an fp32 sum vs of a float64 sum
    assert np.all(np.abs(y - ref) <= 2.0 ** -7 * np.abs(ref) + 1e-6)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_segment_and_scatter_reduce(dtype):
    rng = np.random.default_rng(8)
    n, T, d = 3000, 700, 300
    x = rng.standard_normal((n, d)).astype(np.float32)
    w = rng.uniform(0, 1, n).astype(np.float32)
    idx = rng.integers(0, T, n)
    idx[:5] = [-1, T, T + 3, -7, T]  # dropped by the unsorted form
    xt = dev(x).to(dtype)
    wt = dev(w)
    x64 = xt.double().cpu().numpy()
    tol = 2.0 ** -7 if dtype == torch.bfloat16 else 1e-5
    got = K.fused_scatter_add_weighted(xt, dev(idx), wt, T, 2)
    assert got.dtype == dtype
    ref = MO.scatter_add_weighted(x64, idx, w, T)
    g = got.double().cpu().numpy()
    assert np.all(np.abs(g - ref) <= tol * np.abs(ref) + 1e-5), "scatter"
    # the sorted form (the reference's segment_reduce_weighted input)
    keep = (idx >= 0) & (idx < T)
    order = np.argsort(idx[keep], kind="stable")
    sx = xt[torch.from_numpy(np.nonzero(keep)[0][order]).to(DEV)]
    got_s = K.segment_reduce_weighted(sx, dev(w[keep][order]), dev(idx[keep][order]), T, 2)
    assert np.all(np.abs(got_s.double().cpu().numpy() - ref) <= tol * np.abs(ref) + 1e-5), "segment"
    # a token's entries sum in entry order: repeated calls are bit-identical
    assert torch.equal(got, K.fused_scatter_add_weighted(xt, dev(idx), wt, T, 2))


@pytest.mark.parametrize("T", [1, 300, 1000])
def test_grouped_moe_layer_matches_dense_and_reference(T):
    """The MoE layer with grouped dispatch vs dense dispatch (same weights)
    and vs the fp32 torch restatement of moe_infer + shared expert used by
    the model tests."""
    from llm_from_scratch_amd.decode_model import DecodeModel, DecodeModelConfig
    import test_gpu_model as TM

    cfg = DecodeModelConfig(vocab_size=512, d_model=256, num_layers=1, num_heads=4, num_kv_heads=2,
                            d_ff=256, n_routed_experts=8, num_experts_per_tok=2, max_model_length=64)
    torch.manual_seed(T)
    model = DecodeModel(cfg, device=DEV, seed=3)
    f = model.layers[0].ffn
    with torch.no_grad():
        f.expert_bias.copy_(torch.randn(cfg.n_routed_experts, device=DEV) * 0.1)
    h = (torch.randn(T, cfg.d_model, device=DEV)).to(torch.bfloat16)
    hq, hs = K.act_quant(h)
    f.dispatch = "grouped"
    yg = f(h, hq, hs)
    f.dispatch = "dense"
    yd = f(h, hq, hs)
    ref = TM.ref_moe(f, h, cfg)
    e_gd = TM.rel_err_rows(yg, yd)
    e_g, e_d = TM.rel_err_rows(yg, ref), TM.rel_err_rows(yd, ref)
    assert e_gd.max().item() <= 1e-2, f"grouped vs dense {e_gd.max().item():.4f}"
    # vs the fp32 restatement: row by row no further than the dense dispatch
    # (whose per-op parity the model tests pin), and 99% of rows within the
    # per-layer bar -- single rows whose e4m3 codes flip between an fp32 and
    # an FP8 computation stand further off in both dispatches alike
    assert bool((e_g <= e_d + 2e-3).all()), f"grouped {e_g.max().item():.4f} vs dense {e_d.max().item():.4f}"
    assert torch.quantile(e_g.float(), 0.99).item() <= TM.TOL_LAYER


def test_moe_route_large_batch_kernel_matches_per_token_kernel():
    """Above 1024 tokens the gate runs four tokens per workgroup; its sums
    run in the same order as the one-token-per-workgroup kernel (which the
    model tests pin against the fp32 reference), so every output is
    bit-identical on the rows both compute."""
    g = torch.Generator(device=DEV).manual_seed(21)
    T, d, E, S, k = 2500, 768, 8, 1, 2
    h = torch.randn(T, d, generator=g, device=DEV).to(torch.bfloat16)
    gw = (torch.randn(E, d, generator=g, device=DEV) * 0.05).to(torch.bfloat16)
    eb = torch.randn(E, generator=g, device=DEV) * 0.1
    b2 = torch.randn(E + S, d, generator=g, device=DEV)
    big = K.moe_route(h, gw, eb, b2, k, S, return_topk=True)
    small = K.moe_route(h[:1000].contiguous(), gw, eb, b2, k, S, return_topk=True)
    for a, b, what in zip(big, small, ("dense", "bias", "topk_idx", "topk_weight")):
        assert torch.equal(a[:1000], b), what
    # grouped-only call (no dense / bias outputs) gives the same picks
    _, _, idx, wt = K.moe_route(h, gw, eb, None, k, S, dense=False, return_topk=True)
    assert torch.equal(idx, big[2]) and torch.equal(wt, big[3])

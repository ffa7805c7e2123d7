"""Fused row kernels of the decode step vs the torch ops they replace.

Each kernel is compared with the reference formulation in torch on the
same device (model/utils.py:53-67 RMSNorm, model/attention/utils.py:34-45
RoPE, model/architecture/moe.py:45-90 gate, model/architecture/mlp.py:60-67
SwiGLU).  Row reductions are summed in a different order than torch's, so
norm outputs may differ by one bf16 step in rare elements; everything that
does not depend on a reduction (residual sums, slot writes, the
quantisation of the kernel's own output) is compared bit for bit.
"""
import math

import numpy as np
import pytest
import torch

from llm_from_scratch_amd import kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def bf16_steps(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """|a - b| in units of the bf16 spacing at b."""
    a, b = a.float(), b.float()
    spacing = torch.where(b == 0, torch.full_like(b, 2.0 ** -133),
                          2.0 ** (torch.floor(torch.log2(b.abs())) - 7))
    return (a - b).abs() / spacing


def rms_ref(x, w, eps, residual=None):
    xf = x.float() if residual is None else x.float() + residual.float()
    return (w * xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16), xf.to(torch.bfloat16)


@pytest.mark.parametrize("T,d", [(1, 768), (128, 768), (37, 256), (5, 4096), (3, 8192), (4, 200)])
def test_add_rmsnorm(T, d):
    g = torch.Generator(device=DEV).manual_seed(T * 7 + d)
    x = (torch.randn(T, d, generator=g, device=DEV) * 3).to(torch.bfloat16)
    r = torch.randn(T, d, generator=g, device=DEV).to(torch.bfloat16)
    w = torch.rand(d, generator=g, device=DEV) + 0.5
    quant = d % 128 == 0
    for residual in (None, r):
        out, res_out, q, qs = K.add_rmsnorm(x, w, 1e-5, residual, out=True, quant=quant)
        want, want_res = rms_ref(x, w, 1e-5, residual)
        steps = bf16_steps(out, want)
        assert steps.max() <= 1 and (steps > 0).float().mean() < 1e-3, f"max {steps.max()}"
        if residual is None:
            assert res_out is x
        else:
            assert torch.equal(res_out, want_res)
        if quant:
            q2, qs2 = K.act_quant(out, 128)
            assert torch.equal(q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(qs, qs2)
    if quant:  # quantised output only
        none, _, q3, qs3 = K.add_rmsnorm(x, w, 1e-5, r, out=False, quant=True)
        assert none is None and torch.equal(q3.view(torch.uint8), q.view(torch.uint8)) and torch.equal(qs3, qs)


def rope_ref(x, cos_sin, pos):
    cos, sin = cos_sin[pos].unsqueeze(1).chunk(2, -1)
    x1, x2 = x.float().chunk(2, -1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1).to(torch.bfloat16)


@pytest.mark.parametrize("T,Hq,Hkv,D", [(128, 12, 4, 64), (7, 32, 8, 128), (3, 4, 4, 64), (2, 64, 8, 128)])
def test_qk_norm_rope_store(T, Hq, Hkv, D):
    g = torch.Generator(device=DEV).manual_seed(T + Hq + D)
    W = (Hq + 2 * Hkv) * D
    qkv_full = torch.randn(T, W + 16, generator=g, device=DEV).to(torch.bfloat16)
    qkv = qkv_full[:, :W]  # strided rows
    qw = torch.rand(Hq * D, generator=g, device=DEV) + 0.5
    kw = torch.rand(Hkv * D, generator=g, device=DEV) + 0.5
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device=DEV).float() / D))
    ang = torch.outer(torch.arange(4096, device=DEV).float(), inv)
    cos_sin = torch.cat([ang.cos(), ang.sin()], -1)
    pos = torch.randint(0, 4096, (T,), generator=g, device=DEV)
    NB, BS = 8, 16
    kc = torch.full((NB, BS, Hkv, D), -7.0, device=DEV, dtype=torch.bfloat16)
    vc = torch.full_like(kc, -7.0)
    slots = torch.randperm(NB * BS, generator=g, device=DEV)[:T]
    slots[0] = -1  # skipped
    eps = torch.finfo(torch.float32).eps
    q = K.qk_norm_rope_store(qkv, qw, kw, cos_sin, pos, Hq, Hkv, eps, kc, vc, slots)
    qr, kr, vr = qkv.split([Hq * D, Hkv * D, Hkv * D], -1)
    qn, _ = rms_ref(qr, qw, eps)
    kn, _ = rms_ref(kr, kw, eps)
    want_q = rope_ref(qn.view(T, Hq, D), cos_sin, pos)
    want_k = rope_ref(kn.view(T, Hkv, D), cos_sin, pos)
    steps = bf16_steps(q, want_q)
    # a one-step difference in the norm output can move the rotated value by
    # a few bf16 steps where the rotation cancels; bound by the row scale
    err = (q.float() - want_q.float()).abs().amax() / want_q.float().abs().amax()
    assert err < 1e-2 and (steps > 0).float().mean() < 1e-2
    flat_k = kc.view(-1, Hkv, D)
    flat_v = vc.view(-1, Hkv, D)
    written = torch.zeros(NB * BS, dtype=torch.bool, device=DEV)
    for t in range(1, T):
        s = int(slots[t])
        written[s] = True
        assert torch.equal(flat_v[s], vr[t].reshape(Hkv, D)), f"v slot of token {t}"
        e = (flat_k[s].float() - want_k[t].float()).abs().amax() / want_k[t].float().abs().amax()
        assert e < 1e-2, f"k slot of token {t}: {e}"
    assert (flat_k[~written] == -7.0).all() and (flat_v[~written] == -7.0).all()


@pytest.mark.parametrize("T,d,E,S,k", [(128, 768, 8, 1, 2), (33, 256, 4, 0, 1), (5, 1024, 16, 2, 4)])
def test_moe_route(T, d, E, S, k):
    g = torch.Generator(device=DEV).manual_seed(T + E)
    h = torch.randn(T, d, generator=g, device=DEV).to(torch.bfloat16)
    gw = (torch.randn(E, d, generator=g, device=DEV) / math.sqrt(d)).to(torch.bfloat16)
    eb = torch.randn(E, generator=g, device=DEV) * 0.1
    b2 = torch.randn(E + S, d, generator=g, device=DEV)
    w, bias = K.moe_route(h, gw, eb, b2, k, S)
    logits = h.float() @ gw.float().t()
    scores = torch.sigmoid(logits)
    idx = torch.topk(logits + eb, k, -1).indices
    sel = torch.gather(scores, -1, idx)
    if k > 1:
        sel = sel / (sel.sum(-1, keepdim=True) + 1e-10)
    dense = torch.zeros(T, E + S, device=DEV).scatter_(1, idx, sel)
    dense[:, E:] = 1.0
    assert torch.equal(w > 0, dense > 0), "different experts chosen"
    torch.testing.assert_close(w, dense, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(bias, dense @ b2, rtol=1e-5, atol=1e-5)


def test_moe_route_near_ties():
    """Expert selection on exact and near ties, pinned in the kernel's
    arithmetic: logits (fp32 dot of bf16 rows) are exact small integers
    (h = 1, integer gate weights), the biased keys logit + bias are compared
    in fp32, and exact ties go to the lower expert index.  Token rows:
    (a) two experts tie exactly (key 10): the lower index wins;
    (b) keys 10, 10 + 2^-20, 10 + 2^-20 (one fp32 ulp apart; all equal once
        rounded to bf16, as the reference's bf16 gate would round them): the
        two larger fp32 keys win;
    (c) keys 7, 7, 7 + 2^-20: the one-ulp larger key, then the lower index
        of the exact tie.
    This fixes the deliberate fp32 choice; the reference rounds logits, the
    bias add and the renormalised weights to bf16 (model/architecture/moe.py:
    45-69) and orders ties as torch.topk(sorted=False) does."""
    d, E, k = 256, 8, 2
    ulp = 2.0 ** -20
    rows = [
        # three-way exact tie at 10: the two lowest indices
        ([10, 10, 10, 2, 1, 0, 0, 0], [0.0] * 8, [0, 1]),
        # keys 10, 10 + ulp, 10 + ulp (9 + (1 + 2^-20) is exact in fp32)
        ([10, 9, 9, 2, 1, 0, 0, 0], [0.0, 1.0 + ulp, 1.0 + ulp, 0, 0, 0, 0, 0], [1, 2]),
        # keys 7, 7, 7 + ulp: the near-tie first, then the lower of the exact tie
        ([7, 7, 7, 1, 0, 0, 0, 0], [0.0, 0.0, ulp, 0, 0, 0, 0, 0], [0, 2]),
    ]
    T = len(rows)
    h = torch.ones(T, d, device=DEV, dtype=torch.bfloat16)
    gw = torch.zeros(T * E, d, device=DEV)
    outs = []
    for t, (logit, bias, want) in enumerate(rows):
        gwt = torch.zeros(E, d, device=DEV)
        for e, L in enumerate(logit):  # L ones in the row: the dot with h = 1 is exactly L
            gwt[e, :L] = 1.0
        w, _ = K.moe_route(h[t:t + 1], gwt.to(torch.bfloat16), torch.tensor(bias, device=DEV),
                           torch.zeros(E, d, device=DEV), k, 0)
        chosen = torch.nonzero(w[0] > 0).flatten().tolist()
        assert sorted(chosen) == sorted(want), f"row {t}: chose {chosen}, expected {want}"
        sc = torch.sigmoid(torch.tensor(logit, dtype=torch.float32))[want]
        torch.testing.assert_close(w[0, want].cpu(), sc / (sc.sum() + 1e-10), rtol=1e-6, atol=0)


@pytest.mark.parametrize("T,E,F", [(128, 9, 512), (3, 2, 128), (17, 4, 1024)])
def test_swiglu_quant(T, E, F):
    g = torch.Generator(device=DEV).manual_seed(T + F)
    h13 = (torch.randn(T, E, 2, F, generator=g, device=DEV) * 2).to(torch.bfloat16)
    route = torch.rand(T, E, generator=g, device=DEV)
    route[:, 0] = 0.0
    q, qs = K.swiglu_quant(h13, route)
    gg = torch.nn.functional.silu(h13[:, :, 0]) * h13[:, :, 1]
    q2, qs2 = K.act_quant(gg.reshape(T, E * F), 128)
    same = (q.view(torch.uint8) == q2.view(torch.uint8)).float().mean().item()
    assert same > 0.999, f"codes equal for {same:.5f} of elements"
    want_s = (qs2.view(T, E, F // 128) * route.unsqueeze(-1)).view(T, -1)
    torch.testing.assert_close(qs, want_s, rtol=2e-7, atol=0)


@pytest.mark.parametrize("T,d,E,S,top_k,with_res", [(128, 768, 8, 1, 2, True), (37, 1024, 16, 2, 4, False),
                                                    (9, 2048, 8, 0, 1, True), (5, 4096, 32, 1, 3, True),
                                                    (64, 512, 4, 0, 1, True), (3, 1024, 6, 2, 2, False)])
def test_add_rmsnorm_route_equals_norm_then_gate(T, d, E, S, top_k, with_res):
    """The fused ffn_norm + MoE gate launch gives the outputs of add_rmsnorm
    (quantised) followed by moe_route bit for bit: residual, codes, scales,
    dense routing weights and routed down bias."""
    g = torch.Generator(device="cuda").manual_seed(T + d + E)
    x = torch.randn(T, d, generator=g, device="cuda").to(torch.bfloat16)
    res = torch.randn(T, d, generator=g, device="cuda").to(torch.bfloat16) if with_res else None
    w = (1 + 0.1 * torch.randn(d, generator=g, device="cuda")).float()
    gw = (0.05 * torch.randn(E, d, generator=g, device="cuda")).to(torch.bfloat16)
    eb = (0.1 * torch.randn(E, generator=g, device="cuda")).float()
    b2 = (0.02 * torch.randn(E + S, d, generator=g, device="cuda")).float()
    h, r, q, qs = K.add_rmsnorm(x, w, 1e-5, res, out=True, quant=True)
    rw, rb = K.moe_route(h, gw, eb, b2, top_k, S)
    h2, r2, q2, qs2, rw2, rb2 = K.add_rmsnorm_route(x, w, 1e-5, res, gw, eb, b2, top_k, S, out=True)
    torch.cuda.synchronize()
    assert torch.equal(h2, h) and torch.equal(r2, r)
    assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8)) and torch.equal(qs2, qs)
    assert torch.equal(rw2, rw) and torch.equal(rb2, rb)
    assert int((rw2[:, :E] > 0).sum(1).min()) == top_k and bool((rw2[:, E:] == 1).all())


@pytest.mark.parametrize("T,d,Kd,splits,bias_kind", [(128, 768, 4608, 6, "matrix"), (37, 512, 2048, 3, "vector"),
                                                    (5, 1024, 1536, 12, None), (64, 256, 3072, 8, "matrix"),
                                                    (32, 2048, 3840, 5, "matrix"), (9, 4096, 2048, 4, "vector"),
                                                    (3, 8192, 1536, 3, None)])
def test_add_rmsnorm_partials_equals_reduce_then_norm(T, d, Kd, splits, bias_kind):
    """add & norm over a split-K GEMM's partials (the cfg5 MoE down
    projection feeding the next layer's att_norm) equals the split-K GEMM's
    bf16 output followed by add_rmsnorm, bit for bit: residual, normalised
    row, codes and scales; the partials summed in order with the bias equal
    the GEMM's own split-K output."""
    g = torch.Generator(device=DEV).manual_seed(T + d + Kd)
    a = torch.randn(T, Kd, generator=g, device=DEV).to(torch.bfloat16)
    wgt = (0.02 * torch.randn(d, Kd, generator=g, device=DEV)).to(torch.bfloat16)
    aq, as_ = K.act_quant(a)
    wq, ws = K.weight_quant(wgt)
    bias = None
    if bias_kind == "matrix":
        bias = torch.randn(T, d, generator=g, device=DEV)
    elif bias_kind == "vector":
        bias = torch.randn(d, generator=g, device=DEV)
    res = torch.randn(T, d, generator=g, device=DEV).to(torch.bfloat16)
    nw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).float()
    parts = K.fp8_gemm_splitk_partials(aq, as_, wq, ws, splits)
    assert parts.shape == (K.splitk_used(Kd, splits), T, d)
    y = K.fp8_gemm(aq, as_, wq, ws, bias, splits=splits)
    acc = torch.zeros(T, d, device=DEV)  # 0 + p0 + p1 + ... (+ bias), in fp32
    for s in range(parts.size(0)):
        acc = acc + parts[s]
    if bias is not None:
        acc = acc + bias
    assert torch.equal(y, acc.to(torch.bfloat16))
    h, r, q, qs = K.add_rmsnorm(y, nw, 1e-5, res, out=True, quant=True)
    h2, r2, q2, qs2 = K.add_rmsnorm_partials(parts, bias, nw, 1e-5, res, out=True, quant=True)
    torch.cuda.synchronize()
    assert torch.equal(h2, h) and torch.equal(r2, r)
    assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8)) and torch.equal(qs2, qs)


def test_moe_route_vs_reference_bf16_gate():
    """The fp32 GPU gate against the reference's own bf16 Gate
    (tests/golden/gate_bf16.npz, cfg5 shape: 4096 tokens, 8 experts, top-2):
    the same picks on every token but bf16 near-ties (the reference's k-th
    and (k+1)-th biased logits within two bf16 ulps), and on the others the
    weights within four bf16 roundings of the reference's."""
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).with_name("golden")))
    from make_gate_golden import TOP_K, gate_inputs
    from test_oracle_gate import _fixture, _sorted_picks, near_tie_tokens
    x, w, bias = gate_inputs()
    ref_biased, ref_idx, ref_wts = _fixture()
    h = torch.from_numpy(x).to(torch.bfloat16).to(DEV)
    gw = torch.from_numpy(w).to(torch.bfloat16).to(DEV)
    eb = torch.from_numpy(bias).to(DEV)
    _, _, idx, wt = K.moe_route(h, gw, eb, None, TOP_K, 0, dense=False, return_topk=True)
    torch.cuda.synchronize()
    pi, pw = _sorted_picks(idx.cpu().numpy(), wt.cpu().numpy())
    differ = (pi != ref_idx).any(-1)
    ties = near_tie_tokens(ref_biased, TOP_K)
    assert not (differ & ~ties).any(), f"{int((differ & ~ties).sum())} tokens differ without a bf16 near-tie"
    assert differ.sum() <= 0.02 * len(differ)
    np.testing.assert_allclose(pw[~differ], ref_wts.float().numpy()[~differ], rtol=2 ** -6, atol=0)

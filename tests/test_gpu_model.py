"""FP8Linear, the paged GQA + MoE decode model and the graph-captured decode
step, on the GPU.

The checker is oracle/model.py: the reference's decoder forward restated in
torch (model/transformer.py:90-183, model/attention/GQA.py:65-139,
model/utils.py:44-67, model/architecture/moe.py:45-90, 272-273, 289-341),
itself pinned on the CPU to logits the reference's own TransformerLM wrote
(tests/test_oracle_model.py, tests/golden/model_forward.npz).  Here it runs
on the product's own weights -- each FP8 projection dequantised, the fused
q/k/v and stacked expert matrices split back into the reference's state-dict
layout -- with a linear that emulates the FP8 path:
dequant(act_quant(x)) @ dequant(W)^T + b, rounded to bf16.

Two tolerances:
  * each op of each layer (FP8 linears, norms, K/V writes, paged attention,
    the MoE's SwiGLU + down projection + weighted combine) fed the GPU's own
    input to that op and the GPU-written KV cache (teacher forcing): every
    element within rtol 1e-2 / atol 2e-2 of the reference, and every row
    within TOL_LAYER = 1e-2 relative L2 error -- the single-op bar;
  * e2e_tol(layers) = 4e-2 * sqrt(layers), relative L2 error per row, for
    logits after the whole stack, a drift bound rather than a parity bar.  Two valid FP8
    computations drift apart layer by layer: a bf16 rounding difference in
    one linear's output flips the e4m3 code of some activations in the next
    (one e4m3 step is 2^-3 relative), so a 1e-3 difference entering a MoE
    leaves it as ~1e-2.  Measured on MI355X: 3.0-4.0e-2 after 2 layers,
    3.8-7.9e-2 after 12; every single op stays within 4e-3.
The reference's own logits (the golden fixture, fp32 weights) are also
compared with the product loaded from the same state dict: that distance is
the FP8 quantisation of weights and activations itself, bounded separately
(measured 5.0e-2 after 2 layers).
"""
import math
import sys
import weakref
from pathlib import Path

import numpy as np
import pytest
import torch

from llm_from_scratch_amd.context import reset_context
from llm_from_scratch_amd.decode_model import DecodeModel, DecodeModelConfig
from llm_from_scratch_amd.engine import BlockManager, LLMEngine, ModelRunner, SamplingParams, Sequence
from llm_from_scratch_amd.fp8_linear import FP8Linear
from llm_from_scratch_amd import kernels, workloads
from oracle import fp8 as ofp8
from oracle import model as om

sys.path.insert(0, str(Path(__file__).with_name("golden")))
from make_model_golden import GOLDEN_DIMS, GOLDEN_SEED  # noqa: E402

pytestmark = pytest.mark.gpu

INV448 = torch.tensor(1.0 / 448.0, dtype=torch.float32)


# ---------------------------------------------------------------- helpers --
def q_act(x: torch.Tensor) -> torch.Tensor:
    """fp32 value of act_quant's e4m3 codes times their 1x128 scales."""
    T, K = x.shape
    xf = x.float().view(T, K // 128, 128)
    s = xf.abs().amax(-1, keepdim=True).clamp_min(1e-4) * INV448.to(x.device)
    q = torch.clamp(xf / s, -448, 448).to(torch.float8_e4m3fn).float()
    return (q * s).view(T, K)


def w_deq(m: FP8Linear) -> torch.Tensor:
    s = m.weight_scale.repeat_interleave(128, 0)[:m.out_features].repeat_interleave(128, 1)
    return m.weight.float() * s


def lin(m: FP8Linear, x: torch.Tensor) -> torch.Tensor:
    return lin_w(w_deq(m), m.bias, x)


def lin_w(w: torch.Tensor, bias, x: torch.Tensor) -> torch.Tensor:
    """dequant(act_quant(x)) @ w^T (+ bias), rounded to bf16."""
    y = q_act(x.to(torch.bfloat16)) @ w.t()
    if bias is not None:
        y = y + bias
    return y.to(torch.bfloat16)


def fp8_linear(wd: dict) -> om.Linear:
    """The oracle's projection hook: lin_w on the dequantised weights."""
    return lambda p, x: lin_w(wd[p + ".weight"], wd.get(p + ".bias"), x)


def dims_of(cfg: DecodeModelConfig) -> om.ModelDims:
    return om.ModelDims(cfg.vocab_size, cfg.d_model, cfg.num_layers, cfg.num_heads, cfg.num_kv_heads, cfg.d_ff,
                        cfg.n_routed_experts, cfg.num_experts_per_tok, cfg.n_shared_experts, cfg.rope_theta,
                        cfg.rms_eps)


def split_qkv(y, cfg):
    """Rows of the fused q/k/v projection's output -> q, k, v."""
    Hq, Hkv, D = cfg.num_heads, cfg.num_kv_heads, cfg.head_dim
    return y.split([Hq * D, Hkv * D, Hkv * D], dim=-1)


def expert_weights(f, e):
    """(w1, b1, w3, b3, w2, b2) of expert e (the last one is the shared
    expert), dequantised from the stacked FP8 weights."""
    F = f.d_ff
    w13, b13 = w_deq(f.w13), f.w13.bias
    w2 = w_deq(f.w2)
    r = 2 * F * e
    return (w13[r:r + F], b13[r:r + F], w13[r + F:r + 2 * F], b13[r + F:r + 2 * F],
            w2[:, e * F:(e + 1) * F], f.w2_bias[e])


def moe_weights(f, p: str) -> dict:
    """One MoE layer's dequantised weights under the reference's names."""
    out = {p + "ffn.gate.weight": f.gate_weight.float(), p + "ffn.gate.expert_bias": f.expert_bias}
    names = [f"ffn.experts.{e}" for e in range(f.n_experts)] + ["ffn.shared_expert"] * f.n_shared
    for e, m in enumerate(names):
        for key, t in zip((".w1.weight", ".w1.bias", ".w3.weight", ".w3.bias", ".w2.weight", ".w2.bias"),
                          expert_weights(f, e)):
            out[p + m + key] = t
    return out


_WEIGHTS = weakref.WeakKeyDictionary()


def product_weights(model: DecodeModel) -> dict:
    """The model's weights in the reference's state-dict layout, every FP8
    projection dequantised (computed once per model)."""
    if model in _WEIGHTS:
        return _WEIGHTS[model]
    cfg = model.cfg
    wd = {"token_embeddings.weight": model.embed, "final_norm.weight": model.final_norm.weight,
          "lm_head.weight": w_deq(model.lm_head), "lm_head.bias": model.lm_head.bias}
    for i, blk in enumerate(model.layers):
        p, a = f"layers.{i}.", blk.att
        for n, w, b in zip(("q_proj", "k_proj", "v_proj"), split_qkv(w_deq(a.qkv_proj).t(), cfg),
                           split_qkv(a.qkv_proj.bias, cfg)):
            wd[p + f"att.{n}.weight"], wd[p + f"att.{n}.bias"] = w.t(), b
        wd[p + "att.output_proj.weight"] = w_deq(a.output_proj)
        wd[p + "att.output_proj.bias"] = a.output_proj.bias
        wd[p + "att.q_norm.weight"], wd[p + "att.k_norm.weight"] = a.q_norm.weight, a.k_norm.weight
        wd[p + "att_norm.weight"], wd[p + "ffn_norm.weight"] = blk.att_norm.weight, blk.ffn_norm.weight
        wd.update(moe_weights(blk.ffn, p))
    _WEIGHTS[model] = wd
    return wd


def ref_moe(f, h, cfg):
    """The oracle's MoE on the FP8-emulated weights of one layer."""
    wd = moe_weights(f, "")
    return om.moe(wd, "", h, dims_of(cfg), fp8_linear(wd))


def ref_logits(model: DecodeModel, tokens: list[int]) -> torch.Tensor:
    """The oracle's causal forward over one sequence on the model's
    FP8-emulated weights, bf16 activations; fp32 logits [T, vocab]."""
    wd = product_weights(model)
    return om.forward(wd, tokens, dims_of(model.cfg), fp8_linear(wd), embed_dtype=torch.bfloat16)


def rel_err_rows(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    a, b = a.float(), b.float()
    return (a - b).norm(dim=-1) / b.norm(dim=-1).clamp_min(1e-6)


TOL_LAYER = 1e-2
ELEM_RTOL, ELEM_ATOL = 1e-2, 2e-2  # every element of every teacher-forced op


def e2e_tol(num_layers: int) -> float:
    return 4e-2 * math.sqrt(num_layers)
SMALL = DecodeModelConfig(vocab_size=1024, d_model=256, num_layers=2, num_heads=4, num_kv_heads=2,
                          d_ff=256, n_routed_experts=4, num_experts_per_tok=2, max_model_length=512)


@pytest.fixture
def block_size():
    old = Sequence.block_size
    yield
    Sequence.block_size = old


# ------------------------------------------------------------- FP8Linear --
def test_fp8_linear_cfg1_matches_oracle():
    x = workloads.activation(256, 512, seed=0, device="cuda")
    w = workloads.weight(1344, 512, seed=0, device="cuda")
    bias = torch.randn(1344, generator=torch.Generator().manual_seed(5)).cuda()
    m = FP8Linear(512, 1344, device="cuda").load_weight(w, bias)
    wq, ws = ofp8.weight_quant(w.float().cpu().numpy(), 128)
    assert np.array_equal(m.weight.view(torch.uint8).cpu().numpy(), wq)
    assert np.array_equal(m.weight_scale.cpu().numpy(), ws)
    y = m(x).float().cpu().numpy()
    aq, asc = ofp8.act_quant(x.float().cpu().numpy(), 128)
    want = ofp8.fp8_gemm(aq, asc, wq, ws, bias=bias.cpu().numpy())
    np.testing.assert_allclose(y, want, rtol=1e-2, atol=2e-2)


# ------------------------------------------------------- decode model ----
def _prefill(runner, seqs):
    ids, pos = runner.prepare_prefill(seqs)
    logits = runner.run_model(ids, pos, True)
    from llm_from_scratch_amd.context import get_context
    last = (get_context().cu_seqlens_q[1:] - 1).long()
    reset_context()
    return logits[last].float()


def _gather(cache, table, L):
    t = torch.arange(L, device=cache.device)
    blocks = torch.tensor(table, device=cache.device)[t // cache.size(1)]
    return cache[blocks, t % cache.size(1)]


def check_layers_teacher_forced(model, runner, seqs):
    """Eager decode step with the model's trace on; each op must match the
    reference on the GPU's own input to that op (teacher forcing), so no
    error is carried from one op to the next:
      every FP8 linear (qkv, output, experts' w1/w3, lm_head) vs
      dequant(act_quant(x)) @ dequant(W)^T + b;
      att_norm / ffn_norm / final_norm (fused add & norm, residual out);
      q after q_norm + RoPE, and the newest token's K/V in the pool after
      k_norm + RoPE, vs the same from the GPU's qkv output;
      attention (GQA over the K/V the GPU wrote to the pool) vs its output;
      gate weights and routed bias vs the reference gate;
      MoE down projection from the GPU's w1/w3 output: per-expert SwiGLU and
      w2 (+ bias), combined with the gate weights and the shared expert, vs
      the MoE output.
    Returns the largest error per op kind."""
    model.trace = {}
    try:
        _decode(runner, seqs, eager=True)
        tr = model.trace
    finally:
        model.trace = None
    cfg = model.cfg
    dims = dims_of(cfg)
    worst: dict[str, float] = {}

    def chk(kind, got, want, what):
        e = rel_err_rows(got.reshape(got.shape[0], -1), want.reshape(want.shape[0], -1)).max().item()
        worst[kind] = max(worst.get(kind, 0.0), e)
        assert e <= TOL_LAYER, f"{what}: {kind} rel err {e:.4f}"
        # and element by element, the north star's bar for GEMM / attention outputs
        g, w_ = got.float().reshape(-1), want.float().reshape(-1)
        bad = (g - w_).abs() > ELEM_ATOL + ELEM_RTOL * w_.abs()
        assert not bool(bad.any()), (f"{what}: {kind} {int(bad.sum())} of {g.numel()} elements outside "
                                     f"rtol {ELEM_RTOL} / atol {ELEM_ATOL}, worst |diff| "
                                     f"{(g - w_).abs().max().item():.4g}")

    pos = torch.tensor([len(s) - 1 for s in seqs], device=model.embed.device)
    for layer, blk in enumerate(model.layers):
        t, p = tr[layer], f"layer {layer}"
        if t["residual"] is None:
            h, r = om.rms_norm(t["x"], blk.att_norm.weight, cfg.rms_eps)[0], t["x"]
        else:
            h, r = om.rms_norm(t["x"], blk.att_norm.weight, cfg.rms_eps, t["residual"])
        chk("norm", t["att_h"], h, f"{p} att_norm")
        a = blk.att
        chk("linear", t["qkv"], lin(a.qkv_proj, t["att_h"]), f"{p} qkv_proj")
        q, k, v = om.qkv_heads(*split_qkv(t["qkv"], cfg), a.q_norm.weight, a.k_norm.weight, pos, dims,
                               torch.bfloat16)
        chk("q_norm_rope", t["q"], q, p)
        for i, s in enumerate(seqs):
            L = len(s)
            Kc = _gather(a.k_cache, s.block_table, L)
            Vc = _gather(a.v_cache, s.block_table, L)
            what = f"{p} seq {i} len {L}"
            chk("new_k", Kc[-1:], k[i:i + 1], what)
            chk("new_v", Vc[-1:], v[i:i + 1], what)
            chk("attention", t["att_o"][i:i + 1], om.gqa_attention(t["q"][i:i + 1], Kc, Vc), what)
        chk("linear", t["att_out"], lin(a.output_proj, t["att_o"]), f"{p} output_proj")
        h2, r2 = om.rms_norm(t["att_out"], blk.ffn_norm.weight, cfg.rms_eps, r)
        chk("norm", t["ffn_h"], h2, f"{p} ffn_norm")
        chk("norm", t["res_mid"], r2, f"{p} residual")
        f = blk.ffn
        idx, w = om.route(t["ffn_h"], f.gate_weight, f.expert_bias, f.top_k)
        dense = torch.zeros(len(seqs), f.n_experts + f.n_shared, device=w.device)
        dense.scatter_(1, idx, w)
        dense[:, f.n_experts:] = 1.0
        chk("route", t["route_w"], dense, p)
        chk("route", t["route_bias"], dense @ f.w2_bias, p)
        chk("linear", t["h13"], lin(f.w13, t["ffn_h"]), f"{p} w13")
        outs = []
        for e in range(f.n_experts + f.n_shared):
            _, _, _, _, w2, b2 = expert_weights(f, e)
            r0 = 2 * f.d_ff * e
            h1, h3 = t["h13"][:, r0:r0 + f.d_ff], t["h13"][:, r0 + f.d_ff:r0 + 2 * f.d_ff]
            outs.append(lin_w(w2, b2, om.swiglu(h1.to(torch.bfloat16), h3.to(torch.bfloat16))))
        y = om.combine(idx, w, outs[:f.n_experts], outs[f.n_experts] if f.n_shared else None, torch.bfloat16)
        chk("moe_down_combine", t["ffn_out"], y, p)
    fin = tr["final"]
    chk("norm", fin["h"], om.rms_norm(fin["x"], model.final_norm.weight, cfg.rms_eps, fin["residual"])[0],
        "final_norm")
    chk("linear", fin["logits"], lin(model.lm_head, fin["head_in"]), "lm_head")
    return worst


def _decode(runner, seqs, eager):
    ids, pos = runner.prepare_decode(seqs)
    old = runner.enforce_eager
    runner.enforce_eager = eager
    try:
        logits = runner.run_model(ids, pos, False).float()
    finally:
        runner.enforce_eager = old
        reset_context()
    return logits


@torch.inference_mode()
def test_runner_sizes_pool_after_warmup():
    """Without num_kv_blocks the runner warms up with a full-length prefill
    and sizes the pool as free x gpu_memory_utilization - (peak - current)
    (engine/model_runner.py:151-181); the sized runner then serves a prefill
    and a decode step with the same logits as a runner given the block count
    explicitly (same weights, same block tables)."""
    BS = 16
    Sequence.block_size = BS
    model = DecodeModel(SMALL, device="cuda", seed=13)
    util = 0.02
    cfg = SMALL.runner_config(block_size=BS, max_num_seqs=4, gpu_memory_utilization=util,
                              max_num_batched_tokens=2 * SMALL.max_model_length)
    torch.cuda.empty_cache()
    runner = ModelRunner(model, cfg)
    D = SMALL.head_dim
    block_bytes = BS * 2 * SMALL.num_layers * SMALL.num_kv_heads * D * 2
    free_after = torch.cuda.mem_get_info()[0]
    nb = runner.num_available_kv_blocks
    # the pool took about util x (free before it) minus the warm-up reserve
    assert runner.kv_reserved_bytes > 0, "the warm-up prefill left no peak above the resident memory"
    expect = (free_after + nb * block_bytes) * util - runner.kv_reserved_bytes
    assert abs(nb * block_bytes - expect) <= 0.02 * expect + 4 * block_bytes, (nb, expect / block_bytes)
    assert nb >= 64
    assert all(m.k_cache.shape[0] == nb for m in model.modules() if hasattr(m, "k_cache"))
    prompt = np.random.default_rng(5).integers(0, SMALL.vocab_size, 37).tolist()

    def serve(r):  # prefill, then one graph-replayed decode step
        s = Sequence(list(prompt))
        bm = BlockManager(r.num_available_kv_blocks, BS)
        bm.allocate(s)
        first = _prefill(r, [s])
        s.append_token(7)
        assert bm.can_append(s)
        bm.append(s)
        return first, _decode(r, [s], eager=False)

    sized = serve(runner)  # before the second runner re-attaches the model's caches
    del runner
    fixed = serve(ModelRunner(model, SMALL.runner_config(block_size=BS, num_kv_blocks=nb, max_num_seqs=4)))
    assert torch.isfinite(sized[1]).all()
    assert torch.equal(sized[0], fixed[0]) and torch.equal(sized[1], fixed[1])
    torch.cuda.empty_cache()


@torch.inference_mode()
def test_decode_steps_match_full_forward_small(block_size):
    """Prefill (with a shared cached prefix), then three decode steps crossing
    block boundaries (BS=16); graph replay == eager, replays repeatable."""
    BS = 16
    Sequence.block_size = BS
    model = DecodeModel(SMALL, device="cuda", seed=11)
    runner = ModelRunner(model, SMALL.runner_config(block_size=BS, num_kv_blocks=128, max_num_seqs=8))
    bm = BlockManager(128, BS)
    rng = np.random.default_rng(0)
    prefix = rng.integers(0, SMALL.vocab_size, 2 * BS).tolist()
    prompts = [rng.integers(0, SMALL.vocab_size, n).tolist() for n in (15, 16, 17, 47)]
    prompts.append(prefix + rng.integers(0, SMALL.vocab_size, 5).tolist())
    seqs = [Sequence(p) for p in prompts]
    for s in seqs:
        bm.allocate(s)
    later = Sequence(prefix + rng.integers(0, SMALL.vocab_size, 9).tolist())
    errs = []
    got = _prefill(runner, seqs)
    for i, s in enumerate(seqs):
        errs.append(rel_err_rows(got[i], ref_logits(model, s.token_ids)[-1]).item())
        assert errs[-1] <= e2e_tol(SMALL.num_layers), f"prefill seq {i} len {len(s)} rel err {errs[-1]:.4f}"
    # a second prefill whose first two blocks come from the prefix cache
    bm.allocate(later)
    assert later.num_cached_tokens == 2 * BS
    got = _prefill(runner, [later])
    errs.append(rel_err_rows(got[0], ref_logits(model, later.token_ids)[-1]).item())
    assert errs[-1] <= e2e_tol(SMALL.num_layers), f"cached-prefix prefill rel err {errs[-1]:.4f}"
    seqs.append(later)
    worst = {}
    for step in range(3):
        for s in seqs:
            s.append_token(int(rng.integers(0, SMALL.vocab_size)))
            assert bm.can_append(s)
            bm.append(s)
        g1 = _decode(runner, seqs, eager=False)
        e = _decode(runner, seqs, eager=True)
        g2 = _decode(runner, seqs, eager=False)
        assert torch.equal(g1, g2), f"graph replays differ at step {step}"
        assert (rel_err_rows(g1, e) <= 1e-2).all(), f"graph vs eager at step {step}"
        for i, s in enumerate(seqs):
            errs.append(rel_err_rows(g1[i], ref_logits(model, s.token_ids)[-1]).item())
            assert errs[-1] <= e2e_tol(SMALL.num_layers), f"step {step} seq {i} len {len(s)} rel err {errs[-1]:.4f}"
        for k, v in check_layers_teacher_forced(model, runner, seqs).items():
            worst[k] = max(worst.get(k, 0.0), v)
    print(f"\nsmall model: e2e rel err max {max(errs):.4f} median {np.median(errs):.4f}; "
          f"per-stage max " + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()))


WIDE = DecodeModelConfig(vocab_size=1024, d_model=2048, num_layers=2, num_heads=16, num_kv_heads=4,
                         d_ff=1024, n_routed_experts=4, num_experts_per_tok=2, max_model_length=512)


@torch.inference_mode()
def test_decode_step_wide_model_down_projection_partials(block_size):
    """d_model 2048, above the 1024 columns a 128-thread row of 8-value
    chunks covers: at 32 tokens the dense MoE dispatch splits the down
    projection (K = 5 x 1024) over K and hands its fp32 partials to the next
    layer's att_norm (and the last layer's to the final norm).  Graph replay
    equals eager, and the logits stay within the end-to-end bound of a full
    causal forward."""
    BS = 16
    Sequence.block_size = BS
    T = 32
    model = DecodeModel(WIDE, device="cuda", seed=12)
    N, Kd = model.layers[0].ffn.w2.weight.shape
    assert N == 2048 and not kernels.use_skinny_gemm(T, N, Kd)
    assert kernels.splitk_used(Kd, kernels.default_gemm_splits(T, N, Kd)) >= 2
    runner = ModelRunner(model, WIDE.runner_config(block_size=BS, num_kv_blocks=1024, max_num_seqs=T))
    bm = BlockManager(1024, BS)
    rng = np.random.default_rng(12)
    seqs = [Sequence(rng.integers(0, WIDE.vocab_size, int(n)).tolist()) for n in rng.integers(20, 300, T)]
    for s in seqs:
        bm.allocate(s)
    _prefill(runner, seqs)
    for s in seqs:
        s.append_token(int(rng.integers(0, WIDE.vocab_size)))
        assert bm.can_append(s)
        bm.append(s)
    g = _decode(runner, seqs, eager=False)
    e = _decode(runner, seqs, eager=True)
    assert torch.isfinite(g).all()
    assert (rel_err_rows(g, e) <= 1e-2).all(), "graph vs eager"
    for i in (0, 5, 17, 31):
        err = rel_err_rows(g[i], ref_logits(model, seqs[i].token_ids)[-1]).item()
        assert err <= e2e_tol(WIDE.num_layers), f"seq {i} len {len(seqs[i])} rel err {err:.4f}"


GOLDEN = Path(__file__).with_name("golden") / "model_forward.npz"
FP8_VS_FP32_TOL = 8e-2  # reference fp32 logits vs the FP8 product, 2 layers


@torch.inference_mode()
def test_reference_state_dict_decode_matches_reference_logits(block_size):
    """A reference TransformerLM state dict (GQA, MoE with a shared expert;
    the golden fixture's weights) loaded with load_reference_state_dict and
    served through the engine: a 13-token prefill, then 11 graph-replayed
    decode steps fed the fixture's tokens (crossing the 16-token block
    boundary), three sequences in one batch.  Every step's logits against
      * the reference TransformerLM's own fp32 logits for that position:
        relative L2 per row within FP8_VS_FP32_TOL -- the FP8 quantisation of
        every weight and activation (the oracle's FP8 emulation alone stands
        4.1-5.2e-2 off these logits);
      * the oracle's FP8-emulated forward on the loaded (quantised) weights:
        within e2e_tol(2), as in the other model tests."""
    g = np.load(GOLDEN)
    w = om.reference_weights(GOLDEN_DIMS, GOLDEN_SEED)
    assert om.weights_digest(w) == str(g["weights_sha256"])
    d = GOLDEN_DIMS
    cfg = DecodeModelConfig(vocab_size=d.vocab_size, d_model=d.d_model, num_layers=d.num_layers,
                            num_heads=d.num_heads, num_kv_heads=d.num_kv_heads, d_ff=d.d_ff,
                            n_routed_experts=d.n_routed_experts, num_experts_per_tok=d.num_experts_per_tok,
                            n_shared_experts=d.n_shared_experts, max_model_length=64)
    sd = {k: torch.from_numpy(v) for k, v in w.items()}
    sd["layers.0.ffn.gate.expert_load"] = torch.zeros(d.n_routed_experts, dtype=torch.long)  # ignored
    model = DecodeModel(cfg, device="cuda", seed=0).load_reference_state_dict(sd)
    assert torch.equal(model.embed.float().cpu(), sd["token_embeddings.weight"])
    BS, P = 16, 13
    Sequence.block_size = BS
    runner = ModelRunner(model, cfg.runner_config(block_size=BS, num_kv_blocks=16, max_num_seqs=4))
    bm = BlockManager(16, BS)
    tokens, want = g["tokens"], torch.from_numpy(g["logits"]).cuda()
    seqs = [Sequence(row[:P].tolist()) for row in tokens]
    for s in seqs:
        bm.allocate(s)
    steps = [(P - 1, _prefill(runner, seqs))]
    for t in range(P, tokens.shape[1]):
        for s, row in zip(seqs, tokens):
            s.append_token(int(row[t]))
            assert bm.can_append(s)
            bm.append(s)
        steps.append((t, _decode(runner, seqs, eager=False)))
    emul = [ref_logits(model, row.tolist()) for row in tokens]
    e_ref, e_emul = [], []
    for t, got in steps:
        e_ref.append(rel_err_rows(got, want[:, t]).max().item())
        e_emul.append(max(rel_err_rows(got[b], emul[b][t]).item() for b in range(len(seqs))))
    print(f"\nreference state dict: vs the reference's fp32 logits max {max(e_ref):.4f} "
          f"median {np.median(e_ref):.4f}; vs the FP8-emulated oracle max {max(e_emul):.4f}")
    assert max(e_ref) <= FP8_VS_FP32_TOL, f"vs reference logits {['%.4f' % e for e in e_ref]}"
    assert max(e_emul) <= e2e_tol(cfg.num_layers), f"vs FP8-emulated oracle {['%.4f' % e for e in e_emul]}"


@torch.inference_mode()
def test_reference_state_dict_rejects_mismatches():
    """A missing, an unexpected or a mis-shaped float tensor raises before any
    weight is loaded; integer buffers (the gate's expert_load) are ignored."""
    d = GOLDEN_DIMS
    cfg = DecodeModelConfig(vocab_size=d.vocab_size, d_model=d.d_model, num_layers=d.num_layers,
                            num_heads=d.num_heads, num_kv_heads=d.num_kv_heads, d_ff=d.d_ff,
                            n_routed_experts=d.n_routed_experts, num_experts_per_tok=d.num_experts_per_tok,
                            n_shared_experts=d.n_shared_experts, max_model_length=64)
    model = DecodeModel(cfg, device="cuda", seed=0)
    before = model.lm_head.weight.clone()
    good = {k: torch.from_numpy(v) for k, v in om.reference_weights(d, GOLDEN_SEED).items()}
    missing = dict(good)
    del missing["layers.1.ffn.shared_expert.w2.bias"]
    with pytest.raises(KeyError, match="shared_expert.w2.bias"):
        model.load_reference_state_dict(missing)
    extra = dict(good, **{"layers.0.att.head_gates_logits": torch.zeros(d.num_heads)})
    with pytest.raises(KeyError, match="head_gates_logits"):
        model.load_reference_state_dict(extra)
    bad = dict(good)
    bad["layers.0.att.k_proj.weight"] = torch.zeros(d.d_model, d.d_model)
    with pytest.raises(ValueError, match="k_proj.weight"):
        model.load_reference_state_dict(bad)
    assert torch.equal(model.lm_head.weight, before), "a rejected state dict changed the weights"
    ok = dict(good, **{"layers.0.ffn.gate.expert_load": torch.zeros(d.n_routed_experts, dtype=torch.long)})
    model.load_reference_state_dict(ok)
    assert not torch.equal(model.lm_head.weight, before)


@torch.inference_mode()
def test_decode_step_cfg5_shapes(block_size):
    """The config-5 model (12 layers, d=768, GQA 12/4, 8 experts top-2 + 1
    shared, vocab 32000) on 16 sequences with contexts in [256, 2048]."""
    BS = 256
    Sequence.block_size = BS
    cfg = DecodeModelConfig()
    model = DecodeModel(cfg, device="cuda", seed=4)
    runner = ModelRunner(model, cfg.runner_config(block_size=BS, num_kv_blocks=160, max_num_seqs=16))
    bm = BlockManager(160, BS)
    rng = np.random.default_rng(4)
    seqs = [Sequence(rng.integers(0, cfg.vocab_size, int(n)).tolist())
            for n in rng.integers(256, 2048, 16)]
    seqs[0] = Sequence(rng.integers(0, cfg.vocab_size, 4 * BS - 1).tolist())  # next token fills a block
    for s in seqs:
        bm.allocate(s)
    _prefill(runner, seqs)
    for s in seqs:
        s.append_token(int(rng.integers(0, cfg.vocab_size)))
        bm.append(s)
    got = _decode(runner, seqs, eager=False)
    worst = check_layers_teacher_forced(model, runner, seqs)
    rows = (0, 1, 7, 15)
    errs = [rel_err_rows(got[i], ref_logits(model, seqs[i].token_ids)[-1]).item() for i in rows]
    print(f"\ncfg5 model: e2e rel err {['%.4f' % e for e in errs]}; per-stage max "
          + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()))
    for i, e in zip(rows, errs):
        assert e <= e2e_tol(cfg.num_layers), f"seq {i} len {len(seqs[i])} rel err {e:.4f}"


@torch.inference_mode()
def test_decode_step_cfg5_full_batch():
    """The config-5 decode step at the bench's batch of 128 (contexts uniform
    in [256, 2048]): the bs=128 graph replay against the eager step on every
    row (1e-2 relative) and against itself (two replays bit-identical), every
    op of every layer teacher-forced against its fp32 reference, and 3
    sampled rows end to end against a full causal forward."""
    BS, B = 256, 128
    Sequence.block_size = BS
    cfg = DecodeModelConfig()
    rng = np.random.default_rng(14)
    lens = rng.integers(256, 2049, B)
    nblk = int((-(-(lens + 1) // BS)).sum())
    model = DecodeModel(cfg, device="cuda", seed=14)
    runner = ModelRunner(model, cfg.runner_config(block_size=BS, num_kv_blocks=nblk + 8, max_num_seqs=B))
    assert B in runner.graphs
    bm = BlockManager(nblk + 8, BS)
    seqs = [Sequence(rng.integers(0, cfg.vocab_size, int(n)).tolist()) for n in lens]
    for s in seqs:
        bm.allocate(s)
    for i in range(0, B, 32):  # prefill in four batches of 32 sequences
        _prefill(runner, seqs[i:i + 32])
    for s in seqs:
        s.append_token(int(rng.integers(0, cfg.vocab_size)))
        assert bm.can_append(s)
        bm.append(s)
    g1 = _decode(runner, seqs, eager=False)
    e = _decode(runner, seqs, eager=True)
    g2 = _decode(runner, seqs, eager=False)
    assert torch.equal(g1, g2), "graph replays differ"
    assert torch.isfinite(g1).all()
    err = rel_err_rows(g1, e)
    assert (err <= 1e-2).all(), f"graph vs eager: worst row {int(err.argmax())} rel err {err.max().item():.4f}"
    worst = check_layers_teacher_forced(model, runner, seqs)
    rows = (0, int(np.argmax(lens)), 77)
    errs = [rel_err_rows(g1[i], ref_logits(model, seqs[i].token_ids)[-1]).item() for i in rows]
    print(f"\ncfg5 B=128: graph vs eager max {err.max().item():.2e}; e2e rel err {['%.4f' % x for x in errs]}; "
          f"per-stage max " + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()))
    for i, x in zip(rows, errs):
        assert x <= e2e_tol(cfg.num_layers), f"seq {i} len {len(seqs[i])} rel err {x:.4f}"
    del runner, model
    torch.cuda.empty_cache()


@torch.inference_mode()
def test_engine_generate_runs_to_max_tokens(block_size):
    BS = 16
    Sequence.block_size = BS
    model = DecodeModel(SMALL, device="cuda", seed=3)
    cfg = SMALL.runner_config(block_size=BS, num_kv_blocks=24, max_num_seqs=4, max_num_sequences=4,
                              max_num_batched_tokens=256, eos=-1)
    eng = LLMEngine(model, cfg, generator=torch.Generator(device="cuda").manual_seed(0))
    rng = np.random.default_rng(5)
    prompts = [rng.integers(0, SMALL.vocab_size, n).tolist() for n in (3, 30, 17, 40, 9, 16)]
    out = eng.generate(prompts, SamplingParams(temperature=0.8, max_tokens=20))
    assert [len(t) for t in out["token_ids"]] == [20] * len(prompts)
    assert all(0 <= t < SMALL.vocab_size for toks in out["token_ids"] for t in toks)
    bm = eng.scheduler.block_manager
    assert len(bm.free_block_ids) == 24 and not bm.used_block_ids

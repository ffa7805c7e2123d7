"""GQA + MoE transformer with FP8 linears and a paged KV cache (config 5).

The layer stack is the reference's decoder (model/transformer.py:18-183,
Block with fused add & RMSNorm, model/utils.py:44-67) with its GQA
attention (model/attention/GQA.py: q_norm over d_model and k_norm over
Hkv*D before the head split, half-split RoPE from
model/attention/utils.py:18-45, SDPA scale 1/sqrt(D), no head gates) and
its MoE (model/architecture/moe.py: sigmoid gate scores, top-k on the
biased logits, renormalised weights, one shared expert, SwiGLU experts from
model/architecture/mlp.py:48-67).  Every projection is an FP8Linear.

The attention layer is the one engine/model_runner.py:8 imports but the
reference does not ship: it writes the new K/V with store_kvcache at
Context.slot_mapping; in decode it attends over the paged pool with
paged_attention_decode (Context.context_lens / block_tables), in prefill
with flash_attn_varlen_func (Context.cu_seqlens_q / _k; the pool through
block_tables on a prefix-cache hit, else the just-stored keys).

Interface (nano-vLLM style, as the runner expects):
    hidden = model(input_ids [T], positions [T])      # bf16 [T, d_model]
    logits = model.compute_logits(hidden)             # bf16 [T, vocab]

Kernels per layer: add_rmsnorm (+act_quant) -> qkv FP8 GEMM ->
qk_norm_rope_store -> paged decode (split + merge with the act_quant of its
output; where a single launch is the default split, one launch does the
norms, RoPE, slot write and attention: paged_attention_decode_rope -- in
the paired order, with the act_quant then done inside the output GEMM,
where that order applies and the GEMM is one-shot) -> output FP8 GEMM -> add_rmsnorm_route (the ffn_norm with its act_quant
and the MoE gate in one launch; add_rmsnorm then moe_route for grouped
batches) -> gate/up FP8 GEMM -> swiglu_quant -> down FP8 GEMM.  Setting ``model.trace = {}`` makes an
eager forward record every intermediate (per layer) for parity tests.

MoE in the decode step: every expert runs over the whole batch and is
weighted by the routing weight (0 for experts a token did not pick).  Each
output row depends only on its own input row (act_quant is per row, the
GEMM rows are independent), so this equals the reference's per-expert
gather/scatter (moe_infer, moe.py:288-341) while needing no host sync --
the decode step can be captured in a HIP graph -- and, since a batch of
decode tokens touches every expert anyway, it streams the same weight
bytes.  All experts together take two FP8 GEMMs (see MoE).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import NamedTuple, Optional

import torch
from torch import nn

from . import kernels
from .context import get_context
from .fp8_linear import FP8Linear


@dataclass
class DecodeModelConfig:
    vocab_size: int = 32000
    d_model: int = 768
    num_layers: int = 12
    num_heads: int = 12
    num_kv_heads: int = 4
    d_ff: int = 512
    n_routed_experts: int = 8
    num_experts_per_tok: int = 2
    n_shared_experts: int = 1
    rope_theta: float = 10000.0
    max_model_length: int = 4096
    rms_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    def runner_config(self, **kw) -> dict:
        d = dict(num_layers=self.num_layers, num_heads=self.num_heads, num_kv_heads=self.num_kv_heads,
                 hidden_size=self.d_model, head_dim=self.head_dim, max_model_length=self.max_model_length)
        d.update(kw)
        return d

    def reference_state_keys(self) -> dict[str, tuple]:
        """Float tensors of the reference's TransformerLM state dict for this
        config, name -> shape (model/transformer.py:124-160 with GQA from
        model/attention/GQA.py:34-40, MOE from model/architecture/moe.py:
        153-194 in every layer, MLP from model/architecture/mlp.py:56-58)."""
        d, F, kv = self.d_model, self.d_ff, self.num_kv_heads * self.head_dim
        keys = {"token_embeddings.weight": (self.vocab_size, d), "final_norm.weight": (d,),
                "lm_head.weight": (self.vocab_size, d), "lm_head.bias": (self.vocab_size,)}

        def lin(name, n_out, n_in):
            keys[name + ".weight"], keys[name + ".bias"] = (n_out, n_in), (n_out,)

        for i in range(self.num_layers):
            p = f"layers.{i}."
            for name, n_out in (("q_proj", d), ("k_proj", kv), ("v_proj", kv), ("output_proj", d)):
                lin(p + "att." + name, n_out, d)
            keys[p + "att.q_norm.weight"], keys[p + "att.k_norm.weight"] = (d,), (kv,)
            keys[p + "att_norm.weight"], keys[p + "ffn_norm.weight"] = (d,), (d,)
            keys[p + "ffn.gate.weight"] = (self.n_routed_experts, d)
            keys[p + "ffn.gate.expert_bias"] = (self.n_routed_experts,)
            mlps = [f"ffn.experts.{e}" for e in range(self.n_routed_experts)]
            mlps += ["ffn.shared_expert"] if self.n_shared_experts > 0 else []
            for m in mlps:
                lin(p + m + ".w1", F, d)
                lin(p + m + ".w3", F, d)
                lin(p + m + ".w2", d, F)
        return keys


class SplitKOutput(NamedTuple):
    """An FP8 linear's output left as its split-K partial sums (fp32 [n, T, d])
    and bias: the next add & norm reduces it (kernels.add_rmsnorm_partials),
    so the reduction costs no launch of its own."""
    parts: torch.Tensor
    bias: Optional[torch.Tensor]


class RMSNorm(nn.Module):
    """model/utils.py:44-67: fp32 compute, optional fused residual add; runs
    as one add_rmsnorm launch (optionally also quantising its output)."""

    def __init__(self, d: int, eps: float = 1e-5, device=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d, dtype=torch.float32, device=device))

    def forward(self, x, residual: Optional[torch.Tensor] = None, out: bool = True, quant: bool = False):
        """-> (out, residual_out, q, q_scale); residual_out is x without a
        residual (the reference returns (norm(x), x) in that case).  x is a
        bf16 tensor or a SplitKOutput (then a residual is required)."""
        if isinstance(x, SplitKOutput):
            assert residual is not None
            return kernels.add_rmsnorm_partials(x.parts, x.bias, self.weight, self.eps, residual, out=out,
                                                quant=quant)
        return kernels.add_rmsnorm(x, self.weight, self.eps, residual, out=out, quant=quant)


class Rotary(nn.Module):
    """Half-split RoPE table cat(cos, sin) [max_seq_len, D]
    (model/attention/utils.py:18-31); applied inside qk_norm_rope_store."""

    def __init__(self, theta: float, d_k: int, max_seq_len: int, device=None):
        super().__init__()
        inv_freq = 1.0 / (theta ** (torch.arange(0, d_k, 2, device=device).float() / d_k))
        ang = torch.outer(torch.arange(max_seq_len, device=device).float(), inv_freq)
        self.register_buffer("cos_sin_cached", torch.cat([ang.cos(), ang.sin()], -1), persistent=False)


class PagedGQAAttention(nn.Module):
    def __init__(self, cfg: DecodeModelConfig, rope: Rotary, device=None):
        super().__init__()
        d, D = cfg.d_model, cfg.head_dim
        self.num_heads, self.num_kv_heads, self.head_dim = cfg.num_heads, cfg.num_kv_heads, D
        self.scale = 1.0 / math.sqrt(D)
        # q_proj, k_proj and v_proj (GQA.py:34-36) as one FP8 linear: their
        # row blocks start at multiples of 128, so quantising the stacked
        # weight gives the same codes and scales as quantising each one, and
        # every output column of the GEMM is independent of the others
        self.q_dim, self.kv_dim = d, cfg.num_kv_heads * D
        self.qkv_proj = FP8Linear(d, d + 2 * self.kv_dim, device=device)
        self.output_proj = FP8Linear(d, d, device=device)
        # torch.nn.RMSNorm default eps (machine epsilon of the fp32 compute)
        self.q_norm = RMSNorm(d, eps=torch.finfo(torch.float32).eps, device=device)
        self.k_norm = RMSNorm(cfg.num_kv_heads * D, eps=torch.finfo(torch.float32).eps, device=device)
        self.rope = rope
        self.k_cache = torch.empty(0)  # pool views attached by the model runner
        self.v_cache = torch.empty(0)

    def forward(self, xq: torch.Tensor, xs: torch.Tensor, positions: torch.Tensor,
                trace: Optional[dict] = None) -> torch.Tensor:
        """xq, xs: the attention input already quantised (act_quant codes and
        1x128 scales of the att_norm output)."""
        ctx = get_context()
        T = xq.size(0)
        assert self.k_cache.numel(), "PagedGQAAttention needs the KV pool (ModelRunner.allocate_kv_cache)"
        qkv = self.qkv_proj.gemm(xq, xs)
        shape = (T, self.num_heads, self.num_kv_heads, self.head_dim, ctx.block_tables.size(1),
                 self.k_cache.size(1)) if not ctx.is_prefill else None
        # the paired order (one workgroup per (sequence, kv head), a long and
        # a short one per CU) when the output projection can quantise its
        # input itself; else one workgroup per pair of kv heads with the
        # act_quant fused into the attention
        paired = (shape is not None and kernels.decode_rope_paired(*shape)
                  and self.output_proj.fused_act(T))
        if paired or (shape is not None and kernels.use_fused_decode_rope(*shape)):
            # q/k norms, RoPE, the slot write and the attention in one launch
            q = torch.empty(T, self.num_heads, self.head_dim, dtype=torch.bfloat16,
                            device=qkv.device) if trace is not None else None
            res = kernels.paged_attention_decode_rope(
                qkv, self.q_norm.weight, self.k_norm.weight, self.rope.cos_sin_cached, positions,
                self.num_heads, self.num_kv_heads, self.q_norm.eps, self.k_cache, self.v_cache,
                ctx.slot_mapping, ctx.context_lens, ctx.block_tables, self.scale, quant=not paired, q_rot=q)
            if paired:
                o = res.reshape(T, -1)
                out = self.output_proj(o)  # act_quant inside the GEMM
            else:
                o, oq, os_ = res
                o = o.reshape(T, -1)
                out = self.output_proj.gemm(oq, os_)
            if trace is not None:
                trace.update(qkv=qkv, q=q, att_o=o, att_out=out)
            return out
        q = kernels.qk_norm_rope_store(qkv, self.q_norm.weight, self.k_norm.weight, self.rope.cos_sin_cached,
                                       positions, self.num_heads, self.num_kv_heads, self.q_norm.eps,
                                       self.k_cache, self.v_cache, ctx.slot_mapping)
        if ctx.is_prefill:
            if ctx.block_tables is not None:  # prefix-cache hit: keys from the pool
                o = kernels.flash_attn_varlen_func(q, self.k_cache, self.v_cache, ctx.cu_seqlens_q,
                                                   ctx.cu_seqlens_k, ctx.max_seqlen_q, ctx.max_seqlen_k,
                                                   self.scale, block_table=ctx.block_tables)
            else:  # whole prompts: the keys just stored, in slot order
                flat = (-1, self.num_kv_heads, self.head_dim)
                k = self.k_cache.view(flat)[ctx.slot_mapping]
                v = self.v_cache.view(flat)[ctx.slot_mapping]
                o = kernels.flash_attn_varlen_func(q, k, v, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                                   ctx.max_seqlen_q, ctx.max_seqlen_k, self.scale)
            o = o.reshape(T, -1)
            out = self.output_proj(o)
        else:
            # the merge also writes the output projection's FP8 input (act_quant fused)
            o, oq, os_ = kernels.paged_attention_decode(q, self.k_cache, self.v_cache, ctx.context_lens,
                                                        ctx.block_tables, self.scale, quant=True)
            o = o.reshape(T, -1)
            out = self.output_proj.gemm(oq, os_)
        if trace is not None:
            trace.update(qkv=qkv, q=q, att_o=o, att_out=out)
        return out


class MoE(nn.Module):
    """Routed experts + one shared expert (model/architecture/moe.py:160-260),
    each a SwiGLU MLP w2(silu(w1 x) * w3 x) with biases
    (model/architecture/mlp.py:48-67), computed densely over experts:
      * moe_route: sigmoid gate, top-k of the biased logits, renormalised
        weights as a dense [T, E+1] matrix (shared expert 1, unpicked 0) and
        the bias matrix sum_e w_e * b2_e;
      * one FP8 GEMM with every expert's w1 and w3 stacked along N (rows
        [e][w1 | w3], blocks aligned to 128, so the codes and scales equal
        per-expert quantisation);
      * swiglu_quant: SwiGLU in bf16 as the reference rounds it, act_quant of
        all the experts' hidden rows at once (128-groups never straddle
        experts, d_ff % 128 == 0), each group's scale multiplied by the
        token's routing weight for that expert;
      * one FP8 GEMM with every expert's w2 stacked along K, so the fp32
        accumulator sums sum_e w_e * (w2_e h_e) directly, plus the bias
        matrix.
    The reference rounds each expert's output to bf16 and scatter-adds in
    bf16 (moe.py:288-341); here the weighted sum is rounded once.

    Grouped dispatch (prefill-sized batches, ``dispatch`` "grouped", or
    "auto" with more than GROUPED_MIN_TOKENS tokens): only the picked
    experts run.  moe_route also returns the picks in index form,
    moe_align groups the (token, pick) entries by expert into 128-row
    tiles on the GPU (no host sync), one grouped FP8 GEMM runs w13 over
    each expert's gathered rows (the same stacked weights, viewed
    [E, 2F, d]), swiglu_quant folds each row's routing weight into its
    scales, a second grouped GEMM runs w2 (the K-stacked matrix viewed
    [E, d, F]) into bf16 rows (each expert's weighted output rounded once,
    as the reference rounds each expert's output), and moe_combine sums
    each token's rows and its weighted down biases in fp32, rounding once
    more.  The two dispatches agree to a bf16 rounding per expert."""

    GROUPED_MIN_TOKENS = 256

    def __init__(self, cfg: DecodeModelConfig, device=None):
        super().__init__()
        self.top_k = cfg.num_experts_per_tok
        self.n_experts = cfg.n_routed_experts
        self.n_shared = 1 if cfg.n_shared_experts > 0 else 0
        self.d_ff = cfg.d_ff
        assert cfg.d_ff % 128 == 0, "d_ff must be a multiple of 128"
        E = self.n_experts + self.n_shared
        self.gate_weight = nn.Parameter(torch.empty(cfg.n_routed_experts, cfg.d_model, device=device,
                                                    dtype=torch.bfloat16))
        self.register_buffer("expert_bias", torch.zeros(cfg.n_routed_experts, device=device))
        self.w13 = FP8Linear(cfg.d_model, E * 2 * cfg.d_ff, device=device)
        self.w2 = FP8Linear(E * cfg.d_ff, cfg.d_model, bias=False, device=device)
        self.register_buffer("w2_bias", torch.zeros(E, cfg.d_model, device=device))
        self.dispatch = "auto"  # "dense" | "grouped" | "auto"

    def _expert_views(self):
        """Per-expert views of the stacked weights for the grouped GEMMs:
        w13 [E, 2F, d] (+ scales [E, 2F/128, d/128], bias [E, 2F]) and w2
        [E, d, F] (columns e*F .. of the K-stacked matrix; scales
        [E, ceil(d/128), F/128])."""
        E, F = self.n_experts + self.n_shared, self.d_ff
        d = self.w2.out_features
        w13 = self.w13.weight.view(E, 2 * F, d)
        w13s = self.w13.weight_scale.view(E, 2 * F // 128, d // 128)
        b13 = self.w13.bias.view(E, 2 * F)
        w2 = self.w2.weight.view(d, E, F).permute(1, 0, 2)
        w2s = self.w2.weight_scale.view(-1, E, F // 128).permute(1, 0, 2)
        return w13, w13s, b13, w2, w2s

    @torch.no_grad()
    def load_experts(self, experts: list[tuple]) -> None:
        """experts: (w1 [F, d], b1, w3 [F, d], b3, w2 [d, F], b2) per routed
        expert, then the shared expert."""
        w13 = torch.cat([torch.cat([w1, w3]) for w1, _, w3, _, _, _ in experts])
        b13 = torch.cat([torch.cat([b1, b3]) for _, b1, _, b3, _, _ in experts])
        self.w13.load_weight(w13, b13)
        self.w2.load_weight(torch.cat([e[4] for e in experts], dim=1))
        self.w2_bias.copy_(torch.stack([e[5] for e in experts]).float())

    def forward(self, h: torch.Tensor, hq: torch.Tensor, hs: torch.Tensor,
                trace: Optional[dict] = None) -> torch.Tensor:
        """h: the ffn_norm output (bf16, for the gate); hq, hs: the same
        quantised (for the experts)."""
        T = h.size(0)
        if not self.dense_dispatch(T):
            return self.forward_grouped(h, hq, hs, trace)
        w, bias = kernels.moe_route(h, self.gate_weight, self.expert_bias, self.w2_bias, self.top_k,
                                    self.n_shared)
        return self.forward_routed(hq, hs, w, bias, trace)

    def dense_dispatch(self, T: int) -> bool:
        """Every expert over every token (small batches) rather than grouped."""
        return not (self.dispatch == "grouped" or (self.dispatch == "auto" and T > self.GROUPED_MIN_TOKENS))

    def forward_routed(self, hq: torch.Tensor, hs: torch.Tensor, w: torch.Tensor, bias: torch.Tensor,
                       trace: Optional[dict] = None, partials: bool = False):
        """The dense dispatch given the gate's weights and routed bias (from
        moe_route, or from add_rmsnorm_route together with the ffn_norm).
        With ``partials`` (and a down projection the dispatch splits over K)
        the result is a SplitKOutput for the next add & norm to reduce."""
        T, F = hq.size(0), self.d_ff
        h13 = self.w13.gemm(hq, hs)
        gq, gs = kernels.swiglu_quant(h13.view(T, -1, 2, F), w)
        N, K = self.w2.weight.shape
        if partials and trace is None and not kernels.use_skinny_gemm(T, N, K):
            splits = kernels.default_gemm_splits(T, N, K)
            if kernels.splitk_used(K, splits) >= 2:
                parts = kernels.fp8_gemm_splitk_partials(gq, gs, self.w2.weight, self.w2.weight_scale, splits)
                return SplitKOutput(parts, bias)
        y = kernels.fp8_gemm(gq, gs, self.w2.weight, self.w2.weight_scale, bias)
        if trace is not None:
            trace.update(route_w=w, route_bias=bias, h13=h13, ffn_out=y)
        return y

    def forward_grouped(self, h: torch.Tensor, hq: torch.Tensor, hs: torch.Tensor,
                        trace: Optional[dict] = None) -> torch.Tensor:
        """MoE.moe_infer (model/architecture/moe.py:288-341) plus the shared
        expert, with only the picked experts computed."""
        E, S, F = self.n_experts, self.n_shared, self.d_ff
        _, _, idx, wt = kernels.moe_route(h, self.gate_weight, self.expert_bias, None, self.top_k, S,
                                          dense=False, return_topk=True)
        rows = kernels.moe_align(idx, wt, E, S)
        w13, w13s, b13, w2, w2s = self._expert_views()
        h13 = kernels.fp8_grouped_gemm(hq, hs, rows.row_token, rows.tile_expert, w13, w13s, b13)
        P = rows.num_rows
        gq, gs = kernels.swiglu_quant(h13.view(P, 1, 2, F), rows.row_weight.view(P, 1))
        # bf16 expert rows (the reference also rounds each expert's output), fp32 sum
        out = kernels.fp8_grouped_gemm(gq, gs, None, rows.tile_expert, w2, w2s)
        y = kernels.moe_combine(out, rows.entry_row, idx, wt, E, S, self.w2_bias)
        if trace is not None:
            trace.update(topk_idx=idx, topk_weight=wt, moe_rows=rows, h13_rows=h13, ffn_out=y)
        return y


class Block(nn.Module):
    def __init__(self, cfg: DecodeModelConfig, rope: Rotary, device=None):
        super().__init__()
        self.att = PagedGQAAttention(cfg, rope, device)
        self.ffn = MoE(cfg, device)
        self.att_norm = RMSNorm(cfg.d_model, cfg.rms_eps, device)
        self.ffn_norm = RMSNorm(cfg.d_model, cfg.rms_eps, device)

    def forward(self, x, residual, positions, trace: Optional[dict] = None):
        """Fused add & norm before attention and before the MoE
        (model/transformer.py:90-118)."""
        if trace is not None:
            trace.update(x=x, residual=residual)
        h, residual, hq, hs = self.att_norm(x, residual, out=trace is not None, quant=True)
        x = self.att(hq, hs, positions, trace)
        if self.ffn.dense_dispatch(x.size(0)):
            # ffn_norm and the MoE gate in one launch (the same results as the pair)
            ffn = self.ffn
            h2, residual, hq, hs, w, bias = kernels.add_rmsnorm_route(
                x, self.ffn_norm.weight, self.ffn_norm.eps, residual, ffn.gate_weight, ffn.expert_bias,
                ffn.w2_bias, ffn.top_k, ffn.n_shared, out=trace is not None)
            if trace is not None:
                trace.update(att_h=h, ffn_h=h2, res_mid=residual)
            return ffn.forward_routed(hq, hs, w, bias, trace, partials=True), residual
        h2, residual, hq, hs = self.ffn_norm(x, residual, out=True, quant=True)
        if trace is not None:
            trace.update(att_h=h, ffn_h=h2, res_mid=residual)
        return self.ffn(h2, hq, hs, trace), residual


class DecodeModel(nn.Module):
    def __init__(self, cfg: DecodeModelConfig, device="cuda", seed: int = 4):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Parameter(torch.empty(cfg.vocab_size, cfg.d_model, device=device, dtype=torch.bfloat16))
        self.rope = Rotary(cfg.rope_theta, cfg.head_dim, cfg.max_model_length, device)
        self.layers = nn.ModuleList([Block(cfg, self.rope, device) for _ in range(cfg.num_layers)])
        self.final_norm = RMSNorm(cfg.d_model, cfg.rms_eps, device)
        self.lm_head = FP8Linear(cfg.d_model, cfg.vocab_size, device=device)
        self.trace: Optional[dict] = None
        self.init_weights(seed)

    @torch.no_grad()
    def init_weights(self, seed: int) -> None:
        """nn.Linear's default init (uniform +-1/sqrt(fan_in) for weight and
        bias), clamped-normal embedding, from one seeded generator."""
        g = torch.Generator(device=self.embed.device)
        g.manual_seed(seed)
        dev = self.embed.device

        def uniform(shape, bound):
            return (torch.rand(shape, generator=g, device=dev) * 2 - 1) * bound

        self.embed.copy_(torch.randn(self.embed.shape, generator=g, device=dev).clamp_(-3, 3))
        experts = {id(lin) for layer in self.layers for lin in (layer.ffn.w13, layer.ffn.w2)}
        for m in self.modules():
            if isinstance(m, MoE):
                m.gate_weight.copy_(uniform(m.gate_weight.shape, 1.0 / math.sqrt(m.gate_weight.shape[1])))
                d, F = m.gate_weight.shape[1], m.d_ff
                bd, bf = 1.0 / math.sqrt(d), 1.0 / math.sqrt(F)
                m.load_experts([(uniform((F, d), bd), uniform((F,), bd), uniform((F, d), bd), uniform((F,), bd),
                                 uniform((d, F), bf), uniform((d,), bf))
                                for _ in range(m.n_experts + m.n_shared)])
            elif isinstance(m, FP8Linear) and id(m) not in experts:
                b = 1.0 / math.sqrt(m.in_features)
                m.load_weight(uniform((m.out_features, m.in_features), b),
                              uniform((m.out_features,), b) if m.bias is not None else None)

    @torch.no_grad()
    def load_reference_state_dict(self, sd) -> "DecodeModel":
        """Load the weights of a reference TransformerLM (attention_type
        "GQA", use_moe with MoE in every layer, at most one shared expert)
        from its state dict: q/k/v projections stacked into qkv_proj, each
        layer's experts and then its shared expert stacked into w13 / w2,
        every projection quantised to e4m3 with 128x128 block scales, the
        embedding and gate weights rounded to bf16.  Non-float buffers
        (the gate's expert_load counts) are ignored; a missing, unexpected
        or mis-shaped float tensor raises."""
        want = self.cfg.reference_state_keys()
        have = {k for k, v in sd.items() if torch.is_tensor(v) and v.is_floating_point()}
        if have != set(want):
            raise KeyError(f"reference state dict mismatch: missing {sorted(set(want) - have)}, "
                           f"unexpected {sorted(have - set(want))}")
        for k, shape in want.items():
            if tuple(sd[k].shape) != shape:
                raise ValueError(f"{k}: shape {tuple(sd[k].shape)}, expected {shape}")
        dev = self.embed.device

        def t(k):
            return sd[k].to(device=dev, dtype=torch.float32)

        self.embed.copy_(t("token_embeddings.weight"))
        self.final_norm.weight.copy_(t("final_norm.weight"))
        self.lm_head.load_weight(t("lm_head.weight"), t("lm_head.bias"))
        for i, blk in enumerate(self.layers):
            p = f"layers.{i}."
            a = blk.att
            a.qkv_proj.load_weight(torch.cat([t(p + f"att.{n}.weight") for n in ("q_proj", "k_proj", "v_proj")]),
                                   torch.cat([t(p + f"att.{n}.bias") for n in ("q_proj", "k_proj", "v_proj")]))
            a.output_proj.load_weight(t(p + "att.output_proj.weight"), t(p + "att.output_proj.bias"))
            a.q_norm.weight.copy_(t(p + "att.q_norm.weight"))
            a.k_norm.weight.copy_(t(p + "att.k_norm.weight"))
            blk.att_norm.weight.copy_(t(p + "att_norm.weight"))
            blk.ffn_norm.weight.copy_(t(p + "ffn_norm.weight"))
            f = blk.ffn
            f.gate_weight.copy_(t(p + "ffn.gate.weight"))
            f.expert_bias.copy_(t(p + "ffn.gate.expert_bias"))
            mlps = [f"ffn.experts.{e}" for e in range(f.n_experts)] + (["ffn.shared_expert"] if f.n_shared else [])
            f.load_experts([tuple(t(p + m + s) for s in (".w1.weight", ".w1.bias", ".w3.weight", ".w3.bias",
                                                         ".w2.weight", ".w2.bias")) for m in mlps])
        return self

    def _forward(self, input_ids: torch.Tensor, positions: torch.Tensor, quant: bool):
        x = self.embed[input_ids]
        residual = None
        tr = self.trace
        for i, layer in enumerate(self.layers):
            x, residual = layer(x, residual, positions, None if tr is None else tr.setdefault(i, {}))
        h, _, hq, hs = self.final_norm(x, residual, quant=quant)
        if tr is not None:
            tr["final"] = dict(x=x, residual=residual, h=h)
        return h, hq, hs

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        return self._forward(input_ids, positions, quant=False)[0]

    def forward_q(self, input_ids: torch.Tensor, positions: torch.Tensor):
        """forward, plus the act_quant codes and scales of its output (the
        lm_head's FP8 input) from the final norm's launch: (h, hq, hs)."""
        return self._forward(input_ids, positions, quant=True)

    def compute_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        logits = self.lm_head(hidden)
        if self.trace is not None:
            self.trace["final"].update(head_in=hidden, logits=logits)
        return logits

    def compute_logits_q(self, hq: torch.Tensor, hs: torch.Tensor) -> torch.Tensor:
        """compute_logits on an input already quantised (forward_q)."""
        return self.lm_head.gemm(hq, hs)

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
Context.slot_mapping and, in decode, attends over the paged pool with
paged_attention_decode (Context.context_lens / block_tables).

Interface (nano-vLLM style, as the runner expects):
    hidden = model(input_ids [T], positions [T])      # bf16 [T, d_model]
    logits = model.compute_logits(hidden)             # bf16 [T, vocab]

MoE in the decode step: every expert runs over the whole batch and is
weighted by the routing weight (0 for experts a token did not pick).  Each
output row depends only on its own input row (act_quant is per row, the
GEMM rows are independent), so this equals the reference's per-expert
gather/scatter (moe_infer, moe.py:288-341) while needing no host sync --
the decode step can be captured in a HIP graph -- and, since a batch of
decode tokens touches every expert anyway, it streams the same weight
bytes.  Expert outputs are accumulated in fp32 and rounded once.
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

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


class RMSNorm(nn.Module):
    """model/utils.py:44-67: fp32 compute, optional fused residual add."""

    def __init__(self, d: int, eps: float = 1e-5, device=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d, dtype=torch.float32, device=device))

    def forward(self, x: torch.Tensor, residual: Optional[torch.Tensor] = None):
        dtype = x.dtype
        if residual is None:
            x = x.float()
            return (self.weight * x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)).to(dtype)
        x = x.float().add_(residual.float())
        residual = x
        out = self.weight * x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + self.eps)
        return out.to(dtype), residual.to(dtype)


class Rotary(nn.Module):
    """Half-split RoPE with a cat(cos, sin) table (model/attention/utils.py:18-45)."""

    def __init__(self, theta: float, d_k: int, max_seq_len: int, device=None):
        super().__init__()
        inv_freq = 1.0 / (theta ** (torch.arange(0, d_k, 2, device=device).float() / d_k))
        ang = torch.outer(torch.arange(max_seq_len, device=device).float(), inv_freq)
        self.register_buffer("cos_sin_cached", torch.cat([ang.cos(), ang.sin()], -1), persistent=False)

    def forward(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        # x [T, H, D], positions [T]
        cos, sin = self.cos_sin_cached[positions].unsqueeze(1).chunk(2, dim=-1)
        x1, x2 = x.float().chunk(2, dim=-1)
        return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), dim=-1)


class PagedGQAAttention(nn.Module):
    def __init__(self, cfg: DecodeModelConfig, rope: Rotary, device=None):
        super().__init__()
        d, D = cfg.d_model, cfg.head_dim
        self.num_heads, self.num_kv_heads, self.head_dim = cfg.num_heads, cfg.num_kv_heads, D
        self.scale = 1.0 / math.sqrt(D)
        self.q_proj = FP8Linear(d, d, device=device)
        self.k_proj = FP8Linear(d, cfg.num_kv_heads * D, device=device)
        self.v_proj = FP8Linear(d, cfg.num_kv_heads * D, device=device)
        self.output_proj = FP8Linear(d, d, device=device)
        # torch.nn.RMSNorm default eps (machine epsilon of the fp32 compute)
        self.q_norm = RMSNorm(d, eps=torch.finfo(torch.float32).eps, device=device)
        self.k_norm = RMSNorm(cfg.num_kv_heads * D, eps=torch.finfo(torch.float32).eps, device=device)
        self.rope = rope
        self.k_cache = torch.empty(0)  # pool views attached by the model runner
        self.v_cache = torch.empty(0)

    def qkv(self, x: torch.Tensor, positions: torch.Tensor):
        T = x.size(0)
        q = self.q_norm(self.q_proj(x)).view(T, self.num_heads, self.head_dim)
        k = self.k_norm(self.k_proj(x)).view(T, self.num_kv_heads, self.head_dim)
        v = self.v_proj(x).view(T, self.num_kv_heads, self.head_dim)
        q = self.rope(q, positions).to(torch.bfloat16)
        k = self.rope(k, positions).to(torch.bfloat16)
        return q, k, v

    def forward(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        ctx = get_context()
        q, k, v = self.qkv(x, positions)
        if self.k_cache.numel():
            kernels.store_kvcache(k, v, self.k_cache, self.v_cache, ctx.slot_mapping)
        if ctx.is_prefill:
            o = self._prefill_attention(q, k, v, ctx)
        else:
            o = kernels.paged_attention_decode(q.contiguous(), self.k_cache, self.v_cache,
                                               ctx.context_lens, ctx.block_tables, self.scale)
        return self.output_proj(o.reshape(x.size(0), -1))

    def _prefill_attention(self, q, k, v, ctx) -> torch.Tensor:
        """Causal attention of each prompt over its full context (cached
        prefix gathered from the pool).  fp32, one sequence at a time."""
        G = self.num_heads // self.num_kv_heads
        cu_q = ctx.cu_seqlens_q.tolist()
        cu_k = ctx.cu_seqlens_k.tolist()
        out = torch.empty_like(q)
        BS = self.k_cache.size(1) if self.k_cache.numel() else 1
        for i in range(len(cu_q) - 1):
            qs, qe, lk = cu_q[i], cu_q[i + 1], cu_k[i + 1] - cu_k[i]
            lq = qe - qs
            if ctx.block_tables is not None and lk > lq:
                t = torch.arange(lk, device=q.device)
                blocks = ctx.block_tables[i].long()[t // BS]
                K = self.k_cache[blocks, t % BS]
                V = self.v_cache[blocks, t % BS]
            else:
                K, V = k[qs:qe], v[qs:qe]
            Kh = K.float().repeat_interleave(G, dim=1).transpose(0, 1)  # [Hq, lk, D]
            Vh = V.float().repeat_interleave(G, dim=1).transpose(0, 1)
            Q = q[qs:qe].float().transpose(0, 1)                          # [Hq, lq, D]
            s = torch.matmul(Q, Kh.transpose(1, 2).contiguous()) * self.scale
            pos_q = torch.arange(lk - lq, lk, device=q.device)
            mask = torch.arange(lk, device=q.device)[None, :] <= pos_q[:, None]
            s = s.masked_fill(~mask, float("-inf"))
            out[qs:qe] = torch.matmul(torch.softmax(s, -1), Vh).transpose(0, 1).to(out.dtype)
        return out


class MLP(nn.Module):
    """SwiGLU: w2(silu(w1 x) * w3 x) (model/architecture/mlp.py:48-67)."""

    def __init__(self, d: int, d_ff: int, device=None):
        super().__init__()
        self.w1 = FP8Linear(d, d_ff, device=device)
        self.w3 = FP8Linear(d, d_ff, device=device)
        self.w2 = FP8Linear(d_ff, d, device=device)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w2(torch.nn.functional.silu(self.w1(x)) * self.w3(x))


class MoE(nn.Module):
    def __init__(self, cfg: DecodeModelConfig, device=None):
        super().__init__()
        self.top_k = cfg.num_experts_per_tok
        self.n_experts = cfg.n_routed_experts
        self.gate_weight = nn.Parameter(torch.empty(cfg.n_routed_experts, cfg.d_model, device=device,
                                                    dtype=torch.bfloat16))
        self.register_buffer("expert_bias", torch.zeros(cfg.n_routed_experts, device=device))
        self.experts = nn.ModuleList([MLP(cfg.d_model, cfg.d_ff, device) for _ in range(cfg.n_routed_experts)])
        self.shared_expert = MLP(cfg.d_model, cfg.d_ff, device) if cfg.n_shared_experts > 0 else None

    def route(self, x: torch.Tensor):
        """Gate (moe.py:45-90): sigmoid scores, top-k of the biased logits,
        weights renormalised over the chosen experts; dense [T, E] weights."""
        logits = x.float() @ self.gate_weight.float().t()
        scores = torch.sigmoid(logits)
        idx = torch.topk(logits + self.expert_bias, self.top_k, dim=-1, sorted=False).indices
        w = torch.gather(scores, -1, idx)
        if self.top_k > 1:
            w = w / (w.sum(-1, keepdim=True) + 1e-10)
        return torch.zeros_like(scores).scatter_(1, idx, w), idx

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        dense_w, _ = self.route(x)
        y = torch.zeros(x.shape, dtype=torch.float32, device=x.device)
        for e, expert in enumerate(self.experts):
            y += dense_w[:, e:e + 1] * expert(x).float()
        if self.shared_expert is not None:
            y += self.shared_expert(x).float()
        return y.to(x.dtype)


class Block(nn.Module):
    def __init__(self, cfg: DecodeModelConfig, rope: Rotary, device=None):
        super().__init__()
        self.att = PagedGQAAttention(cfg, rope, device)
        self.ffn = MoE(cfg, device)
        self.att_norm = RMSNorm(cfg.d_model, cfg.rms_eps, device)
        self.ffn_norm = RMSNorm(cfg.d_model, cfg.rms_eps, device)

    def forward(self, x, residual, positions):
        if residual is None:
            x, residual = self.att_norm(x), x
        else:
            x, residual = self.att_norm(x, residual)
        x = self.att(x, positions)
        x, residual = self.ffn_norm(x, residual)
        return self.ffn(x), residual


class DecodeModel(nn.Module):
    def __init__(self, cfg: DecodeModelConfig, device="cuda", seed: int = 4):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Parameter(torch.empty(cfg.vocab_size, cfg.d_model, device=device, dtype=torch.bfloat16))
        self.rope = Rotary(cfg.rope_theta, cfg.head_dim, cfg.max_model_length, device)
        self.layers = nn.ModuleList([Block(cfg, self.rope, device) for _ in range(cfg.num_layers)])
        self.final_norm = RMSNorm(cfg.d_model, cfg.rms_eps, device)
        self.lm_head = FP8Linear(cfg.d_model, cfg.vocab_size, device=device)
        self.init_weights(seed)

    @torch.no_grad()
    def init_weights(self, seed: int) -> None:
        """nn.Linear's default init (uniform +-1/sqrt(fan_in) for weight and
        bias), truncated-normal embedding, from one seeded generator."""
        g = torch.Generator(device=self.embed.device)
        g.manual_seed(seed)
        dev = self.embed.device

        def uniform(shape, bound):
            return (torch.rand(shape, generator=g, device=dev) * 2 - 1) * bound

        self.embed.copy_(torch.randn(self.embed.shape, generator=g, device=dev).clamp_(-3, 3))
        for m in self.modules():
            if isinstance(m, FP8Linear):
                b = 1.0 / math.sqrt(m.in_features)
                m.load_weight(uniform((m.out_features, m.in_features), b),
                              uniform((m.out_features,), b) if m.bias is not None else None)
            elif isinstance(m, MoE):
                m.gate_weight.copy_(uniform(m.gate_weight.shape, 1.0 / math.sqrt(m.gate_weight.shape[1])))

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        x = self.embed[input_ids]
        residual = None
        for layer in self.layers:
            x, residual = layer(x, residual, positions)
        x, _ = self.final_norm(x, residual)
        return x

    def compute_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        return self.lm_head(hidden)

"""fp32 restatement of the reference's GQA + MoE decoder forward (torch).
TEST INFRASTRUCTURE: the checker for the decode model; only ``tests/`` use it.

Reference semantics (``/root/reference/model/``):
  * TransformerLM.forward: token embedding, the blocks, final norm fused
    with the last residual add, lm_head .................. transformer.py:162-183
  * Block.forward: att_norm (fused add once a residual exists), attention,
    ffn_norm (fused add), MoE ........................... transformer.py:90-118
  * RMSNorm: x (+ residual) in fp32, w * x * rsqrt(mean(x^2) + eps), cast
    back to the input dtype; the sum is the new residual . utils.py:44-67
  * GroupedQueryAttention: q_proj then q_norm over all of d_model, k_proj
    then k_norm over Hkv*D (torch.nn.RMSNorm with fp32 weights: eps is the
    fp32 machine epsilon, output fp32), v_proj; heads split after the
    norms; half-split RoPE on q and k; query head h reads kv head h // G;
    SDPA with a boolean causal mask; output_proj ......... attention/GQA.py:65-139
  * RotaryPositionalEmbedding: angles pos * theta^(-2i/D), y1 = x1 cos -
    x2 sin, y2 = x2 cos + x1 sin over the two halves ...... attention/utils.py:18-45
  * Gate: sigmoid of x @ W^T; top-k of logits + expert_bias (the bias
    only selects); weights gathered from the unbiased scores and divided
    by their sum + 1e-10 ................................. architecture/moe.py:45-90
  * moe_infer: each token's chosen experts' outputs times their weights,
    summed; the shared expert added on top .............. architecture/moe.py:272-273, 289-341
  * MLP: w2(silu(w1 x) * w3 x), every projection with a bias
    ..................................................... architecture/mlp.py:48-67

Weights are a dict in the reference's state-dict layout (``token_embeddings.
weight``, ``layers.{i}.att.q_proj.weight``, ``layers.{i}.ffn.experts.{e}.w1.
weight``, ``layers.{i}.ffn.gate.expert_bias``, ``layers.{i}.ffn.shared_expert.
w2.bias``, ``lm_head.bias`` ...).  ``forward`` takes the projection as an
argument, so the same composition checks the FP8 product (a linear that
emulates act_quant + the block-scaled GEMM, bf16 activations) and is itself
checked in fp32 against logits the reference's own TransformerLM wrote.

Pinning (tests/test_oracle_model.py): ``forward`` in fp32 on the weights of
``reference_weights`` equals the logits of the reference's TransformerLM.
forward on the same weights and tokens (tests/golden/model_forward.npz,
written by tests/golden/make_model_golden.py) to 2e-5 (measured 7e-7);
nine planted mistakes (interleaved RoPE, head map h % Hkv, per-head q_norm,
a softmax gate, biased scores as weights, no renormalisation, dropped
biases, the newest token not attended, the residual stream dropped) each
miss those logits by 2.7e-2 or more.
"""
from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass
from typing import Callable, Optional

import numpy as np
import torch

from .fp8 import bf16_round

FP32_EPS = float(np.finfo(np.float32).eps)


@dataclass(frozen=True)
class ModelDims:
    """Shape of a GQA + MoE TransformerLM (model/config.py field names)."""
    vocab_size: int
    d_model: int
    num_layers: int
    num_heads: int
    num_kv_heads: int
    d_ff: int
    n_routed_experts: int
    num_experts_per_tok: int
    n_shared_experts: int = 1
    rope_theta: float = 10000.0
    rms_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads


# ------------------------------------------------------------ weights --
def reference_weights(dims: ModelDims, seed: int) -> dict[str, np.ndarray]:
    """Every float tensor of the reference's TransformerLM state dict for
    ``dims``, drawn from one numpy PCG64 stream in key order and rounded to
    bfloat16 values (so a bf16 copy is exact).  Linear weights and biases are
    uniform in +-1/sqrt(fan_in) (nn.Linear's default bound), the embedding
    uniform with unit variance, norm weights uniform in [0.5, 1.5] (so a norm
    applied over the wrong span shows), expert_bias uniform in +-0.5 (so the
    bias changes which experts are picked)."""
    rng = np.random.default_rng(seed)
    d, F, V = dims.d_model, dims.d_ff, dims.vocab_size
    kv = dims.num_kv_heads * dims.head_dim
    out: dict[str, np.ndarray] = {}

    def uni(name, shape, lo, hi):
        out[name] = bf16_round(lo + (hi - lo) * rng.random(shape, dtype=np.float32))

    def linear(name, n_out, n_in):
        b = 1.0 / math.sqrt(n_in)
        uni(name + ".weight", (n_out, n_in), -b, b)
        uni(name + ".bias", (n_out,), -b, b)

    def mlp(name):
        linear(name + ".w1", F, d)
        linear(name + ".w3", F, d)
        linear(name + ".w2", d, F)

    s3 = math.sqrt(3.0)
    uni("token_embeddings.weight", (V, d), -s3, s3)
    for i in range(dims.num_layers):
        p = f"layers.{i}."
        linear(p + "att.q_proj", d, d)
        linear(p + "att.k_proj", kv, d)
        linear(p + "att.v_proj", kv, d)
        linear(p + "att.output_proj", d, d)
        uni(p + "att.q_norm.weight", (d,), 0.5, 1.5)
        uni(p + "att.k_norm.weight", (kv,), 0.5, 1.5)
        for e in range(dims.n_routed_experts):
            mlp(p + f"ffn.experts.{e}")
        b = 1.0 / math.sqrt(d)
        uni(p + "ffn.gate.weight", (dims.n_routed_experts, d), -b, b)
        uni(p + "ffn.gate.expert_bias", (dims.n_routed_experts,), -0.5, 0.5)
        if dims.n_shared_experts > 0:
            mlp(p + "ffn.shared_expert")
        uni(p + "att_norm.weight", (d,), 0.5, 1.5)
        uni(p + "ffn_norm.weight", (d,), 0.5, 1.5)
    uni("final_norm.weight", (d,), 0.5, 1.5)
    linear("lm_head", V, d)
    return out


def weights_digest(w: dict[str, np.ndarray]) -> str:
    """sha256 over the keys (sorted) and the float32 bytes of each tensor."""
    h = hashlib.sha256()
    for k in sorted(w):
        h.update(k.encode())
        h.update(np.ascontiguousarray(w[k], dtype=np.float32).tobytes())
    return h.hexdigest()


# -------------------------------------------------------------- layers --
Linear = Callable[[str, torch.Tensor], torch.Tensor]


def fp32_linear(w: dict[str, torch.Tensor]) -> Linear:
    """x @ W^T + b in fp32 for the projection named ``prefix``."""
    def lin(prefix: str, x: torch.Tensor) -> torch.Tensor:
        y = x.float() @ w[prefix + ".weight"].float().t()
        b = w.get(prefix + ".bias")
        return y if b is None else y + b.float()
    return lin


def rms_norm(x, weight, eps, residual=None):
    """(weight * s * rsqrt(mean(s^2) + eps)).to(x.dtype) with s = x (+
    residual) in fp32; returns (out, s.to(x.dtype)) -- utils.py:54-67."""
    s = x.float() if residual is None else x.float() + residual.float()
    out = (weight.float() * s * torch.rsqrt(s.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype)
    return out, s.to(x.dtype)


def head_norm(x, weight):
    """torch.nn.RMSNorm with fp32 weights and eps=None (GQA.py:39-40, 81-82):
    fp32 out, eps the fp32 machine epsilon."""
    xf = x.float()
    return weight.float() * xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + FP32_EPS)


def rope(x, pos, theta):
    """Half-split rotary embedding of x [T, H, D] at positions pos [T], fp32
    (attention/utils.py:24-45)."""
    D = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, device=x.device).float() / D))
    ang = pos.float()[:, None] * inv[None, :]
    cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]
    x1, x2 = x.float().chunk(2, -1)
    return torch.cat((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1)


def gqa_attention(q, k, v, mask=None):
    """SDPA in fp32 with query head h reading kv head h // G (GQA.py:
    118-130).  q [Tq, Hq, D], k/v [Tk, Hkv, D], mask [Tq, Tk] bool (True =
    attend) -> [Tq, Hq*D] fp32."""
    Tq, Hq, D = q.shape
    G = Hq // k.shape[1]
    kh = k.float().repeat_interleave(G, 1).transpose(0, 1)
    vh = v.float().repeat_interleave(G, 1).transpose(0, 1)
    s = torch.matmul(q.float().transpose(0, 1), kh.transpose(1, 2).contiguous()) / math.sqrt(D)
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    return torch.matmul(torch.softmax(s, -1), vh).transpose(0, 1).reshape(Tq, Hq * D)


def qkv_heads(q, k, v, qn_w, kn_w, pos, dims: ModelDims, act_dtype):
    """q_norm / k_norm over the whole projection, split into heads, RoPE;
    q and k cast to the activation dtype (the dtype the K cache holds)."""
    T, Hq, Hkv, D = q.shape[0], dims.num_heads, dims.num_kv_heads, dims.head_dim
    q = rope(head_norm(q, qn_w).view(T, Hq, D), pos, dims.rope_theta).to(act_dtype)
    k = rope(head_norm(k, kn_w).view(T, Hkv, D), pos, dims.rope_theta).to(act_dtype)
    return q, k, v.reshape(T, Hkv, D).to(act_dtype)


def route(h, gate_weight, expert_bias, top_k):
    """(indices [T, k], weights [T, k]) of the gate (moe.py:45-90), every
    step in fp32 -- the build's choice (route_bf16 is the reference's bf16
    arithmetic; the two pick different experts only on bf16 near-ties, as
    tests/test_oracle_model.py checks against the reference's own bf16 picks
    in tests/golden/gate_bf16.npz)."""
    logits = h.float() @ gate_weight.float().t()
    scores = torch.sigmoid(logits)
    idx = torch.topk(logits + expert_bias.float(), top_k, -1).indices
    wts = torch.gather(scores, -1, idx)
    if top_k > 1:
        wts = wts / (wts.sum(-1, keepdim=True) + 1e-10)
    return idx, wts


def route_bf16(h, gate_weight, expert_bias, top_k):
    """The gate as a bf16 TransformerLM runs it (moe.py:45-69): logits = h
    @ W^T rounded to bf16, sigmoid scores in bf16, the fp32 expert bias cast
    to bf16 and added in bf16, top-k of those biased logits
    (torch.topk(sorted=False)), the picked scores renormalised in bf16 by
    their bf16 sum + 1e-10.  h, gate_weight bf16; returns (indices [T, k],
    weights bf16 [T, k], biased logits bf16 [T, E])."""
    logits = h.to(torch.bfloat16) @ gate_weight.to(torch.bfloat16).t()
    scores = torch.sigmoid(logits)
    biased = logits + expert_bias.to(logits.dtype).unsqueeze(0)
    idx = torch.topk(biased, top_k, -1, sorted=False).indices
    wts = torch.gather(scores, -1, idx)
    if top_k > 1:
        wts = wts / (wts.sum(-1, keepdim=True) + 1e-10)
    return idx, wts, biased


def swiglu(a, b):
    """silu(w1 x) * (w3 x) in the dtype of the projections' outputs."""
    return torch.nn.functional.silu(a) * b


def combine(idx, wts, outs, shared, out_dtype):
    """Sum over each token's picks of weight * expert output, plus the shared
    expert's output, in fp32 (moe.py:272-273, 319-339); outs[e] [T, d] is
    expert e's output for every token (only the picked rows are used)."""
    y = torch.zeros_like(outs[0], dtype=torch.float32) if shared is None else shared.float().clone()
    for j in range(idx.shape[1]):
        for e, o in enumerate(outs):
            sel = idx[:, j] == e
            y[sel] += wts[sel, j:j + 1] * o[sel].float()
    return y.to(out_dtype)


def moe(w, p, h, dims: ModelDims, linear: Linear):
    """The MoE of layer prefix p on h [T, d] (moe.py:196-275, eval mode)."""
    def mlp(name):
        return linear(name + ".w2", swiglu(linear(name + ".w1", h), linear(name + ".w3", h)))
    outs = [mlp(p + f"ffn.experts.{e}") for e in range(dims.n_routed_experts)]
    shared = mlp(p + "ffn.shared_expert") if dims.n_shared_experts > 0 else None
    idx, wts = route(h, w[p + "ffn.gate.weight"], w[p + "ffn.gate.expert_bias"], dims.num_experts_per_tok)
    return combine(idx, wts, outs, shared, h.dtype)


def block(w, i, x, residual, pos, dims: ModelDims, linear: Linear, attend):
    """Decoder block i (transformer.py:90-118); ``attend(q, k, v)`` returns
    the attention over the right context, [T, Hq*D] fp32."""
    p = f"layers.{i}."
    if residual is None:
        h, residual = rms_norm(x, w[p + "att_norm.weight"], dims.rms_eps)[0], x
    else:
        h, residual = rms_norm(x, w[p + "att_norm.weight"], dims.rms_eps, residual)
    q, k, v = qkv_heads(linear(p + "att.q_proj", h), linear(p + "att.k_proj", h),
                        linear(p + "att.v_proj", h), w[p + "att.q_norm.weight"],
                        w[p + "att.k_norm.weight"], pos, dims, h.dtype)
    x = linear(p + "att.output_proj", attend(q, k, v).to(h.dtype))
    h, residual = rms_norm(x, w[p + "ffn_norm.weight"], dims.rms_eps, residual)
    return moe(w, p, h, dims, linear), residual


def causal_mask(T: int, device) -> torch.Tensor:
    """[T, T] bool, True where query t may attend key s (s <= t) --
    transformer.py:170-172."""
    return torch.tril(torch.ones(T, T, dtype=torch.bool, device=device))


def forward(w: dict[str, torch.Tensor], tokens, dims: ModelDims, linear: Optional[Linear] = None,
            embed_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Causal forward over one sequence (transformer.py:162-183): fp32
    logits [T, vocab].  ``linear`` defaults to fp32 x @ W^T + b; the
    activations keep the embedding's dtype (``embed_dtype`` casts it)."""
    linear = fp32_linear(w) if linear is None else linear
    emb = w["token_embeddings.weight"]
    dev = emb.device
    tok = torch.as_tensor(tokens, device=dev, dtype=torch.long)
    T = tok.numel()
    pos = torch.arange(T, device=dev)
    x = emb[tok] if embed_dtype is None else emb[tok].to(embed_dtype)
    causal = causal_mask(T, dev)
    residual = None
    for i in range(dims.num_layers):
        x, residual = block(w, i, x, residual, pos, dims, linear,
                            lambda q, k, v: gqa_attention(q, k, v, causal))
    h, _ = rms_norm(x, w["final_norm.weight"], dims.rms_eps, residual)
    return linear("lm_head", h).float()

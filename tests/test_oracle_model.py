"""The decode model's checker (oracle/model.py) against the reference's own
TransformerLM.

tests/golden/model_forward.npz holds logits that the reference's
model/transformer.py TransformerLM (GQA, MoE with a shared expert, eval mode,
fp32) wrote for three 24-token sequences on the weights of
oracle.model.reference_weights(GOLDEN_DIMS, GOLDEN_SEED); the fixture keeps
the weights' sha256, so a change in the weight stream fails before any
logit is compared.  The restatement must reproduce those logits to 2e-5
(measured: 7e-7), and each planted mistake -- swapped into the oracle here
on the CPU -- must miss them by more than 1e-2.
"""
import math
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import model as om

sys.path.insert(0, str(Path(__file__).with_name("golden")))
from make_model_golden import GOLDEN_DIMS, GOLDEN_SEED  # noqa: E402

GOLDEN = Path(__file__).with_name("golden") / "model_forward.npz"
ATOL = 2e-5
PLANT_MIN = 1e-2


@pytest.fixture(scope="module")
def golden():
    g = np.load(GOLDEN)
    w = om.reference_weights(GOLDEN_DIMS, GOLDEN_SEED)
    assert om.weights_digest(w) == str(g["weights_sha256"]), "weight stream differs from the fixture's"
    d = GOLDEN_DIMS
    assert g["dims"].tolist() == [d.vocab_size, d.d_model, d.num_layers, d.num_heads, d.num_kv_heads,
                                  d.d_ff, d.n_routed_experts, d.num_experts_per_tok, d.n_shared_experts]
    return {k: torch.from_numpy(v) for k, v in w.items()}, g["tokens"], g["logits"]


def worst_error(golden) -> float:
    w, tokens, logits = golden
    return max(float(np.abs(om.forward(w, tokens[b], GOLDEN_DIMS).numpy() - logits[b]).max())
               for b in range(tokens.shape[0]))


def test_weights_are_bf16_values():
    w = om.reference_weights(GOLDEN_DIMS, GOLDEN_SEED)
    for k, v in w.items():
        t = torch.from_numpy(v)
        assert torch.equal(t.to(torch.bfloat16).float(), t), k


def test_forward_matches_reference_transformer_lm(golden):
    err = worst_error(golden)
    assert err <= ATOL, f"max |logit diff| {err:.3g} vs the reference's TransformerLM"


def test_last_position_is_a_prefix_forward(golden):
    """Causality: the logits of a prefix equal the first rows of the whole
    sequence's (what a decode step over a KV cache must reproduce)."""
    w, tokens, logits = golden
    y = om.forward(w, tokens[0][:9], GOLDEN_DIMS).numpy()
    np.testing.assert_allclose(y, logits[0][:9], rtol=0, atol=ATOL)


# ----------------------------------------------------- planted mistakes --
def _interleaved_rope(x, pos, theta):
    D = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, D, 2).float() / D))
    ang = pos.float()[:, None] * inv[None, :]
    cos, sin = ang.cos()[:, None, :], ang.sin()[:, None, :]
    x1, x2 = x.float()[..., 0::2], x.float()[..., 1::2]
    return torch.stack((x1 * cos - x2 * sin, x2 * cos + x1 * sin), -1).flatten(-2)


def _gqa_head_map(q, k, v, mask, head_of):
    Tq, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    sel = torch.tensor([head_of(h, Hkv, G) for h in range(Hq)])
    kh, vh = k.float()[:, sel].transpose(0, 1), v.float()[:, sel].transpose(0, 1)
    s = torch.matmul(q.float().transpose(0, 1), kh.transpose(1, 2).contiguous()) / math.sqrt(D)
    if mask is not None:
        s = s.masked_fill(~mask, float("-inf"))
    return torch.matmul(torch.softmax(s, -1), vh).transpose(0, 1).reshape(Tq, Hq * D)


def _per_head_qnorm(q, k, v, qn_w, kn_w, pos, dims, act_dtype):
    T, Hq, D = q.shape[0], dims.num_heads, dims.head_dim
    qh = q.float().view(T, Hq, D)
    qh = qh * torch.rsqrt(qh.pow(2).mean(-1, keepdim=True) + om.FP32_EPS) * qn_w.float().view(Hq, D)
    _, k2, v2 = _orig["qkv_heads"](q, k, v, qn_w, kn_w, pos, dims, act_dtype)
    return om.rope(qh, pos, dims.rope_theta).to(act_dtype), k2, v2


def _route_variant(kind):
    def route(h, gate_weight, expert_bias, top_k):
        logits = h.float() @ gate_weight.float().t()
        scores = torch.softmax(logits, -1) if kind == "softmax" else torch.sigmoid(logits)
        biased = logits + expert_bias.float()
        idx = torch.topk(biased, top_k, -1).indices
        src = torch.sigmoid(biased) if kind == "biased_weights" else scores
        wts = torch.gather(src, -1, idx)
        if kind != "no_renorm":
            wts = wts / (wts.sum(-1, keepdim=True) + 1e-10)
        return idx, wts
    return route


def _no_bias_forward(w, tokens, dims, linear=None, embed_dtype=None):
    stripped = {k: v for k, v in w.items() if not k.endswith(".bias")}
    return _orig["forward"](w, tokens, dims, om.fp32_linear(stripped), embed_dtype)


def _strict_causal_mask(T, device):
    m = torch.tril(torch.ones(T, T, dtype=torch.bool, device=device), -1)
    m[0, 0] = True  # the first query keeps one key so its softmax stays finite
    return m


def _no_residual_block(w, i, x, residual, pos, dims, linear, attend):
    out, _ = _orig["block"](w, i, x, residual, pos, dims, linear, attend)
    return out, None


_orig = {n: getattr(om, n) for n in ("gqa_attention", "qkv_heads", "forward", "block")}

PLANTS = {
    "interleaved RoPE": ("rope", _interleaved_rope),
    "head map h % Hkv": ("gqa_attention", lambda q, k, v, mask=None: _gqa_head_map(q, k, v, mask,
                                                                              lambda h, Hkv, G: h % Hkv)),
    "q_norm per head": ("qkv_heads", _per_head_qnorm),
    "softmax gate": ("route", _route_variant("softmax")),
    "biased scores as weights": ("route", _route_variant("biased_weights")),
    "top-k weights not renormalised": ("route", _route_variant("no_renorm")),
    "linear biases dropped": ("forward", _no_bias_forward),
    "newest token not attended": ("causal_mask", _strict_causal_mask),
    "residual stream dropped": ("block", _no_residual_block),
}


@pytest.mark.parametrize("name", list(PLANTS))
def test_planted_mistake_misses_reference(golden, monkeypatch, name):
    attr, fn = PLANTS[name]
    monkeypatch.setattr(om, attr, fn)
    err = worst_error(golden)
    assert err > PLANT_MIN, f"planted mistake '{name}' is not caught: max |logit diff| {err:.3g}"


def test_decode_model_loader_names_the_reference_state_dict():
    """DecodeModel.load_reference_state_dict expects exactly the float
    tensors (names and shapes) of the reference's TransformerLM state dict:
    the fixture script checked that key set against the reference's own
    state_dict() when it wrote the golden logits."""
    from llm_from_scratch_amd.decode_model import DecodeModelConfig
    d = GOLDEN_DIMS
    cfg = DecodeModelConfig(vocab_size=d.vocab_size, d_model=d.d_model, num_layers=d.num_layers,
                            num_heads=d.num_heads, num_kv_heads=d.num_kv_heads, d_ff=d.d_ff,
                            n_routed_experts=d.n_routed_experts, num_experts_per_tok=d.num_experts_per_tok,
                            n_shared_experts=d.n_shared_experts)
    w = om.reference_weights(d, GOLDEN_SEED)
    assert cfg.reference_state_keys() == {k: v.shape for k, v in w.items()}

"""Write tests/golden/model_forward.npz: logits of the reference's own
TransformerLM (GQA attention, MoE with a shared expert) on fixed weights and
tokens.

Run once in a container that has the reference checkout (it is not needed at
test time, and nothing else imports the reference):

    python tests/golden/make_model_golden.py /root/reference

The weights are ``oracle.model.reference_weights(GOLDEN_DIMS, GOLDEN_SEED)``
(a numpy PCG64 stream, every value a bfloat16 value); the fixture stores
their sha256 instead of the weights, and the tests regenerate them.  The
model is built from the reference's model/config.py Config and
model/transformer.py TransformerLM, every float tensor of its state dict is
overwritten with these weights (the key sets must match exactly), and its
forward runs in eval mode (MoE.moe_infer, no dropout) in fp32 on the CPU.
"""
import sys
from pathlib import Path

import numpy as np
import torch

REPO = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(REPO))
from oracle.model import ModelDims, reference_weights, weights_digest  # noqa: E402

# d_model, d_ff multiples of 128 and head_dim 64, so the FP8 decode model
# can load the same weights; vocab 160 leaves a ragged 128-row block
GOLDEN_DIMS = ModelDims(vocab_size=160, d_model=256, num_layers=2, num_heads=4, num_kv_heads=2,
                        d_ff=128, n_routed_experts=4, num_experts_per_tok=2, n_shared_experts=1)
GOLDEN_SEED = 2024
BATCH, SEQ = 3, 24


def golden_tokens() -> np.ndarray:
    return np.random.default_rng(GOLDEN_SEED + 1).integers(0, GOLDEN_DIMS.vocab_size, (BATCH, SEQ))


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from model.config import Config
    from model.transformer import TransformerLM

    d = GOLDEN_DIMS
    cfg = Config(vocab_size=d.vocab_size, context_length=64, d_model=d.d_model, num_layers=d.num_layers,
                 num_heads=d.num_heads, d_ff=d.d_ff, dropout=0.0, attention_type="GQA",
                 num_kv_heads=d.num_kv_heads, rope_theta=d.rope_theta, use_moe=True,
                 n_routed_experts=d.n_routed_experts, num_experts_per_tok=d.num_experts_per_tok,
                 n_shared_experts=d.n_shared_experts, aux_seq_loss_alpha=0.0)
    model = TransformerLM(cfg).eval()
    w = reference_weights(d, GOLDEN_SEED)
    sd = model.state_dict()
    floats = {k for k, v in sd.items() if v.is_floating_point()}
    if floats != set(w):
        raise SystemExit(f"state-dict keys differ: missing {sorted(floats - set(w))}, "
                         f"extra {sorted(set(w) - floats)}")
    for k in floats:
        assert tuple(sd[k].shape) == w[k].shape, (k, tuple(sd[k].shape), w[k].shape)
        sd[k] = torch.from_numpy(w[k].copy())
    model.load_state_dict(sd)
    tokens = golden_tokens()
    with torch.no_grad():
        logits = model(torch.from_numpy(tokens)).float().numpy()
    out = Path(__file__).with_name("model_forward.npz")
    np.savez_compressed(out, tokens=tokens.astype(np.int64), logits=logits.astype(np.float32),
                        weights_sha256=np.array(weights_digest(w)), seed=np.int64(GOLDEN_SEED),
                        dims=np.array([d.vocab_size, d.d_model, d.num_layers, d.num_heads, d.num_kv_heads,
                                       d.d_ff, d.n_routed_experts, d.num_experts_per_tok,
                                       d.n_shared_experts], dtype=np.int64))
    print(f"wrote {out}: tokens {tokens.shape}, logits {logits.shape}, "
          f"|logits| max {np.abs(logits).max():.3f}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")

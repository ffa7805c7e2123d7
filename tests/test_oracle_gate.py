"""The MoE gate in bfloat16 against the reference's own Gate.

tests/golden/gate_bf16.npz holds what the reference's Gate
(model/architecture/moe.py:45-90) computed in bf16 on the cfg5 gate shape
(4096 tokens, d 768, 8 experts, top-2; inputs regenerated from seeds by
tests/golden/make_gate_golden.py): its biased logits, picks and weights.
  * oracle.model.route_bf16 reproduces all three bit for bit: the
    reference's bf16 arithmetic is completely restated;
  * the build gates in fp32 (oracle.model.route, and the GPU kernel
    moe_route in tests/test_gpu_fused.py): its picks equal the reference's
    on every token except bf16 near-ties -- tokens where the reference's
    k-th and (k+1)-th biased logits lie within two bf16 ulps of each other,
    so bf16 rounding alone decides the order -- and on tokens with the same
    picks its weights equal the reference's bf16 weights to bf16 rounding
    (2^-6 relative: four roundings).
"""
import sys
from pathlib import Path

import numpy as np
import torch

from oracle import model as om

sys.path.insert(0, str(Path(__file__).with_name("golden")))
from make_gate_golden import TOP_K, gate_inputs  # noqa: E402

GOLDEN = Path(__file__).with_name("golden") / "gate_bf16.npz"


def _fixture():
    f = np.load(GOLDEN)
    biased = torch.from_numpy(f["biased_logits_bf16"]).view(torch.bfloat16)
    return biased, f["topk_idx"].astype(np.int64), torch.from_numpy(f["topk_weight_bf16"]).view(torch.bfloat16)


def _sorted_picks(idx, wts):
    order = np.argsort(idx, axis=-1, kind="stable")
    return np.take_along_axis(idx, order, -1), np.take_along_axis(wts, order, -1)


def bf16_ulp(x):
    """Spacing of bf16 values at |x| (8 significand bits)."""
    e = np.floor(np.log2(np.maximum(np.abs(x), 1e-30)))
    return np.exp2(e - 7)


def near_tie_tokens(biased_ref, k):
    """Tokens whose reference k-th and (k+1)-th biased logits are within two
    bf16 ulps of each other."""
    srt = np.sort(biased_ref.float().numpy(), axis=-1)[:, ::-1]
    gap = srt[:, k - 1] - srt[:, k]
    return gap <= 2 * bf16_ulp(srt[:, k - 1])


def test_bf16_restatement_equals_reference_gate():
    x, w, bias = gate_inputs()
    ref_biased, ref_idx, ref_wts = _fixture()
    idx, wts, biased = om.route_bf16(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(bias), TOP_K)
    assert torch.equal(biased.view(torch.int16), ref_biased.view(torch.int16))
    pi, pw = _sorted_picks(idx.numpy(), wts.float().numpy())
    np.testing.assert_array_equal(pi, ref_idx)
    np.testing.assert_array_equal(pw, ref_wts.float().numpy())


def test_fp32_gate_differs_from_reference_only_on_bf16_near_ties():
    x, w, bias = gate_inputs()
    ref_biased, ref_idx, ref_wts = _fixture()
    idx, wts = om.route(torch.from_numpy(x), torch.from_numpy(w), torch.from_numpy(bias), TOP_K)
    pi, pw = _sorted_picks(idx.numpy(), wts.numpy())
    differ = (pi != ref_idx).any(-1)
    ties = near_tie_tokens(ref_biased, TOP_K)
    assert not (differ & ~ties).any(), f"{int((differ & ~ties).sum())} tokens differ without a bf16 near-tie"
    assert differ.sum() <= 0.02 * len(differ), f"{int(differ.sum())} of {len(differ)} tokens pick differently"
    same = ~differ
    ref_w = ref_wts.float().numpy()[same]
    # the reference's weights pass through four bf16 roundings (logit, sigmoid,
    # sum, divide): within 4 half-ulps, 2^-6 relative
    np.testing.assert_allclose(pw[same], ref_w, rtol=2 ** -6, atol=0)
    print(f"\nfp32 gate vs the reference's bf16 gate: {int(differ.sum())} of {len(differ)} tokens pick "
          f"differently, all bf16 near-ties ({int(ties.sum())} near-tie tokens in all)")


def test_near_tie_criterion_catches_a_planted_swap():
    """Swapping the picks of a token whose top-k boundary is not a near-tie
    must be flagged (the criterion is not vacuous)."""
    ref_biased, ref_idx, _ = _fixture()
    ties = near_tie_tokens(ref_biased, TOP_K)
    t = int(np.flatnonzero(~ties)[0])
    srt = np.argsort(-ref_biased.float().numpy()[t])
    planted = ref_idx.copy()
    planted[t] = np.sort(np.concatenate([srt[:TOP_K - 1], srt[TOP_K:TOP_K + 1]]))
    differ = (planted != ref_idx).any(-1)
    assert (differ & ~ties).any()

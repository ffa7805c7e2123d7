"""Fused temperature + Gumbel-max sampler (HIP) against the CPU oracle.

  * noise: every element's Exp(1) variate equals the oracle's Philox4x32-10
    word mapped by -log((w + 1) 2^-32) (the generator is pinned to the
    Random123 known-answer vectors on the CPU), to float rounding;
  * pick: the token the kernel returns maximises the reference formula
    softmax(logits / T) / clamp(noise, 1e-10) computed in float64 on the
    same noise (a pick within 1e-5 relative of the maximum is accepted:
    exp/division rounding can reorder near-ties);
  * distribution: with fresh noise per call, token frequencies match the
    softmax probabilities;
  * Sampler (engine) advances the offset: repeated calls differ, a fixed
    (seed, offset) repeats.
"""
import numpy as np
import pytest
import torch

from llm_from_scratch_amd import kernels as K
from llm_from_scratch_amd.engine import Sampler
from oracle import sampler as S

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("B,V", [(4, 32000), (3, 1001), (128, 4096)])
def test_sample_gumbel_noise_and_pick(B, V):
    g = torch.Generator(device=DEV).manual_seed(B + V)
    logits = (torch.randn(B, V, generator=g, device=DEV) * 4).to(torch.bfloat16)
    temps = torch.rand(B, generator=g, device=DEV) + 0.3
    seed, offset = 0x1234_5678_9ABC_DEF1, 7 << 32 | 5
    tok, noise = K.sample_gumbel(logits, temps, seed, offset, return_noise=True)
    want_noise = S.exp_noise(S.noise_words(B, V, seed, offset))
    np.testing.assert_allclose(noise.cpu().numpy(), want_noise, rtol=1e-6, atol=1e-7)
    _, score = S.sample_gumbel(logits.float().cpu().numpy(), temps.cpu().numpy(), noise.double().cpu().numpy())
    t = tok.cpu().numpy()
    got = score[np.arange(B), t]
    assert np.all(got >= score.max(axis=1) * (1 - 1e-5)), (t, score.argmax(axis=1))
    # the same (seed, offset) repeats; the next offset draws new noise
    assert torch.equal(K.sample_gumbel(logits, temps, seed, offset), tok)
    _, n2 = K.sample_gumbel(logits, temps, seed, offset + (V + 3) // 4, return_noise=True)
    assert not torch.equal(n2, noise)


def test_sample_gumbel_distribution():
    logits = torch.tensor([[0.0, 1.0, 2.0, -1.0, 0.5]], device=DEV).to(torch.bfloat16)
    p = torch.softmax(logits.float() / 0.7, -1)[0].cpu().numpy()
    n = 40000
    toks = K.sample_gumbel(logits.expand(n, 5), torch.full((n,), 0.7, device=DEV), seed=99, offset=0)
    freq = np.bincount(toks.cpu().numpy(), minlength=5) / n
    assert np.abs(freq - p).max() < 0.01, (freq, p)


def test_engine_sampler_advances():
    s = Sampler()
    g = torch.Generator(device=DEV).manual_seed(5)
    logits = torch.zeros(64, 1000, device=DEV, dtype=torch.bfloat16)
    temps = torch.ones(64, device=DEV)
    a = s(logits, temps, g)
    b = s(logits, temps, g)
    assert a.dtype == torch.int64 and a.shape == (64,)
    assert not torch.equal(a, b)  # uniform logits: fresh noise picks other tokens

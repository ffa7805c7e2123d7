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


@pytest.mark.parametrize("B,V", [(128, 32000), (4, 32000), (16, 50000), (1, 7), (2048, 4096), (5, 4100)])
def test_sample_gumbel_slices_pick_what_one_pass_picks(B, V):
    """lfs_sample_gumbel_split (rows cut into slices, a per-row reduce)
    returns exactly the tokens of the one-pass lfs_sample_gumbel, with the
    same noise, on random logits and on rows whose equal maxima start in a
    later slice (ties go to the lowest index in both)."""
    from llm_from_scratch_amd import _lib
    L = _lib.load()
    g = torch.Generator(device=DEV).manual_seed(7 * B + V)
    for case in ("random", "ties"):
        if case == "random":
            logits = (torch.randn(B, V, generator=g, device=DEV) * 4).to(torch.bfloat16)
        else:  # equal maxima from mid-row on; T = 1e-30 makes x / T swamp the noise: exact score ties
            logits = torch.zeros(B, V, device=DEV).to(torch.bfloat16)
            logits[:, V // 2::97] = 30.0
        temps = torch.full((B,), 0.7 if case == "random" else 1e-30, device=DEV)
        one = torch.empty(B, dtype=torch.int64, device=DEV)
        rc = L.lfs_sample_gumbel(logits.data_ptr(), V, temps.data_ptr(), B, V, 1234, 99, one.data_ptr(), None,
                                 torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        need = int(L.lfs_sample_gumbel_workspace_bytes(B, V))
        ws = torch.empty(max(need, 8), dtype=torch.uint8, device=DEV)
        sl = torch.empty(B, dtype=torch.int64, device=DEV)
        rc = L.lfs_sample_gumbel_split(logits.data_ptr(), V, temps.data_ptr(), B, V, 1234, 99, sl.data_ptr(), None,
                                       ws.data_ptr(), ws.numel(), torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.equal(one, sl), f"{case}: {int((one != sl).sum())} rows differ"
        if case == "ties":
            assert bool((sl == V // 2).all()), "ties must go to the lowest index"
        assert torch.equal(K.sample_gumbel(logits, temps, 1234, 99), one)
    if need:  # too small a workspace is refused, nothing launched
        rc = L.lfs_sample_gumbel_split(logits.data_ptr(), V, temps.data_ptr(), B, V, 1, 0, sl.data_ptr(), None,
                                       ws.data_ptr(), need - 8, torch.cuda.current_stream().cuda_stream)
        assert rc != 0

"""FP8 indexer score (HIP) against the CPU oracle (model/attention/utils.py:
175-250 semantics).

Bar: bit-exact on small-integer codes with scales of the form 2^k (every
dot product, ReLU, weighted sum and key scale is exact in fp32); within
1e-5 relative of the float64 oracle (scaled by the row's largest |score|)
on random codes and scales; within 1e-4 on the act_quant ue8m0 pipeline,
whose codes span the whole e4m3 range (products up to 2e5 summed inside
the MFMA, which does not round like a sequential fp32 sum).  Cases: head dims 32 / 64 / 128, head
counts that are and are not multiples of 16, key counts across the 16-key
and 256-key chunk edges, a key slice of a longer FP8 cache, and the
reference's indexer pipeline (act_quant block 32 with ue8m0 scales).
"""
import numpy as np
import pytest
import torch

from llm_from_scratch_amd import kernels as K
from oracle import fp8 as F

pytestmark = pytest.mark.gpu
DEV = "cuda"


def codes(x):
    return torch.from_numpy(F.e4m3_encode(x)).view(torch.float8_e4m3fn).to(DEV)


@pytest.mark.parametrize("B,M,N,H,D", [(2, 5, 300, 64, 128), (1, 3, 17, 20, 64), (3, 2, 257, 16, 32)])
def test_fp8_index_exact_integers(B, M, N, H, D):
    rng = np.random.default_rng(B * M + N + H + D)
    ints = np.arange(-4, 5, dtype=np.float32)
    q = codes(rng.choice(ints, (B, M, H, D)))
    k = codes(rng.choice(ints, (B, N, D)))
    qs = torch.from_numpy(2.0 ** rng.integers(-3, 3, (B, M, H)).astype(np.float32)).to(DEV)
    ks = torch.from_numpy(2.0 ** rng.integers(-3, 3, (B, N)).astype(np.float32)).to(DEV)
    o = K.fp8_index(q, qs, k, ks)
    ref = F.fp8_index(q.view(torch.uint8).cpu().numpy(), qs.cpu().numpy(), k.view(torch.uint8).cpu().numpy(),
                      ks.cpu().numpy())
    np.testing.assert_array_equal(o.cpu().numpy(), ref.astype(np.float32))


def test_fp8_index_random_and_cache_slice():
    rng = np.random.default_rng(4)
    B, M, H, D, NMAX, N = 2, 4, 64, 128, 1000, 700
    q = codes(rng.standard_normal((B, M, H, D)) * 8)
    kcache = codes(rng.standard_normal((B, NMAX, D)) * 8)
    scache = torch.from_numpy(rng.uniform(1e-3, 1e-1, (B, NMAX)).astype(np.float32)).to(DEV)
    qs = torch.from_numpy(rng.uniform(1e-3, 1e-1, (B, M, H)).astype(np.float32)).to(DEV)
    k, ks = kcache[:, :N], scache[:, :N]  # the first N cached keys, no copy
    o = K.fp8_index(q, qs, k, ks).cpu().numpy()
    ref = F.fp8_index(q.view(torch.uint8).cpu().numpy(), qs.cpu().numpy(),
                      k.contiguous().view(torch.uint8).cpu().numpy(), ks.cpu().numpy())
    err = np.abs(o - ref) / np.abs(ref).max(axis=-1, keepdims=True)
    assert err.max() < 1e-5, err.max()


def test_fp8_index_reference_pipeline():
    """The reference indexer's inputs (DSA.py:92-105): q and k quantised by
    act_quant with block 32 and ue8m0 scales at head_dim 32 (one scale per
    head row and per key), head weights times the q scale."""
    g = torch.Generator(device=DEV).manual_seed(8)
    B, M, N, H, D = 2, 6, 130, 32, 32
    qx = torch.randn(B, M, H, D, generator=g, device=DEV).to(torch.bfloat16)
    kx = torch.randn(B, N, D, generator=g, device=DEV).to(torch.bfloat16)
    q8, q_scale = K.act_quant(qx, 32, "ue8m0")   # [B, M, H, 1]
    k8, k_scale = K.act_quant(kx, 32, "ue8m0")   # [B, N, 1]
    w = torch.rand(B, M, H, 1, generator=g, device=DEV) * H ** -0.5
    weights = w * q_scale * D ** -0.5
    o = K.fp8_index(q8, weights, k8, k_scale.squeeze(-1)).cpu().numpy()
    ref = F.fp8_index(q8.view(torch.uint8).cpu().numpy(), weights.squeeze(-1).cpu().numpy(),
                      k8.view(torch.uint8).cpu().numpy(), k_scale.squeeze(-1).cpu().numpy())
    err = np.abs(o - ref) / np.maximum(np.abs(ref).max(axis=-1, keepdims=True), 1e-30)
    assert err.max() < 1e-4, err.max()
    # approximates the bf16 score
    qf, kf = qx.float().cpu().numpy(), kx.float().cpu().numpy()
    full = np.maximum(np.einsum("bmhd,bnd->bmhn", qf, kf), 0) * (w * D ** -0.5).cpu().numpy()
    approx = full.sum(2)
    assert np.abs(o - approx).max() < 0.1 * np.abs(approx).max()

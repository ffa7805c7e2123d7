"""Varlen causal prefill attention (HIP) against the CPU oracle.

Bar: within 1e-2 relative / 2e-2 absolute of the float64 oracle on the same
bf16 inputs (P is rounded to bf16 for the P.V MFMA, accumulation is fp32).
Cases: D 64 and 128, GQA group sizes 1-8, sequence lengths across the
16-query and 32-key tile boundaries (1, 15, 16, 17, 31, 33, ...), contiguous
keys, paged keys with cached prefixes (lq < lk) at block sizes 16 and 256,
block tables with -1 padding past each sequence, and a pool whose slots past
every context hold NaN.
"""
import numpy as np
import pytest
import torch

from llm_from_scratch_amd import kernels as K
from oracle import paged_kv as P

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-2, 2e-2


def f64(t):
    return t.double().cpu().numpy()


def assert_close(got, ref, what):
    err = np.abs(got - ref)
    bad = np.argwhere(err > ATOL + RTOL * np.abs(ref))
    assert bad.size == 0, f"{what}: {len(bad)} mismatches, worst {err.max():.4g}, first {bad[:3].tolist()}"


def bf16(rng, *shape, scale=1.0):
    return torch.from_numpy((rng.standard_normal(shape) * scale).astype(np.float32)).to(torch.bfloat16).to(DEV)


@pytest.mark.parametrize("Hq,Hkv,D", [(12, 4, 64), (32, 8, 128), (8, 8, 64), (16, 2, 128), (8, 1, 64)])
def test_prefill_contiguous(Hq, Hkv, D):
    rng = np.random.default_rng(Hq * 100 + Hkv + D)
    lens = [1, 15, 16, 17, 31, 33, 100, 257]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    T = int(sum(lens))
    q = bf16(rng, T, Hq, D)
    k = bf16(rng, T, Hkv, D)
    v = bf16(rng, T, Hkv, D)
    scale = 1.0 / np.sqrt(D)
    o = K.flash_attn_varlen_func(q, k, v, cu, cu, max(lens), max(lens), scale)
    ref = P.prefill_attention(f64(q), f64(k), f64(v), cu.cpu().numpy(), cu.cpu().numpy(), scale)
    assert_close(f64(o), ref, f"contiguous Hq={Hq} Hkv={Hkv} D={D}")


@pytest.mark.parametrize("BS", [16, 256])
@pytest.mark.parametrize("Hq,Hkv,D", [(12, 4, 64), (32, 8, 128)])
def test_prefill_paged_cached_prefix(BS, Hq, Hkv, D):
    """Keys from a randomly permuted pool through -1-padded block tables;
    sequences with a cached prefix (lq < lk), a whole prompt (lq == lk) and
    a single new token."""
    rng = np.random.default_rng(BS + Hq + D)
    lens_k = [300, 64, 17, 520, 1]
    lens_q = [44, 64, 1, 7, 1]
    B = len(lens_k)
    nblk = [-(-L // BS) for L in lens_k]
    NB = sum(nblk) + 7
    maxb = max(nblk) + 2
    perm = rng.permutation(NB)
    bt = np.full((B, maxb), -1, np.int32)
    pos = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[pos:pos + n]
        pos += n
    kc = bf16(rng, NB, BS, Hkv, D)
    vc = bf16(rng, NB, BS, Hkv, D)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lens_q)]), dtype=torch.int32, device=DEV)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens_k)]), dtype=torch.int32, device=DEV)
    q = bf16(rng, int(sum(lens_q)), Hq, D)
    btd = torch.from_numpy(bt).to(DEV)
    o = K.flash_attn_varlen_func(q, kc, vc, cu_q, cu_k, max(lens_q), max(lens_k), 0.125, block_table=btd)
    ref = P.prefill_attention(f64(q), f64(kc), f64(vc), cu_q.cpu().numpy(), cu_k.cpu().numpy(), 0.125,
                              block_tables=bt)
    assert_close(f64(o), ref, f"paged BS={BS} Hq={Hq} Hkv={Hkv} D={D}")


@pytest.mark.parametrize("BS", [16, 64])
def test_prefill_paged_pool_poisoned_past_context(BS):
    """Pool slots that hold no key of any sequence (tails of the last
    blocks, unused blocks) are NaN: keys past a context are masked, and
    their V rows must not reach the output either (0 * NaN)."""
    rng = np.random.default_rng(BS + 7)
    Hq, Hkv, D = 12, 4, 64
    lens_k = [37, 20, 5, 70]
    lens_q = [37, 3, 5, 10]
    B = len(lens_k)
    nblk = [-(-L // BS) for L in lens_k]
    NB = sum(nblk) + 3
    perm = rng.permutation(NB)
    bt = np.full((B, max(nblk) + 1), -1, np.int32)
    kc = torch.full((NB, BS, Hkv, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    vc = torch.full((NB, BS, Hkv, D), float("nan"), dtype=torch.bfloat16, device=DEV)
    pos = 0
    for i, n in enumerate(nblk):
        bt[i, :n] = perm[pos:pos + n]
        pos += n
        for t in range(lens_k[i]):  # only the context's own slots hold data
            blk, o = bt[i, t // BS], t % BS
            kc[blk, o] = bf16(rng, Hkv, D)
            vc[blk, o] = bf16(rng, Hkv, D)
    cu_q = torch.tensor(np.concatenate([[0], np.cumsum(lens_q)]), dtype=torch.int32, device=DEV)
    cu_k = torch.tensor(np.concatenate([[0], np.cumsum(lens_k)]), dtype=torch.int32, device=DEV)
    q = bf16(rng, int(sum(lens_q)), Hq, D)
    o = K.flash_attn_varlen_func(q, kc, vc, cu_q, cu_k, max(lens_q), max(lens_k), 0.125,
                                 block_table=torch.from_numpy(bt).to(DEV))
    assert torch.isfinite(o.float()).all(), "NaN from slots past a context"
    ref = P.prefill_attention(f64(q), np.nan_to_num(f64(kc)), np.nan_to_num(f64(vc)), cu_q.cpu().numpy(),
                              cu_k.cpu().numpy(), 0.125, block_tables=bt)
    assert_close(f64(o), ref, f"poisoned pool BS={BS}")


def test_prefill_long_prompt_and_graph_grid():
    """One 1000-token prompt next to short ones, with max_seqlen_q larger
    than every length (the grid only depends on it): rows of idle tiles are
    not written, every real row matches."""
    rng = np.random.default_rng(11)
    Hq, Hkv, D = 12, 4, 64
    lens = [1000, 3, 40]
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=DEV)
    T = int(sum(lens))
    q, k, v = bf16(rng, T, Hq, D), bf16(rng, T, Hkv, D), bf16(rng, T, Hkv, D)
    o = K.flash_attn_varlen_func(q, k, v, cu, cu, 1100, 1100)
    ref = P.prefill_attention(f64(q), f64(k), f64(v), cu.cpu().numpy(), cu.cpu().numpy(), 1.0 / 8)
    assert_close(f64(o), ref, "long prompt")


@pytest.mark.parametrize("B,L,Hq,Hkv,D", [(8, 1024, 16, 8, 64), (16, 2048, 12, 4, 64)])
def test_prefill_large_grid_subtiles_vs_torch_fp32(B, L, Hq, Hkv, D):
    """Grids large enough for two (8 x 1024 tokens, G = 2) or four (16 x 2048
    tokens, G = 3: the bench shape) 16-query sub-tiles per workgroup (G * 2
    or G * 4 waves sharing each K / V tile): against causal attention
    computed per sequence in float32 with torch on the GPU (the float64
    oracle is too slow at this size)."""
    g = torch.Generator(device=DEV).manual_seed(13)
    q = torch.randn(B * L, Hq, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B * L, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B * L, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(0, (B + 1) * L, L, dtype=torch.int32, device=DEV)
    o = K.flash_attn_varlen_func(q, k, v, cu, cu, L, L)
    G = Hq // Hkv
    mask = torch.ones(L, L, device=DEV, dtype=torch.bool).tril()
    worst = 0.0
    for b in range(B):
        sl = slice(b * L, (b + 1) * L)
        qf = q[sl].float().permute(1, 0, 2).contiguous()                      # [Hq, L, D]
        kf = k[sl].float().repeat_interleave(G, 1).permute(1, 2, 0).contiguous()  # [Hq, D, L]
        vf = v[sl].float().repeat_interleave(G, 1).permute(1, 0, 2).contiguous()  # [Hq, L, D]
        s = torch.matmul(qf, kf) / D ** 0.5
        s = s.masked_fill(~mask, float("-inf"))
        ref = torch.matmul(torch.softmax(s, -1), vf).permute(1, 0, 2)
        err = (o[sl].float() - ref).abs()
        assert bool((err <= ATOL + RTOL * ref.abs()).all()), f"sequence {b}: worst {err.max().item():.4g}"
        worst = max(worst, err.max().item())


def _torch_causal_ref(qs, ks, vs, G, D, scale):
    """Causal attention of one sequence in float32 with torch on the GPU:
    qs [lq, Hq, D] are the last lq positions of ks / vs [lk, Hkv, D]."""
    lq, lk = qs.size(0), ks.size(0)
    qf = qs.float().permute(1, 0, 2).contiguous()                       # [Hq, lq, D]
    kf = ks.float().repeat_interleave(G, 1).permute(1, 2, 0).contiguous()  # [Hq, D, lk]
    vf = vs.float().repeat_interleave(G, 1).permute(1, 0, 2).contiguous()  # [Hq, lk, D]
    s = torch.matmul(qf, kf) * scale
    pos = torch.arange(lk - lq, lk, device=DEV)[:, None]
    s = s.masked_fill(torch.arange(lk, device=DEV)[None, :] > pos, float("-inf"))
    return torch.matmul(torch.softmax(s, -1), vf).permute(1, 0, 2)


def test_prefill_large_grid_four_subtiles_d128():
    """Four 16-query sub-tiles per workgroup at D = 128 and G = 4 (the cfg4
    heads, 32 / 8): 4 x 4096-token prompts fill every CU eight times with
    64-query workgroups.  Against causal attention per sequence in float32."""
    B, L, Hq, Hkv, D = 4, 4096, 32, 8, 128
    g = torch.Generator(device=DEV).manual_seed(14)
    q = torch.randn(B * L, Hq, D, generator=g, device=DEV).to(torch.bfloat16)
    k = torch.randn(B * L, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    v = torch.randn(B * L, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    cu = torch.arange(0, (B + 1) * L, L, dtype=torch.int32, device=DEV)
    o = K.flash_attn_varlen_func(q, k, v, cu, cu, L, L)
    for b in range(B):
        sl = slice(b * L, (b + 1) * L)
        ref = _torch_causal_ref(q[sl], k[sl], v[sl], Hq // Hkv, D, D ** -0.5)
        err = (o[sl].float() - ref).abs()
        assert bool((err <= ATOL + RTOL * ref.abs()).all()), f"sequence {b}: worst {err.max().item():.4g}"


@pytest.mark.parametrize("B,lq,cached,Hq,Hkv,D", [(16, 2048, 1536, 12, 4, 64), (8, 2048, 512, 32, 8, 128)])
def test_prefill_large_grid_paged_cached_prefix_subtiles(B, lq, cached, Hq, Hkv, D):
    """The paged kernel (a prefix-cache hit: `cached` keys already in the
    pool) on a grid large enough for four 16-query sub-tiles per workgroup:
    block size 256, a randomly permuted pool, -1-padded tables.  Against
    causal attention per sequence in float32 over the gathered keys."""
    BS = 256
    lk = cached + lq
    rng = np.random.default_rng(B + lq + D)
    nblk = -(-lk // BS)
    NB = B * nblk + 3
    perm = rng.permutation(NB)
    bt = np.full((B, nblk + 1), -1, np.int32)
    for b in range(B):
        bt[b, :nblk] = perm[b * nblk:(b + 1) * nblk]
    g = torch.Generator(device=DEV).manual_seed(15)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(B * lq, Hq, D, generator=g, device=DEV).to(torch.bfloat16)
    cu_q = torch.arange(0, (B + 1) * lq, lq, dtype=torch.int32, device=DEV)
    cu_k = torch.arange(0, (B + 1) * lk, lk, dtype=torch.int32, device=DEV)
    btd = torch.from_numpy(bt).to(DEV)
    scale = D ** -0.5
    o = K.flash_attn_varlen_func(q, kc, vc, cu_q, cu_k, lq, lk, scale, block_table=btd)
    for b in range(B):
        ids = torch.from_numpy(bt[b, :nblk].astype(np.int64)).to(DEV)
        ks = kc[ids].reshape(-1, Hkv, D)[:lk]
        vs = vc[ids].reshape(-1, Hkv, D)[:lk]
        sl = slice(b * lq, (b + 1) * lq)
        ref = _torch_causal_ref(q[sl], ks, vs, Hq // Hkv, D, scale)
        err = (o[sl].float() - ref).abs()
        assert bool((err <= ATOL + RTOL * ref.abs()).all()), f"sequence {b}: worst {err.max().item():.4g}"


def test_prefill_argument_errors():
    q = torch.zeros(4, 8, 64, dtype=torch.bfloat16, device=DEV)
    kv = torch.zeros(4, 2, 64, dtype=torch.bfloat16, device=DEV)
    cu = torch.tensor([0, 4], dtype=torch.int32, device=DEV)
    with pytest.raises(TypeError):
        K.flash_attn_varlen_func(q, kv, kv, cu.long(), cu, 4, 4)
    with pytest.raises(AssertionError):
        K.flash_attn_varlen_func(q, kv, kv, cu, cu, 4, 4, causal=False)
    bad = torch.zeros(4, 3, 64, dtype=torch.bfloat16, device=DEV)  # 8 q heads over 3 kv heads
    with pytest.raises(ValueError):
        K.flash_attn_varlen_func(q, bad, bad, cu, cu, 4, 4)

"""GPU parity of the paged-KV kernels against the CPU oracle (C ABI).

Bar: store_kvcache bit-exact (and nothing else in the pool changes);
paged decode within rtol 1e-2 / atol 2e-2 of the float64 oracle on the same
bf16 inputs; properties that hold at any size: split-count independence,
zero padding rows, L=1 -> v0.
"""
import math

import numpy as np
import pytest
import torch

from llm_from_scratch_amd import kernels as K
from llm_from_scratch_amd import workloads as W
from oracle import paged_kv as P

pytestmark = pytest.mark.gpu
DEV = "cuda"
RTOL, ATOL = 1e-2, 2e-2


def bits(t):
    return t.view(torch.int16).cpu().numpy()


def assert_close(got, ref, what=""):
    err = np.abs(got - ref)
    bad = np.argwhere(err > ATOL + RTOL * np.abs(ref))
    assert bad.size == 0, f"{what}: {len(bad)} mismatches, worst {err.max():.4g}, first {bad[:3].tolist()}"


# ----------------------------------------------------------- store_kvcache --
@pytest.mark.parametrize("Hkv,D", [(4, 64), (8, 128), (3, 36)])
def test_store_kvcache_bitexact(Hkv, D):
    NB, BS, T = 64, 16, 200
    g = torch.Generator(device=DEV).manual_seed(Hkv * D)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    k0, v0 = bits(kc), bits(vc)
    key = torch.randn(T, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    val = torch.randn(T, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    rng = np.random.default_rng(D)
    slots = rng.choice(NB * BS, T, replace=False).astype(np.int64)
    slots[::7] = -1
    K.store_kvcache(key, val, kc, vc, torch.from_numpy(slots).to(DEV))
    torch.cuda.synchronize()
    P.store_kvcache(bits(key), bits(val), k0, v0, slots)
    np.testing.assert_array_equal(bits(kc), k0)
    np.testing.assert_array_equal(bits(vc), v0)


def test_store_kvcache_strided_views_of_fused_qkv():
    """key/value as column slices of a fused qkv projection output (token
    stride = qkv width), as an attention layer produces them."""
    T, Hq, Hkv, D, NB, BS = 37, 16, 4, 64, 8, 256
    qkv = torch.randn(T, (Hq + 2 * Hkv) * D, device=DEV).to(torch.bfloat16)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(T, Hkv, D)
    kc = torch.zeros(NB, BS, Hkv, D, device=DEV, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    slots = torch.arange(T, device=DEV, dtype=torch.int64) * 3
    K.store_kvcache(k, v, kc, vc, slots)
    torch.cuda.synchronize()
    assert torch.equal(kc.view(-1, Hkv, D)[slots], k)
    assert torch.equal(vc.view(-1, Hkv, D)[slots], v)
    mask = torch.ones(NB * BS, dtype=torch.bool, device=DEV)
    mask[slots] = False
    assert not kc.view(-1, Hkv, D)[mask].any() and not vc.view(-1, Hkv, D)[mask].any()


def test_store_kvcache_skips_all_padding():
    kc = torch.ones(4, 16, 2, 64, device=DEV, dtype=torch.bfloat16)
    vc = torch.ones_like(kc)
    key = torch.zeros(5, 2, 64, device=DEV, dtype=torch.bfloat16)
    K.store_kvcache(key, key, kc, vc, torch.full((5,), -1, device=DEV, dtype=torch.int64))
    torch.cuda.synchronize()
    assert bool((kc == 1).all()) and bool((vc == 1).all())


def test_store_kvcache_cfg4_full_pool_past_2_31_elements():
    """cfg4's whole 65536-block pool (2^34 bf16 elements per cache): the
    decode slots of all 256 sequences (most of them past element 2^31), the
    pool's last slot, -1 padding and one slot past the pool (skipped) are
    written into NaN-poisoned caches.  The written blocks equal the oracle's
    store on a compacted copy of those blocks bit for bit, and a reduction on
    the GPU finds every other element still poisoned."""
    case = W.paged_case("cfg4", seed=3)
    NB, BS, Hkv, D = case.num_blocks, case.block_size, case.num_kv_heads, case.head_dim
    assert NB == 65536 and NB * BS * Hkv * D == 1 << 34
    slots = np.concatenate([case.slot_mapping, [NB * BS - 1, -1, NB * BS, 5]]).astype(np.int64)
    T = len(slots)
    valid = (slots >= 0) & (slots < NB * BS)
    assert (slots[valid] * Hkv * D >= 1 << 31).sum() > T // 2
    POISON = -1  # 0xFFFF: a bf16 NaN
    kc = torch.full((NB, BS, Hkv, D), POISON, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    vc = torch.full((NB, BS, Hkv, D), POISON, dtype=torch.int16, device=DEV).view(torch.bfloat16)
    g = torch.Generator(device=DEV).manual_seed(31)
    key = torch.randn(T, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    val = torch.randn(T, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    K.store_kvcache(key, val, kc, vc, torch.from_numpy(slots).to(DEV))
    torch.cuda.synchronize()
    blocks = np.unique(slots[valid] // BS)
    remap = {int(b): i for i, b in enumerate(blocks)}
    local = np.array([remap[int(s_) // BS] * BS + int(s_) % BS if ok else -1 for s_, ok in zip(slots, valid)],
                     np.int64)
    k0 = np.full((len(blocks), BS, Hkv, D), POISON, np.int16)
    v0 = k0.copy()
    P.store_kvcache(bits(key), bits(val), k0, v0, local)
    idx = torch.from_numpy(blocks).to(DEV)
    np.testing.assert_array_equal(kc.view(torch.int16)[idx].cpu().numpy(), k0)
    np.testing.assert_array_equal(vc.view(torch.int16)[idx].cpu().numpy(), v0)
    for cache in (kc, vc):  # nothing outside the written slots changed (checked in 8 slices of 4 GiB)
        rows = cache.view(torch.int16).view(NB * BS, Hkv * D)
        step = NB * BS // 8
        hit = np.concatenate([torch.nonzero((rows[i:i + step] != POISON).any(dim=1)).flatten().cpu().numpy() + i
                              for i in range(0, NB * BS, step)])
        np.testing.assert_array_equal(hit, np.unique(slots[valid]))
    del kc, vc
    torch.cuda.empty_cache()


# ------------------------------------------------------------ paged decode --
def host_inputs(case, kc, vc, q):
    """Copy only the referenced blocks to the host for the oracle."""
    ids = W.referenced_blocks(case)
    remap = np.full(case.num_blocks, -1, np.int64)
    remap[ids] = np.arange(len(ids))
    idt = torch.from_numpy(ids).to(DEV)
    kh = kc[idt].float().cpu().numpy()
    vh = vc[idt].float().cpu().numpy()
    bt = case.block_tables
    bt_local = np.where(bt >= 0, remap[np.maximum(bt, 0)], -1)
    return q.float().cpu().numpy(), kh, vh, bt_local


def run_decode(case, kc, vc, q, bps=None):
    cl = torch.from_numpy(case.context_lens).to(DEV)
    bt = torch.from_numpy(case.block_tables).to(DEV)
    return K.paged_attention_decode(q, kc, vc, cl, bt, case.scale, blocks_per_split=bps)


def make_q(case, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(case.batch, case.num_q_heads, case.head_dim, generator=g, device=DEV,
                       dtype=torch.bfloat16)


@pytest.mark.parametrize("bps", [None, 0, -1, -2])
def test_paged_decode_cfg3_full(bps):
    """cfg3 against the float64 oracle: the default split, the balanced
    split, the single launch (one workgroup per (sequence, pair of kv
    heads)) and the single launch in the paired order (one per (sequence, kv
    head))."""
    case = W.paged_case("cfg3", seed=2)
    kc, vc = W.fill_pool(case, seed=2, device=DEV, only_referenced=False)
    q = make_q(case, 2)
    o = run_decode(case, kc, vc, q, bps)
    torch.cuda.synchronize()
    qh, kh, vh, bth = host_inputs(case, kc, vc, q)
    ref = P.paged_decode(qh, kh, vh, case.context_lens, bth, case.scale)
    assert_close(o.float().cpu().numpy(), ref, "cfg3")


def test_paged_decode_cfg4_subset_full_pool():
    """16 sequences of cfg4 over the full 65536-block pool (2^34 elements
    per cache: exercises 64-bit addressing and long split-K reductions)."""
    case = W.paged_case("cfg4", seed=3, batch=16)
    kc, vc = W.fill_pool(case, seed=3, device=DEV, only_referenced=True)
    q = make_q(case, 3)
    o = run_decode(case, kc, vc, q)
    torch.cuda.synchronize()
    qh, kh, vh, bth = host_inputs(case, kc, vc, q)
    ref = P.paged_decode(qh, kh, vh, case.context_lens, bth, case.scale)
    assert_close(o.float().cpu().numpy(), ref, "cfg4-subset")
    del kc, vc
    torch.cuda.empty_cache()


def test_paged_decode_cfg4_full_batch():
    """cfg4 at its full batch of 256 (lengths log-uniform to 32768 over the
    65536-block pool): the balanced split (the default) against 8-block
    fixed chunks on every (sequence, head), and 8 sampled sequences (the
    shortest, the longest and 6 random) against the float64 oracle on their
    own blocks."""
    case = W.paged_case("cfg4", seed=3)
    assert case.batch == 256
    kc, vc = W.fill_pool(case, seed=3, device=DEV, only_referenced=True)
    q = make_q(case, 11)
    o = run_decode(case, kc, vc, q, 0)
    fixed = run_decode(case, kc, vc, q, 8)
    torch.cuda.synchronize()
    on, fn = o.float().cpu().numpy(), fixed.float().cpu().numpy()
    assert np.isfinite(on).all()
    assert_close(on, fn, "cfg4 balanced vs fixed chunks")
    lens = case.context_lens
    pick = np.unique(np.concatenate([[int(lens.argmin()), int(lens.argmax())],
                                     np.random.default_rng(12).choice(256, 6, replace=False)]))
    BS = case.block_size
    for b in pick:
        nb = -(-int(lens[b]) // BS)
        ids = torch.from_numpy(case.block_tables[b, :nb].astype(np.int64)).to(DEV)
        kh, vh = kc[ids].float().cpu().numpy(), vc[ids].float().cpu().numpy()
        ref = P.paged_decode(q[b:b + 1].float().cpu().numpy(), kh, vh, lens[b:b + 1],
                             np.arange(nb, dtype=np.int32)[None, :], case.scale)
        assert_close(on[b:b + 1], ref, f"cfg4 sequence {b} (L={int(lens[b])})")
    del kc, vc
    torch.cuda.empty_cache()


def test_paged_decode_split_independence():
    case = W.paged_case("cfg3", seed=5, batch=12)
    kc, vc = W.fill_pool(case, seed=5, device=DEV)
    q = make_q(case, 5)
    outs = [run_decode(case, kc, vc, q, bps).float() for bps in (0, 1, 2, 3, 16, -1, -2)]
    for o in outs[1:]:
        assert_close(o.cpu().numpy(), outs[0].cpu().numpy(), "split")


@pytest.mark.parametrize("B,Hkv,G,D", [(128, 4, 3, 64), (96, 4, 3, 64), (256, 2, 4, 128), (40, 8, 2, 64)])
def test_paged_decode_paired_order(B, Hkv, G, D):
    """The paired order (blocks_per_split -2) at grids of one to two
    workgroups per CU (cfg5's B 128 x Hkv 4 = 512 on 256 CUs, 384, 512 and
    320): every (sequence, kv head) lands in exactly one workgroup whatever
    the ranking, so the output equals the single launch's (-1, the same four
    interleaved walks per head) bit for bit, and the float64 oracle within
    the file's bar.  Lengths with ties, zeros and a one-token context."""
    rng = np.random.default_rng(B * 10 + Hkv)
    BS = 256
    lens = rng.integers(1, 2049, B).astype(np.int64)
    lens[:6] = [0, 1, 2048, 2048, 700, 700]
    nblk = -(-lens // BS)
    NB = int(nblk.sum()) + 4
    maxb = int(nblk.max())
    perm = rng.permutation(NB)
    bt = np.full((B, maxb), -1, np.int32)
    off = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[off:off + nblk[b]]
        off += int(nblk[b])
    g = torch.Generator(device=DEV).manual_seed(B + D)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(B, Hkv * G, D, generator=g, device=DEV).to(torch.bfloat16)
    cl, btd = torch.from_numpy(lens).to(DEV), torch.from_numpy(bt).to(DEV)
    print(f"paired order: B {B} Hkv {Hkv} G {G} D {D}", flush=True)
    o2 = K.paged_attention_decode(q, kc, vc, cl, btd, blocks_per_split=-2)
    o1 = K.paged_attention_decode(q, kc, vc, cl, btd, blocks_per_split=-1)
    torch.cuda.synchronize()
    assert torch.equal(o2, o1)
    ref = P.paged_decode(q.float().cpu().numpy(), kc.float().cpu().numpy(), vc.float().cpu().numpy(), lens, bt,
                         1 / math.sqrt(D))
    assert_close(o2.float().cpu().numpy(), ref, "paired order")
    assert bool((o2[0] == 0).all())


def test_paged_decode_paired_order_rejects():
    """-2 needs B <= 256, and a quantised output needs whole 128-value
    groups per kv head (G * D % 128 == 0)."""
    BS, D, Hkv = 16, 64, 2
    kc = torch.zeros(4, BS, Hkv, D, device=DEV, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    for B, Hq, quant, msg in ((257, 4, False, "B <= 256"), (4, 6, True, "cannot quantise")):
        q = torch.zeros(B, Hq, D, device=DEV, dtype=torch.bfloat16)
        cl = torch.ones(B, device=DEV, dtype=torch.int64)
        bt = torch.zeros(B, 1, device=DEV, dtype=torch.int32)
        with pytest.raises(ValueError, match=msg):
            K.paged_attention_decode(q, kc, vc, cl, bt, blocks_per_split=-2, quant=quant)


@pytest.mark.parametrize("Hq,Hkv,D,BS", [(12, 4, 64, 256), (8, 8, 128, 16), (16, 2, 128, 32),
                                         (32, 4, 64, 64), (6, 2, 64, 48), (4, 1, 64, 16), (9, 3, 128, 64)])
def test_paged_decode_shapes(Hq, Hkv, D, BS):
    rng = np.random.default_rng(Hq * 1000 + D + BS)
    B, NB = 7, 128
    lens = np.array([1, 0, BS, BS + 1, 3 * BS - 1, 5, 2 * BS], np.int64)
    maxb = int((-(-lens // BS)).max()) + 1   # one extra -1 column
    perm = rng.permutation(NB)
    bt = np.full((B, maxb), -1, np.int32)
    pos = 0
    for b, L in enumerate(lens):
        nb = -(-int(L) // BS)
        bt[b, :nb] = perm[pos:pos + nb]
        pos += nb
    g = torch.Generator(device=DEV).manual_seed(7)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g, device=DEV).to(torch.bfloat16)
    scale = 1 / math.sqrt(D)
    ref = P.paged_decode(q.float().cpu().numpy(), kc.float().cpu().numpy(), vc.float().cpu().numpy(),
                         lens, bt, scale)
    G = Hq // Hkv
    v0 = vc[int(bt[0, 0]), 0].float().cpu().numpy()  # L=1 -> v0 of the matching kv head
    for bps in (None, -1, -2):  # the default split and the single launches
        o = K.paged_attention_decode(q, kc, vc, torch.from_numpy(lens).to(DEV), torch.from_numpy(bt).to(DEV),
                                     blocks_per_split=bps)
        torch.cuda.synchronize()
        got = o.float().cpu().numpy()
        assert_close(got, ref, f"Hq={Hq} Hkv={Hkv} D={D} BS={BS} bps={bps}")
        assert np.all(got[1] == 0)  # padding row
        assert_close(got[0], np.repeat(v0, G, axis=0), f"L=1 bps={bps}")


@pytest.mark.parametrize("Hq,Hkv,D,BS", [(12, 4, 64, 256), (16, 2, 128, 32), (6, 2, 64, 48)])
def test_paged_decode_fused_quant_equals_act_quant(Hq, Hkv, D, BS):
    """The merge's act_quant of each output row: codes and scales equal
    act_quant of the bf16 output bit for bit, for single-chunk, multi-chunk
    and padding rows alike; the bf16 output equals the unfused call's."""
    rng = np.random.default_rng(Hq + D + BS)
    B, NB = 7, 128
    lens = np.array([1, 0, BS, BS + 1, 3 * BS - 1, 5, 2 * BS], np.int64)
    maxb = int((-(-lens // BS)).max()) + 1
    perm = rng.permutation(NB)
    bt = np.full((B, maxb), -1, np.int32)
    pos = 0
    for b, L in enumerate(lens):
        nb = -(-int(L) // BS)
        bt[b, :nb] = perm[pos:pos + nb]
        pos += nb
    g = torch.Generator(device=DEV).manual_seed(17)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g, device=DEV).to(torch.bfloat16)
    cl, btd = torch.from_numpy(lens).to(DEV), torch.from_numpy(bt).to(DEV)
    # balanced (7 rows over the whole grid), chunks of one and two blocks, and
    # the single launch (its act_quant inside the workgroup: one kv head per
    # workgroup when G*D is a multiple of 128, else two)
    for bps in (0, 1, 2, -1) + ((-2,) if (Hq // Hkv) * D % 128 == 0 else ()):
        o, oq, os_ = K.paged_attention_decode(q, kc, vc, cl, btd, blocks_per_split=bps, quant=True)
        plain = K.paged_attention_decode(q, kc, vc, cl, btd, blocks_per_split=bps)
        assert torch.equal(o, plain)
        rq, rs = K.act_quant(o.view(B, -1))
        assert torch.equal(oq.view(torch.uint8), rq.view(torch.uint8)), f"codes bps={bps}"
        assert torch.equal(os_, rs), f"scales bps={bps}"
        assert bool((o[1] == 0).all())  # padding row


def _rope_table(D, max_pos=4096):
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device=DEV).float() / D))
    ang = torch.outer(torch.arange(max_pos, device=DEV).float(), inv)
    return torch.cat([ang.cos(), ang.sin()], -1).contiguous()


@pytest.mark.parametrize("Hq,Hkv,D,BS,B", [(12, 4, 64, 256, 128), (16, 4, 64, 256, 64), (6, 3, 64, 48, 20),
                                           (16, 2, 128, 32, 16), (8, 8, 128, 16, 9)])
def test_paged_decode_rope_equals_store_then_decode(Hq, Hkv, D, BS, B):
    """paged_attention_decode_rope (q/k norms, RoPE, slot write and the
    single-launch decode in one kernel) against qk_norm_rope_store followed
    by paged_attention_decode(-1, quant): the rotated q and the whole K/V
    pools bit-identical, the output within the file's bar of the unfused
    output and of the float64 oracle (the newest token enters the softmax in
    another order), the output's FP8 codes equal act_quant of its bf16
    output.  Rows: L = 1 (only the new token), a padding row (L = 0, slot
    -1), block-boundary lengths and random ones up to 4 blocks."""
    rng = np.random.default_rng(Hq * 100 + D + B)
    lens = rng.integers(1, 4 * BS + 1, B).astype(np.int64)
    lens[:5] = [1, 0, BS, BS + 1, 2 * BS]
    nblk = -(-lens // BS)
    NB = int(nblk.sum()) + 8
    maxb = int(nblk.max()) + 1
    perm = rng.permutation(NB)
    bt = np.full((B, maxb), -1, np.int32)
    off = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[off:off + nblk[b]]
        off += int(nblk[b])
    slots = np.where(lens > 0, bt[np.arange(B), np.maximum(lens - 1, 0) // BS].astype(np.int64) * BS
                     + (np.maximum(lens - 1, 0) % BS), -1)
    g = torch.Generator(device=DEV).manual_seed(B + D)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    width = (Hq + 2 * Hkv) * D
    qkv = torch.randn(B, width + 8, generator=g, device=DEV).to(torch.bfloat16)[:, :width]  # strided rows
    qw = torch.rand(Hq * D, generator=g, device=DEV) + 0.5
    kw = torch.rand(Hkv * D, generator=g, device=DEV) + 0.5
    cos_sin = _rope_table(D)
    pos = torch.from_numpy(np.maximum(lens - 1, 0)).to(DEV)
    eps = torch.finfo(torch.float32).eps
    cl, btd, sl = (torch.from_numpy(x).to(DEV) for x in (lens, bt, slots))
    scale = 1 / math.sqrt(D)
    print(f"rope decode: Hq {Hq} Hkv {Hkv} D {D} BS {BS} B {B}", flush=True)
    kc_a, vc_a = kc.clone(), vc.clone()
    q = K.qk_norm_rope_store(qkv, qw, kw, cos_sin, pos, Hq, Hkv, eps, kc_a, vc_a, sl)
    o_a, _, _ = K.paged_attention_decode(q, kc_a, vc_a, cl, btd, scale, -1, quant=True)
    q_b = torch.empty_like(q)
    o_b, oq_b, os_b = K.paged_attention_decode_rope(qkv, qw, kw, cos_sin, pos, Hq, Hkv, eps, kc, vc, sl, cl, btd,
                                                    scale, quant=True, q_rot=q_b)
    torch.cuda.synchronize()
    assert torch.equal(q_b.view(torch.int16), q.view(torch.int16)), "rotated q differs"
    assert torch.equal(kc.view(torch.int16), kc_a.view(torch.int16)), "K pool differs"
    assert torch.equal(vc.view(torch.int16), vc_a.view(torch.int16)), "V pool differs"
    got = o_b.float().cpu().numpy()
    assert_close(got, o_a.float().cpu().numpy(), "fused vs unfused")
    ref = P.paged_decode(q.float().cpu().numpy(), kc_a.float().cpu().numpy(), vc_a.float().cpu().numpy(),
                         lens, bt, scale)
    assert_close(got, ref, "fused vs oracle")
    assert np.all(got[1] == 0)  # padding row
    rq, rs = K.act_quant(o_b.view(B, -1))
    assert torch.equal(oq_b.view(torch.uint8), rq.view(torch.uint8)) and torch.equal(os_b, rs)
    # and without the quantised output: the paired order where B * Hkv is
    # between one and two workgroups per CU (the newest token then enters
    # the softmax last), the same launch as above elsewhere
    q_c = torch.empty_like(q)
    kc_c, vc_c = kc_a.clone(), vc_a.clone()
    o_c = K.paged_attention_decode_rope(qkv, qw, kw, cos_sin, pos, Hq, Hkv, eps, kc_c, vc_c, sl, cl, btd, scale,
                                        q_rot=q_c)
    torch.cuda.synchronize()
    assert torch.equal(q_c.view(torch.int16), q.view(torch.int16)), "rotated q differs (no quant)"
    assert torch.equal(kc_c.view(torch.int16), kc_a.view(torch.int16))
    assert torch.equal(vc_c.view(torch.int16), vc_a.view(torch.int16))
    assert_close(o_c.float().cpu().numpy(), ref, "fused, no quant, vs oracle")
    assert np.all(o_c[1].float().cpu().numpy() == 0)


def test_paged_decode_rope_rejects_bad_shapes():
    """The fused prologue holds one q/k unit per thread: (Hq + Hkv) * D / 16
    above 256 is refused (use_fused_decode_rope says no for it)."""
    B, Hq, Hkv, D, BS = 2, 32, 8, 128, 16
    assert not K.use_fused_decode_rope(256, Hq, Hkv, D, 4, BS)
    qkv = torch.zeros(B, (Hq + 2 * Hkv) * D, device=DEV, dtype=torch.bfloat16)
    kc = torch.zeros(4, BS, Hkv, D, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="must be <= 256"):
        K.paged_attention_decode_rope(qkv, torch.ones(Hq * D, device=DEV), torch.ones(Hkv * D, device=DEV),
                                      _rope_table(D), torch.zeros(B, dtype=torch.int64, device=DEV), Hq, Hkv,
                                      1e-6, kc, kc.clone(), None, torch.ones(B, dtype=torch.int64, device=DEV),
                                      torch.zeros(B, 1, dtype=torch.int32, device=DEV))


def _short_sequences(B, BS, max_len, seed):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, max_len + 1, B).astype(np.int64)
    lens[::7] = 0  # padding rows between live ones
    nblk = -(-lens // BS)
    NB = int(nblk.sum()) + 1
    maxb = int(nblk.max()) + 1
    perm = rng.permutation(NB)
    bt = np.full((B, maxb), -1, np.int32)
    pos = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[pos:pos + nblk[b]]
        pos += int(nblk[b])
    return lens, bt, NB


def test_paged_decode_balanced_many_short_sequences():
    """Balanced split with many more sequences than threads of a workgroup
    (the per-thread runs of the tile-count scan) and workgroups that cover
    several whole sequences plus pieces of their neighbours: every row is
    within tolerance of the oracle, padding rows are zero, and the fused
    act_quant codes equal act_quant of the output."""
    B, Hq, Hkv, D, BS = 2000, 8, 2, 64, 16
    lens, bt, NB = _short_sequences(B, BS, 90, seed=21)
    g = torch.Generator(device=DEV).manual_seed(21)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g, device=DEV).to(torch.bfloat16)
    cl, btd = torch.from_numpy(lens).to(DEV), torch.from_numpy(bt).to(DEV)
    assert K.default_blocks_per_split(B, Hkv, bt.shape[1], BS) == 0
    o, oq, os_ = K.paged_attention_decode(q, kc, vc, cl, btd, quant=True)
    plain = K.paged_attention_decode(q, kc, vc, cl, btd)
    torch.cuda.synchronize()
    assert torch.equal(o, plain)
    ref = P.paged_decode(q.float().cpu().numpy(), kc.float().cpu().numpy(), vc.float().cpu().numpy(),
                         lens, bt, 1 / math.sqrt(D))
    got = o.float().cpu().numpy()
    assert_close(got, ref, "balanced, 2000 short sequences")
    assert np.all(got[lens == 0] == 0)
    rq, rs = K.act_quant(o.view(B, -1))
    assert torch.equal(oq.view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(os_, rs)


def test_paged_decode_large_batch_falls_back_to_fixed_chunks():
    """Above BALANCED_MAX_BATCH sequences the default is fixed chunks, and an
    explicit balanced request is refused rather than run."""
    B, Hq, Hkv, D, BS = K.BALANCED_MAX_BATCH + 8, 4, 1, 64, 16
    lens, bt, NB = _short_sequences(B, BS, 20, seed=22)
    g = torch.Generator(device=DEV).manual_seed(22)
    kc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    vc = torch.randn(NB, BS, Hkv, D, generator=g, device=DEV).to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=g, device=DEV).to(torch.bfloat16)
    cl, btd = torch.from_numpy(lens).to(DEV), torch.from_numpy(bt).to(DEV)
    assert K.default_blocks_per_split(B, Hkv, bt.shape[1], BS) > 0
    o = K.paged_attention_decode(q, kc, vc, cl, btd)
    torch.cuda.synchronize()
    ref = P.paged_decode(q.float().cpu().numpy(), kc.float().cpu().numpy(), vc.float().cpu().numpy(),
                         lens, bt, 1 / math.sqrt(D))
    assert_close(o.float().cpu().numpy(), ref, "fixed chunks, large batch")
    with pytest.raises(Exception, match="balanced split"):
        K.paged_attention_decode(q, kc, vc, cl, btd, blocks_per_split=0)


def test_paged_decode_balanced_workspace_bound():
    """The balanced split's partial rows stay inside the byte count that
    paged_decode_workspace_bytes promises: a workspace of exactly that size,
    guarded by NaN-filled canaries on both sides, is enough and the canaries
    survive (cfg4 geometry, the largest partial count per call)."""
    case = W.paged_case("cfg4", seed=3, batch=48)
    kc, vc = W.fill_pool(case, seed=3, device=DEV, only_referenced=True)
    q = make_q(case, 4)
    cl = torch.from_numpy(case.context_lens).to(DEV)
    bt = torch.from_numpy(case.block_tables).to(DEV)
    need = K.paged_decode_workspace_bytes(case.batch, case.num_q_heads, case.head_dim, bt.shape[1], 0)
    guard = 4096
    buf = torch.full((need + 2 * guard,), 0xFF, dtype=torch.uint8, device=DEV)
    ws = buf[guard:guard + need]
    o = K.paged_attention_decode(q, kc, vc, cl, bt, case.scale, 0, ws)
    ref = K.paged_attention_decode(q, kc, vc, cl, bt, case.scale, 8)
    torch.cuda.synchronize()
    assert bool((buf[:guard] == 0xFF).all()) and bool((buf[guard + need:] == 0xFF).all())
    assert_close(o.float().cpu().numpy(), ref.float().cpu().numpy(), "balanced vs fixed chunks")
    del kc, vc
    torch.cuda.empty_cache()


def test_decode_step_store_then_attend():
    """The decode step of the attention layer: write the new token's K/V at
    its slot, then attend over the context including it."""
    case = W.paged_case("cfg3", seed=8, batch=8)
    kc, vc = W.fill_pool(case, seed=8, device=DEV)
    g = torch.Generator(device=DEV).manual_seed(9)
    k_new = torch.randn(case.batch, case.num_kv_heads, case.head_dim, generator=g, device=DEV).to(torch.bfloat16)
    v_new = torch.randn(case.batch, case.num_kv_heads, case.head_dim, generator=g, device=DEV).to(torch.bfloat16)
    slots = P.decode_slots(case.block_tables, case.context_lens, case.block_size)
    np.testing.assert_array_equal(slots, case.slot_mapping)
    K.store_kvcache(k_new, v_new, kc, vc, torch.from_numpy(slots).to(DEV))
    q = make_q(case, 9)
    o = run_decode(case, kc, vc, q)
    torch.cuda.synchronize()
    qh, kh, vh, bth = host_inputs(case, kc, vc, q)
    assert_close(o.float().cpu().numpy(), P.paged_decode(qh, kh, vh, case.context_lens, bth, case.scale),
                 "store+decode")

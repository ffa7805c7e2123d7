"""Seeded synthetic inputs for the benchmark configurations.

Shapes and distributions follow the benchmark configs (cfg1..cfg4):
  cfg1  FP8 linear: x bf16 [256, 512] ~N(0,1), W bf16 [1344, 512] ~N(0,0.02)
  cfg2  FP8 GEMM sweep: (K, N) in {(1024,4096), (4096,1024), (2048,5632)},
        M in {1, 16, 128, 4096, 16384}; x ~N(0,1) with 0.1% of entries at
        +-40; W ~N(0,0.02)
  cfg3  paged decode, GQA 16/4 heads, D 64, block 256, batch 64, context
        lengths uniform in [128, 4096], tables = rows of a permutation of a
        4096-block pool, scale 1/8
  cfg4  long-context decode, GQA 32/8, D 128, block 256, batch 256, lengths
        log-uniform in [512, 32768], 65536-block pool, scale 1/sqrt(128)
  cfg3_4k  cfg3's geometry with every context 4096 tokens (batch 64 / 4K
        context, the decode target's literal reading)

Host-side metadata (lengths, tables, slots) comes from numpy's seeded
generator; tensor contents from a seeded torch generator on the target
device, so the same seed gives the same bits on every run.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

GEMM_KN = [(1024, 4096), (4096, 1024), (2048, 5632)]
GEMM_M = [1, 16, 128, 4096, 16384]


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activation(M: int, K: int, seed: int, device="cpu", outliers: bool = True) -> torch.Tensor:
    """bf16 [M, K] ~N(0,1); with outliers, 0.1% of entries (seeded positions
    and signs) set to +-40."""
    g = _gen(device, seed)
    x = torch.randn(M, K, generator=g, device=device, dtype=torch.float32)
    if outliers and M * K > 0:
        n = max(1, (M * K) // 1000)
        idx = torch.randperm(M * K, generator=g, device=device)[:n]
        sign = torch.where(torch.rand(n, generator=g, device=device) < 0.5, -40.0, 40.0)
        x.view(-1)[idx] = sign
    return x.to(torch.bfloat16)


def weight(N: int, K: int, seed: int, device="cpu", std: float = 0.02) -> torch.Tensor:
    g = _gen(device, seed)
    return (torch.randn(N, K, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)


@dataclass
class PagedCase:
    num_q_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    context_lens: np.ndarray   # int64 [B]
    block_tables: np.ndarray   # int32 [B, max_blocks], -1 padded
    slot_mapping: np.ndarray   # int64 [B], slot of each sequence's newest token
    scale: float

    @property
    def batch(self) -> int:
        return len(self.context_lens)

    def kv_bytes(self) -> int:
        """Algorithmic decode traffic: K and V rows read once, q read, o
        written, tables and lengths read."""
        B = self.batch
        rows = int(self.context_lens.sum()) * self.num_kv_heads * self.head_dim * 2 * 2
        qo = 2 * B * self.num_q_heads * self.head_dim * 2
        return rows + qo + 4 * B * self.block_tables.shape[1] + 8 * B


CONFIGS = {
    "cfg3": dict(Hq=16, Hkv=4, D=64, BS=256, B=64, NB=4096, lens=("uniform", 128, 4096), scale=1 / 8),
    # the north star's decode target read literally: batch 64, every context 4096 tokens
    "cfg3_4k": dict(Hq=16, Hkv=4, D=64, BS=256, B=64, NB=4096, lens=("fixed", 4096, 4096), scale=1 / 8),
    "cfg4": dict(Hq=32, Hkv=8, D=128, BS=256, B=256, NB=65536, lens=("loguniform", 512, 32768),
                 scale=1 / math.sqrt(128)),
}


def paged_case(name: str, seed: int, batch: int | None = None) -> PagedCase:
    """Metadata of a paged-decode config: lengths, block tables from one
    permutation of the pool (each sequence takes ceil(L/BS) consecutive
    entries of it), and the decode slot of each newest token."""
    c = CONFIGS[name]
    rng = np.random.default_rng(seed)
    B = c["B"]
    kind, lo, hi = c["lens"]
    if kind == "uniform":
        lens = rng.integers(lo, hi + 1, B)
    elif kind == "fixed":
        lens = np.full(B, lo, np.int64)
    else:
        lens = np.round(np.exp(rng.uniform(math.log(lo), math.log(hi), B))).astype(np.int64)
    if batch is not None:
        lens = lens[:batch]
        B = batch
    BS, NB = c["BS"], c["NB"]
    nblk = -(-lens // BS)
    maxb = int(nblk.max()) if B else 0
    perm = rng.permutation(NB)
    assert int(nblk.sum()) <= NB
    bt = np.full((B, maxb), -1, np.int32)
    pos = 0
    for b in range(B):
        bt[b, :nblk[b]] = perm[pos:pos + nblk[b]]
        pos += int(nblk[b])
    last = lens - 1
    slots = bt[np.arange(B), last // BS].astype(np.int64) * BS + last % BS
    return PagedCase(c["Hq"], c["Hkv"], c["D"], BS, NB, lens.astype(np.int64), bt, slots, c["scale"])


def referenced_blocks(case: PagedCase) -> np.ndarray:
    bt = case.block_tables
    return np.unique(bt[bt >= 0])


def fill_pool(case: PagedCase, seed: int, device, only_referenced: bool = True):
    """bf16 K and V pools [NB, BS, Hkv, D] ~N(0,1).  With only_referenced,
    blocks no table points at are left unwritten (they are never read)."""
    shape = (case.num_blocks, case.block_size, case.num_kv_heads, case.head_dim)
    g = _gen(device, seed)
    if not only_referenced:
        k = torch.randn(shape, generator=g, device=device, dtype=torch.bfloat16)
        v = torch.randn(shape, generator=g, device=device, dtype=torch.bfloat16)
        return k, v
    k = torch.empty(shape, device=device, dtype=torch.bfloat16)
    v = torch.empty(shape, device=device, dtype=torch.bfloat16)
    ids = torch.from_numpy(referenced_blocks(case)).to(device)
    blk = (len(ids), *shape[1:])
    k[ids] = torch.randn(blk, generator=g, device=device, dtype=torch.bfloat16)
    v[ids] = torch.randn(blk, generator=g, device=device, dtype=torch.bfloat16)
    return k, v

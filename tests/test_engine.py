"""Host-side engine: sequences, block manager, scheduler, metadata, context,
sampler (CPU only).

Slots are checked against the brute-force restatement
slot(b, t) = bt[b][t // BS] * BS + t % BS of the oracle, including the
L % BS == 0 case where the reference's formula is off by a block.
"""
import math

import numpy as np
import pytest
import torch

from llm_from_scratch_amd.context import get_context, reset_context, set_context
from llm_from_scratch_amd.engine import BlockManager, Sampler, SamplingParams, Scheduler, Sequence
from llm_from_scratch_amd.engine.model_runner import decode_metadata, prefill_metadata
from llm_from_scratch_amd.engine.sequence import SequenceStatus
from oracle import paged_kv as ref


@pytest.fixture(autouse=True)
def block_size_16():
    old = Sequence.block_size
    Sequence.block_size = 16
    yield 16
    Sequence.block_size = old


def test_sequence_block_accounting():
    BS = Sequence.block_size
    for n in range(1, 3 * BS + 2):
        s = Sequence(list(range(n)))
        assert s.num_blocks == math.ceil(n / BS)
        assert s.last_block_num_tokens == (n - 1) % BS + 1
        assert sum(len(s.block(i)) for i in range(s.num_blocks)) == n
        assert s.block(s.num_blocks - 1) == list(range((s.num_blocks - 1) * BS, n))


def test_decode_slots_match_brute_force():
    BS = Sequence.block_size
    bm = BlockManager(64, BS)
    rng = np.random.default_rng(0)
    seqs = []
    # lengths around block boundaries, including exact multiples of BS
    for n in [1, BS - 1, BS, BS + 1, 2 * BS, 3 * BS - 1, 3 * BS, 37]:
        s = Sequence(rng.integers(0, 1000, n).tolist())
        bm.allocate(s)
        seqs.append(s)
    m = decode_metadata(seqs, BS)
    width = max(len(s.block_table) for s in seqs)
    bt = np.array([s.block_table + [-1] * (width - len(s.block_table)) for s in seqs])
    want = ref.decode_slots(bt, [len(s) for s in seqs], BS)
    assert m["slot_mapping"] == want.tolist()
    assert m["positions"] == [len(s) - 1 for s in seqs]
    assert m["context_lens"] == [len(s) for s in seqs]
    assert m["input_ids"] == [s.token_ids[-1] for s in seqs]


def test_prefill_slots_cover_every_uncached_token():
    BS = Sequence.block_size
    bm = BlockManager(64, BS)
    shared = list(range(100, 100 + 2 * BS))
    a = Sequence(shared + [1, 2, 3])
    b = Sequence(shared + [7] * (BS + 5))
    c = Sequence(list(range(3 * BS)))          # full last block
    for s in (a, b, c):
        bm.allocate(s)
    assert a.num_cached_tokens == 0 and b.num_cached_tokens == 2 * BS and c.num_cached_tokens == 0
    m = prefill_metadata([a, b, c], BS)
    slots, k = m["slot_mapping"], 0
    for s in (a, b, c):
        start = s.num_cached_tokens
        bt = np.array([s.block_table])
        for t in range(start, len(s)):
            assert slots[k] == ref.decode_slots(bt, [t + 1], BS)[0], (s.seq_id, t)
            k += 1
    assert k == len(slots)
    assert m["cu_seqlens_q"] == [0, len(a), len(a) + len(b) - 2 * BS, len(a) + len(b) - 2 * BS + len(c)]
    assert m["cu_seqlens_k"] == [0, len(a), len(a) + len(b), len(a) + len(b) + len(c)]
    assert m["positions"][len(a):len(a) + 3] == [2 * BS, 2 * BS + 1, 2 * BS + 2]


def test_block_manager_refcounts_and_free_list():
    BS = Sequence.block_size
    bm = BlockManager(8, BS)
    prompt = list(range(2 * BS + 3))
    a, b = Sequence(prompt), Sequence(prompt)
    bm.allocate(a)
    assert len(bm.free_block_ids) == 5 and all(bm.blocks[i].ref_count == 1 for i in a.block_table)
    bm.allocate(b)  # two full blocks hit the prefix cache, the partial one does not
    assert b.block_table[:2] == a.block_table[:2] and b.block_table[2] != a.block_table[2]
    assert b.num_cached_tokens == 2 * BS
    assert [bm.blocks[i].ref_count for i in b.block_table] == [2, 2, 1]
    bm.deallocate(a)
    bm.deallocate(b)
    assert len(bm.free_block_ids) == 8 and not bm.used_block_ids
    assert all(blk.ref_count == 0 for blk in bm.blocks)
    # freeing a block forgets its tokens (engine/block_manager.py:71-78), so a
    # later identical prompt is a cache miss and gets fresh blocks
    c = Sequence(prompt)
    bm.allocate(c)
    assert c.num_cached_tokens == 0 and [bm.blocks[i].ref_count for i in c.block_table] == [1, 1, 1]


def test_block_manager_append_at_block_boundaries():
    BS = Sequence.block_size
    bm = BlockManager(4, BS)
    s = Sequence(list(range(BS - 1)))
    bm.allocate(s)
    assert len(s.block_table) == 1
    s.append_token(5)                       # fills block 0
    assert bm.can_append(s)
    bm.append(s)
    assert bm.blocks[s.block_table[0]].hash != -1 and len(s.block_table) == 1
    s.append_token(6)                       # opens block 1
    assert bm.can_append(s)
    bm.append(s)
    assert len(s.block_table) == 2
    for t in range(BS - 1):
        s.append_token(t)
        bm.append(s)
    assert len(s.block_table) == 2 and len(s) == 2 * BS
    # exhaust the pool: appending a token that opens a new block must be refused
    bm.allocate(Sequence(list(range(2 * BS))))
    assert not bm.free_block_ids
    s.append_token(1)
    assert not bm.can_append(s)


def _drive(sched: Scheduler, eos: int, rng) -> dict[int, list[int]]:
    """Run the scheduler to completion with random tokens (never eos)."""
    finished, steps = {}, 0
    seen = set()
    while not sched.is_finished():
        seqs, is_prefill = sched.schedule()
        assert seqs, "scheduler made no progress"
        for s in seqs:
            assert s.status == SequenceStatus.RUNNING
            assert len(s.block_table) == s.num_blocks
        sched.postprocess(seqs, rng.integers(0, eos, len(seqs)).tolist())
        for s in seqs:
            seen.add(s.seq_id)
            if s.is_finished:
                finished[s.seq_id] = s.completion_token_ids
        steps += 1
        assert steps < 10000
    return finished


def test_scheduler_runs_every_sequence_to_max_tokens_with_preemption():
    BS = Sequence.block_size
    rng = np.random.default_rng(1)
    # a pool too small for all sequences at full length forces preemption
    sched = Scheduler(max_num_sequences=4, max_num_batched_tokens=256, max_cached_blocks=9,
                      block_size=BS, eos=1000)
    seqs = [Sequence(rng.integers(0, 1000, n).tolist(), SamplingParams(max_tokens=mt))
            for n, mt in [(20, 30), (5, 40), (33, 12), (16, 17), (1, 25), (40, 8)]]
    for s in seqs:
        sched.add_sequence(s)
    out = _drive(sched, 1000, rng)
    assert sorted(out) == sorted(s.seq_id for s in seqs)
    for s in seqs:
        assert len(out[s.seq_id]) == s.max_tokens
    bm = sched.block_manager
    assert len(bm.free_block_ids) == 9 and not bm.used_block_ids


def test_scheduler_keeps_sequences_when_decode_batch_is_full():
    BS = Sequence.block_size
    rng = np.random.default_rng(2)
    sched = Scheduler(max_num_sequences=2, max_num_batched_tokens=64, max_cached_blocks=32,
                      block_size=BS, eos=1000)
    seqs = [Sequence([i] * 4, SamplingParams(max_tokens=6)) for i in range(5)]
    for s in seqs:
        sched.add_sequence(s)
    out = _drive(sched, 1000, rng)
    assert sorted(out) == [s.seq_id for s in seqs]
    assert all(len(v) == 6 for v in out.values())


def test_scheduler_stops_on_eos_and_max_model_length():
    BS = Sequence.block_size
    sched = Scheduler(4, 256, 16, BS, eos=7)
    a = Sequence([1, 2, 3], SamplingParams(max_tokens=100))
    b = Sequence([1, 2, 3], SamplingParams(max_tokens=100, ignore_eos=True, max_model_length=6))
    sched.add_sequence(a)
    sched.add_sequence(b)
    seqs, is_prefill = sched.schedule()
    assert is_prefill and seqs == [a, b]
    sched.postprocess(seqs, [7, 7])
    assert a.is_finished and not b.is_finished
    while not b.is_finished:
        seqs, _ = sched.schedule()
        sched.postprocess(seqs, [7] * len(seqs))
    assert len(b) == 6 and sched.is_finished()


def test_context_roundtrip():
    sm = torch.arange(4)
    set_context(False, slot_mapping=sm, context_lens=sm + 1, block_tables=sm.view(2, 2))
    ctx = get_context()
    assert not ctx.is_prefill and ctx.slot_mapping is sm and ctx.block_tables.shape == (2, 2)
    reset_context()
    ctx = get_context()
    assert ctx.slot_mapping is None and ctx.context_lens is None and not ctx.is_prefill


def test_sampler_needs_gpu_tensors():
    """The sampler is one HIP kernel (its distribution and parity with the
    reference formula are tested on the GPU): CPU tensors are refused, no
    CPU fallback."""
    s = Sampler()
    with pytest.raises(ValueError):
        s(torch.zeros(2, 8, dtype=torch.bfloat16), torch.ones(2), torch.Generator().manual_seed(0))


def test_block_aligned_prompt_fully_matching_keeps_a_query_token():
    """Two sequences with the same block-aligned prompt: the second one hits
    the prefix cache on every block but the last, which it recomputes into a
    block of its own, so its prefill has at least one query token (the
    reference would cache all blocks and leave none to sample from)."""
    BS = 16
    Sequence.block_size = BS
    bm = BlockManager(16, BS)
    prompt = list(range(3 * BS))
    a, b = Sequence(list(prompt)), Sequence(list(prompt))
    bm.allocate(a)
    bm.allocate(b)
    assert a.num_cached_tokens == 0
    assert b.num_cached_tokens == 2 * BS < b.num_tokens
    assert b.block_table[:2] == a.block_table[:2] and b.block_table[2] != a.block_table[2]
    assert bm.blocks[a.block_table[0]].ref_count == 2 and bm.blocks[b.block_table[2]].ref_count == 1
    m = prefill_metadata([a, b], BS)
    q = np.diff(m["cu_seqlens_q"])
    assert q.tolist() == [3 * BS, BS]
    assert len(m["slot_mapping"]) == 4 * BS  # every uncached block's slots
    bm.deallocate(b)
    bm.deallocate(a)
    assert len(bm.free_block_ids) == 16


def test_block_hash_is_chained_xxh64():
    """Prefix-cache block hashes: xxh64 (the reference's engine/block_manager.py:45-57 calls
    the same library) over the previous block's hash as 8 little-endian bytes, then the
    block's token ids as int32.  The library is pinned by xxHash's published known answers
    (empty input and "abc", seed 0); the chaining by hashes that must differ and agree."""
    import xxhash
    assert xxhash.xxh64(b"").intdigest() == 0xEF46DB3751D8E999
    assert xxhash.xxh64(b"abc").intdigest() == 0x44BC2CF5AD770999
    h0 = BlockManager.compute_hash([1, 2, 3])
    assert h0 == xxhash.xxh64(b"\x01\x00\x00\x00\x02\x00\x00\x00\x03\x00\x00\x00").intdigest()
    h1 = BlockManager.compute_hash([4, 5, 6], h0)
    assert h1 == xxhash.xxh64(h0.to_bytes(8, "little") + bytes([4, 0, 0, 0, 5, 0, 0, 0, 6, 0, 0, 0])).intdigest()
    assert h1 != BlockManager.compute_hash([4, 5, 6])  # the prefix changes the hash
    assert BlockManager.compute_hash([-1]) == xxhash.xxh64(b"\xff\xff\xff\xff").intdigest()

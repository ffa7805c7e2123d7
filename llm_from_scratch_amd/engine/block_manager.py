"""KV-block pool with prefix caching, as engine/block_manager.py of the
reference (same classes, methods and xxh64 block hashing over int32 token
bytes chained with the previous block's hash, :45-57).

Behavioural fixes (the reference's bugs are not copied):
  * a newly allocated block gets ref_count 1 (the reference never sets it,
    :60-69, so ``deallocate`` drives it to -1 and freed blocks never return
    to the free list, :116-124);
  * ``can_append`` asks for a free block when the sequence's newest token
    starts a new block (num_tokens % BS == 1) -- the case in which
    ``append`` allocates -- rather than at num_tokens % BS == 0 (:130-134
    vs :149-153), which let ``append`` pop an empty free list;
  * a prompt's last block is never taken from the prefix cache (:85-114
    would cache every block of a block-aligned prompt that matches another
    sequence's, leaving the prefill no query token to sample from): it is
    recomputed into a fresh block, so num_cached_tokens < num_tokens.
"""
from __future__ import annotations

from collections import deque

import numpy as np
import xxhash

from .sequence import Sequence


class Block:
    def __init__(self, block_id: int):
        self.block_id = block_id
        self.hash = -1
        self.ref_count = 0
        self.token_ids: list[int] = []

    def update(self, h: int, token_ids: list[int]):
        self.hash = h
        self.token_ids = token_ids

    def reset(self):
        self.hash = -1
        self.ref_count = 0
        self.token_ids = []


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.hash_to_block_id: dict[int, int] = {}
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()

    @staticmethod
    def compute_hash(token_ids: list[int], prefix_hash_value: int = -1) -> int:
        h = xxhash.xxh64()
        if prefix_hash_value != -1:
            h.update(prefix_hash_value.to_bytes(8, "little"))
        h.update(np.array(token_ids, dtype=np.int32).tobytes())
        return h.intdigest()

    def _allocate_block(self, block_id: int) -> Block:
        block = self.blocks[block_id]
        assert block.ref_count == 0, "Block is already allocated"
        block.reset()
        block.ref_count = 1
        self.free_block_ids.remove(block_id)
        self.used_block_ids.add(block_id)
        return block

    def _deallocate_block(self, block_id: int) -> None:
        assert self.blocks[block_id].ref_count == 0, "Block is still in use"
        self.blocks[block_id].token_ids = []
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)

    def can_allocate(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= seq.num_blocks

    def allocate(self, seq: Sequence) -> None:
        assert not seq.block_table
        h = -1
        cache_miss = False
        for i in range(seq.num_blocks):
            token_ids = seq.block(i)
            h = self.compute_hash(token_ids, h) if len(token_ids) == self.block_size else -1
            block_id = self.hash_to_block_id.get(h, -1)
            if block_id == -1 or self.blocks[block_id].token_ids != token_ids:
                cache_miss = True
            if i == seq.num_blocks - 1:
                cache_miss = True  # the last prompt token is always computed
            if not cache_miss:
                seq.num_cached_tokens += self.block_size
                if block_id in self.used_block_ids:
                    block = self.blocks[block_id]
                    block.ref_count += 1
                else:
                    block = self._allocate_block(block_id)
            else:
                block = self._allocate_block(self.free_block_ids[0])
                block.update(h, token_ids)
                if h != -1:
                    self.hash_to_block_id[h] = block.block_id
            seq.block_table.append(block.block_id)

    def deallocate(self, seq: Sequence) -> None:
        for block_id in seq.block_table:
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self._deallocate_block(block_id)
        seq.block_table = []
        seq.num_cached_tokens = 0

    def can_append(self, seq: Sequence) -> bool:
        if seq.num_tokens % self.block_size == 1:
            return len(self.free_block_ids) > 0
        return True

    def append(self, seq: Sequence) -> None:
        """Account for the sequence's newest token (already appended)."""
        table = seq.block_table
        last = self.blocks[table[-1]]
        if seq.num_tokens % self.block_size == 1:
            # the newest token opens a new block
            assert last.hash != -1, "previous block should be full and hashed"
            block = self._allocate_block(self.free_block_ids[0])
            table.append(block.block_id)
        elif seq.num_tokens % self.block_size == 0:
            # the newest token fills the last block: it becomes cacheable
            assert last.hash == -1
            token_ids = seq.block(seq.num_blocks - 1)
            prefix = self.blocks[table[-2]].hash if len(table) > 1 else -1
            h = self.compute_hash(token_ids, prefix)
            last.update(h, token_ids)
            self.hash_to_block_id[h] = last.block_id
        else:
            assert last.hash == -1

"""Prefill-first scheduler with preemption, as engine/scheduler.py of the
reference (same queues, policy and stopping rules).

Behavioural fixes (the reference's bugs are not copied):
  * a running sequence popped when the decode batch is already full goes
    back to the front of ``running`` (the reference's ``break`` at :59-61
    drops it from every queue);
  * after preempting the newest running sequence the current one is retried
    with the freed blocks (the reference, :53-54, drops it);
  * ``max_tokens`` stops a sequence after exactly ``max_tokens`` completion
    tokens (the reference's ``1 + num_completion_tokens`` test, :89, stops
    one token early).
"""
from __future__ import annotations

from collections import deque

from .block_manager import BlockManager
from .sequence import Sequence, SequenceStatus


class Scheduler:
    def __init__(self, max_num_sequences: int, max_num_batched_tokens: int, max_cached_blocks: int,
                 block_size: int, eos: int):
        self.block_manager = BlockManager(max_cached_blocks, block_size)
        self.max_num_batched_tokens = max_num_batched_tokens
        self.max_num_sequences = max_num_sequences
        self.waiting: deque[Sequence] = deque()
        self.running: deque[Sequence] = deque()
        self.eos = eos

    def is_finished(self) -> bool:
        return not self.waiting and not self.running

    def add_sequence(self, sequence: Sequence) -> None:
        self.waiting.append(sequence)

    def schedule(self) -> tuple[list[Sequence], bool]:
        """Prefill as many waiting sequences as fit; otherwise one decode token
        for each running sequence, preempting the newest ones when the pool
        cannot hold another block (engine/scheduler.py:26-69)."""
        scheduled: list[Sequence] = []
        num_tokens = 0
        while self.waiting and len(scheduled) < self.max_num_sequences:
            seq = self.waiting[0]
            if (self.block_manager.can_allocate(seq)
                    and len(seq) + num_tokens <= self.max_num_batched_tokens):
                self.waiting.popleft()
                self.block_manager.allocate(seq)
                seq.status = SequenceStatus.RUNNING
                self.running.append(seq)
                scheduled.append(seq)
                num_tokens += len(seq)
            else:
                break
        if scheduled:
            return scheduled, True

        while self.running:
            seq = self.running.popleft()
            if not self.block_manager.can_append(seq):
                if self.running:
                    self.preempt(self.running.pop())
                    self.running.appendleft(seq)  # retry it with the freed blocks
                    continue
                self.preempt(seq)
                break
            if num_tokens >= self.max_num_batched_tokens or len(scheduled) >= self.max_num_sequences:
                self.running.appendleft(seq)
                break
            self.block_manager.append(seq)
            scheduled.append(seq)
            num_tokens += 1
        if scheduled:
            self.running.extendleft(reversed(scheduled))
        return scheduled, False

    def preempt(self, seq: Sequence) -> None:
        self.block_manager.deallocate(seq)
        seq.status = SequenceStatus.WAITING
        self.waiting.appendleft(seq)

    def postprocess(self, seqs: list[Sequence], token_ids: list[int]) -> None:
        """Append each sampled token; finish on EOS, max_tokens or
        max_model_length (engine/scheduler.py:79-95)."""
        for seq, token_id in zip(seqs, token_ids):
            seq.append_token(token_id)
            stop_eos = not seq.ignore_eos and token_id == self.eos
            stop_max_tokens = seq.num_completion_tokens >= seq.max_tokens
            stop_max_len = seq.max_model_length is not None and seq.num_tokens >= seq.max_model_length
            if stop_eos or stop_max_tokens or stop_max_len:
                seq.status = SequenceStatus.FINISHED
                self.block_manager.deallocate(seq)
                self.running.remove(seq)

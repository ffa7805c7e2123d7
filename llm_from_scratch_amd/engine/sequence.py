"""Sequence state, as engine/sequence.py of the reference (same attributes and
methods).  One behavioural fix: ``last_block_num_tokens`` is ``block_size``
(not 0) when the length is a positive multiple of the block size, so the
decode slot ``block_table[-1]*BS + last_block_num_tokens - 1`` and the
prefill slot list of a full last block are right (the reference returns 0,
engine/sequence.py:67-69, which points the decode slot into the previous
block and gives a full last block an empty slot list).
"""
from __future__ import annotations

import math
from copy import copy
from dataclasses import dataclass
from enum import Enum, auto
from itertools import count
from typing import Optional


@dataclass
class SamplingParams:
    """utils/sampler.py:7-23 of the reference, plus the ``max_model_length``
    field engine/sequence.py:34 reads from it."""
    temperature: float = 1.0
    max_tokens: int = 256
    ignore_eos: bool = False
    max_model_length: Optional[int] = None

    def __post_init__(self):
        assert self.temperature > 1e-10, "greedy sampling is not permitted"


class SequenceStatus(Enum):
    WAITING = auto()
    RUNNING = auto()
    FINISHED = auto()


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, token_ids: list[int], sampling_params: Optional[SamplingParams] = None):
        sp = sampling_params or SamplingParams()
        self.seq_id = next(Sequence.counter)
        self.status = SequenceStatus.WAITING
        self.token_ids = copy(token_ids)
        self.last_token = self.token_ids[-1] if self.token_ids else None
        self.num_tokens = len(self.token_ids)
        self.num_prompt_tokens = len(self.token_ids)
        self.num_cached_tokens = 0
        self.block_table: list[int] = []
        self.temperature = sp.temperature
        self.max_tokens = sp.max_tokens
        self.ignore_eos = sp.ignore_eos
        self.max_model_length = sp.max_model_length

    def __len__(self):
        return self.num_tokens

    def __getitem__(self, idx):
        return self.token_ids[idx]

    @property
    def is_finished(self):
        return self.status == SequenceStatus.FINISHED

    @property
    def num_completion_tokens(self):
        return self.num_tokens - self.num_prompt_tokens

    @property
    def prompt_token_ids(self):
        return self.token_ids[:self.num_prompt_tokens]

    @property
    def completion_token_ids(self):
        return self.token_ids[self.num_prompt_tokens:]

    @property
    def num_cached_blocks(self):
        return int(math.ceil(self.num_cached_tokens / self.block_size))

    @property
    def num_blocks(self):
        return int(math.ceil(self.num_tokens / self.block_size))

    @property
    def last_block_num_tokens(self):
        """Tokens in the last (possibly full) block: num_tokens - (num_blocks-1)*BS."""
        if self.num_tokens == 0:
            return 0
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def block(self, i):
        assert 0 <= i < self.num_blocks, f"Block index {i} out of range [0, {self.num_blocks})"
        return self.token_ids[i * self.block_size:(i + 1) * self.block_size]

    def append_token(self, token_id):
        self.token_ids.append(token_id)
        self.last_token = token_id
        self.num_tokens += 1

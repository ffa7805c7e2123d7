"""Generation loop over the scheduler and the model runner, as
engine/llm_engine.py of the reference (step / add_prompt / generate).

One GPU, one process: the runner is called directly instead of through the
reference's worker processes and shared-memory RPC.  Prompts are token-id
lists; a tokenizer object (anything with ``encode``/``decode``) may be passed
for string prompts, since the reference's ``AutoTokenizer.from_pretrained``
fetches from the network.  ``step`` always returns three values (the
reference returns two when nothing is scheduled, :62-64).
"""
from __future__ import annotations

import time
from typing import Optional, Sequence as Seq, Union

import torch

from .model_runner import ModelRunner
from .scheduler import Scheduler
from .sequence import SamplingParams, Sequence


class LLMEngine:
    def __init__(self, model: torch.nn.Module, config: dict, tokenizer=None, device="cuda",
                 generator: Optional[torch.Generator] = None, verbose: bool = False):
        self.model_runner = ModelRunner(model, config, device)
        block_size = config.get("block_size", 256)
        Sequence.block_size = block_size
        self.scheduler = Scheduler(
            max_num_sequences=config.get("max_num_sequences", config.get("max_num_seqs", 16)),
            max_num_batched_tokens=config.get("max_num_batched_tokens", 1024),
            max_cached_blocks=min(config.get("max_cached_blocks", self.model_runner.num_available_kv_blocks),
                                  self.model_runner.num_available_kv_blocks),
            block_size=block_size,
            eos=config.get("eos", 50256))
        self.tokenizer = tokenizer
        self.generator = generator
        self.verbose = verbose

    def step(self):
        seqs, is_prefill = self.scheduler.schedule()
        if not seqs:
            return [], 0, is_prefill
        token_ids = self.model_runner.run(seqs, is_prefill, self.generator)
        self.scheduler.postprocess(seqs, token_ids)
        outputs = [(s.seq_id, s.completion_token_ids) for s in seqs if s.is_finished]
        n = sum(len(s) for s in seqs) if is_prefill else len(seqs)
        return outputs, n, is_prefill

    def add_prompt(self, prompt: Union[str, list[int]], sampling_params: SamplingParams) -> None:
        if isinstance(prompt, str):
            assert self.tokenizer is not None, "string prompts need a tokenizer"
            prompt = self.tokenizer.encode(prompt)
        self.scheduler.add_sequence(Sequence(list(prompt), sampling_params))

    def generate(self, prompts: Seq[Union[str, list[int]]], sampling_params: SamplingParams) -> dict:
        for p in prompts:
            self.add_prompt(p, sampling_params)
        done: dict[int, list[int]] = {}
        while not self.scheduler.is_finished():
            t0 = time.perf_counter()
            outputs, n, is_prefill = self.step()
            if self.verbose:
                dt = time.perf_counter() - t0 + 1e-10
                print(f"{'prefill' if is_prefill else 'decode'}: {n} tokens, {n / dt:.1f} tokens/s")
            done.update(outputs)
        token_ids = [done[k] for k in sorted(done)]
        text = [self.tokenizer.decode(t) for t in token_ids] if self.tokenizer is not None else None
        return {"text": text, "token_ids": token_ids}

"""Paged-KV serving engine: sequences, block manager, scheduler, model runner."""
from .block_manager import Block, BlockManager
from .llm_engine import LLMEngine
from .model_runner import ModelRunner, Sampler
from .scheduler import Scheduler
from .sequence import SamplingParams, Sequence, SequenceStatus

__all__ = ["Block", "BlockManager", "LLMEngine", "ModelRunner", "Sampler", "Scheduler",
           "SamplingParams", "Sequence", "SequenceStatus"]

"""Single-GPU model runner: KV pool, attention metadata, graph-captured decode.

Counterpart of engine/model_runner.py of the reference with the same method
names and data contract (one MI355X, so no process group or shared-memory
RPC):
  warmup_model        one prefill of max_num_batched_tokens // max_model_length
                      full-length sequences before the pool exists, so the
                      peak activation memory is known (:151-159)
  allocate_kv_cache   one pool [2, L, NB, BS, Hkv, D] of free x
                      gpu_memory_utilization - (peak - current) bytes after
                      the warm-up (or num_kv_blocks blocks when given);
                      per-layer k_cache / v_cache views attached to modules
                      that have them (:162-190)
  prepare_prefill     input ids / positions of uncached tokens, cu_seqlens,
                      slot_mapping over uncached blocks, block tables when a
                      prefix is cached (:202-249)
  prepare_decode      last token, position L-1, slot of the newest token,
                      context_lens (int64), block tables padded with -1
                      (:253-278)
  run_model           eager prefill; decode replays the smallest captured
                      graph whose batch fits, with padding rows given slot -1
                      and context length 0 (:288-312)
  capture_cudagraph   graphs for bs in [1,2,4,8] + range(16, max_bs+1, 16)
                      over static buffers (:339-392)
The decode slot is bt[-1]*BS + last_block_num_tokens - 1 with the corrected
last_block_num_tokens (a full last block counts BS tokens).
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .. import kernels
from ..context import get_context, reset_context, set_context
from .sequence import Sequence


def prefill_metadata(seqs: list[Sequence], block_size: int) -> dict:
    """Host lists for a prefill batch (engine/model_runner.py:202-249): ids and
    positions of the tokens not covered by cached blocks, cu_seqlens over
    query (uncached) and key (full) lengths, and the slots of every token in
    the uncached blocks (a full last block contributes block_size slots)."""
    input_ids, positions, slots = [], [], []
    cu_q, cu_k = [0], [0]
    max_q = max_k = 0
    BS = block_size
    for seq in seqs:
        start = seq.num_cached_tokens
        input_ids.extend(seq.token_ids[start:])
        positions.extend(range(start, seq.num_tokens))
        lq, lk = seq.num_tokens - start, seq.num_tokens
        cu_q.append(cu_q[-1] + lq)
        cu_k.append(cu_k[-1] + lk)
        max_q, max_k = max(max_q, lq), max(max_k, lk)
        for i in range(seq.num_cached_blocks, seq.num_blocks):
            n = BS if i != seq.num_blocks - 1 else seq.last_block_num_tokens
            slots.extend(range(seq.block_table[i] * BS, seq.block_table[i] * BS + n))
    return dict(input_ids=input_ids, positions=positions, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k,
                max_seqlen_q=max_q, max_seqlen_k=max_k, slot_mapping=slots)


def decode_metadata(seqs: list[Sequence], block_size: int) -> dict:
    """Host lists for a decode batch (engine/model_runner.py:253-278): the
    newest token of each sequence at position L-1, its slot
    block_table[-1]*BS + last_block_num_tokens - 1, and L as context length."""
    return dict(input_ids=[s.last_token for s in seqs],
                positions=[len(s) - 1 for s in seqs],
                context_lens=[len(s) for s in seqs],
                slot_mapping=[s.block_table[-1] * block_size + s.last_block_num_tokens - 1 for s in seqs])


class Sampler:
    """Temperature + Gumbel-max sampling (utils/sampler.py:35-53): argmax of
    softmax(logits / T) / Exp(1) noise, in one kernel (kernels.sample_gumbel).

    The noise comes from a counter-based generator keyed by a seed and a
    per-call offset: the seed is the given generator's initial seed, or one
    drawn from torch's default generator on first use (so torch.manual_seed
    makes runs repeatable); the offset advances every call."""

    def __init__(self):
        self._seed: Optional[int] = None
        self._offset = 0

    def __call__(self, logits: torch.Tensor, temperatures: torch.Tensor,
                 generator: Optional[torch.Generator] = None) -> torch.Tensor:
        if generator is not None:
            seed = generator.initial_seed()
        else:
            if self._seed is None:
                self._seed = int(torch.randint(0, 2 ** 62, (1,)).item())
            seed = self._seed
        offset = self._offset
        self._offset += (logits.size(-1) + 3) // 4
        return kernels.sample_gumbel(logits.to(torch.bfloat16), temperatures.to(torch.float32), seed, offset)


class ModelRunner:
    def __init__(self, model: torch.nn.Module, config: dict, device="cuda"):
        self.model = model
        self.config = config
        self.device = torch.device(device)
        self.block_size = config.get("block_size", 256)
        self.enforce_eager = config.get("enforce_eager", False)
        self.sampler = Sampler()
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.graph_vars: dict[str, torch.Tensor] = {}
        if "num_kv_blocks" not in config:
            self.warmup_model()
        self.allocate_kv_cache()
        if not self.enforce_eager:
            self.capture_cudagraph()

    # ------------------------------------------------------------ KV pool --
    def _attach_pool(self, pool: torch.Tensor) -> None:
        layer = 0
        for module in self.model.modules():
            if hasattr(module, "k_cache") and hasattr(module, "v_cache"):
                module.k_cache = pool[0, layer]
                module.v_cache = pool[1, layer]
                layer += 1
        assert layer == self.config["num_layers"], \
            f"found {layer} attention layers, expected {self.config['num_layers']}"

    @torch.inference_mode()
    def warmup_model(self) -> None:
        """One prefill of max_num_batched_tokens // max_model_length sequences
        of max_model_length tokens (at least one sequence, at most the token
        budget long), as engine/model_runner.py:151-159, so that the peak of
        allocated memory holds the largest prefill's activations when
        allocate_kv_cache sizes the pool.  This model's attention writes
        every prompt's K/V into the pool before attending, so the warm-up
        runs over a temporary pool of exactly the warm-up's blocks, freed
        afterwards (its bytes count towards the reserved peak)."""
        cfg = self.config
        max_len = int(cfg.get("max_model_length", 4096))
        budget = int(cfg.get("max_num_batched_tokens", cfg.get("max_num_batch_tokens", max_len)))
        n_seq = max(1, budget // max_len)
        seq_len = min(max_len, budget)
        torch.cuda.empty_cache()
        torch.cuda.reset_peak_memory_stats(self.device)
        nblk = n_seq * math.ceil(seq_len / self.block_size)
        pool = torch.empty(2, cfg["num_layers"], nblk, self.block_size, cfg["num_kv_heads"],
                           cfg.get("head_dim", cfg["hidden_size"] // cfg["num_heads"]),
                           device=self.device, dtype=cfg.get("kv_dtype", torch.bfloat16))
        self._attach_pool(pool)
        seqs = [Sequence([0] * seq_len) for _ in range(n_seq)]
        per = math.ceil(seq_len / self.block_size)
        for i, sq in enumerate(seqs):
            sq.block_table = list(range(i * per, (i + 1) * per))
        ids, pos = self.prepare_prefill(seqs)
        self.model(ids, pos)
        torch.cuda.synchronize(self.device)
        reset_context()
        for module in self.model.modules():
            if hasattr(module, "k_cache") and hasattr(module, "v_cache"):
                module.k_cache = torch.empty(0)
                module.v_cache = torch.empty(0)
        del pool, ids, pos
        torch.cuda.empty_cache()

    def allocate_kv_cache(self) -> None:
        cfg = self.config
        num_layers = cfg["num_layers"]
        num_kv_heads = cfg["num_kv_heads"]
        head_dim = cfg.get("head_dim", cfg["hidden_size"] // cfg["num_heads"])
        dtype = cfg.get("kv_dtype", torch.bfloat16)
        block_bytes = self.block_size * 2 * num_layers * num_kv_heads * head_dim * dtype.itemsize
        if "num_kv_blocks" in cfg:
            nb = int(cfg["num_kv_blocks"])
        else:
            # free x utilisation, minus the room the warm-up prefill's
            # activations needed above what stays allocated
            # (engine/model_runner.py:162-168)
            free, _ = torch.cuda.mem_get_info(self.device)
            stats = torch.cuda.memory_stats(self.device)
            reserve = stats["allocated_bytes.all.peak"] - stats["allocated_bytes.all.current"]
            available = free * cfg.get("gpu_memory_utilization", 0.9) - reserve
            nb = int(available // block_bytes)
            self.kv_reserved_bytes = reserve
        assert nb >= 1, "Not enough memory to hold at least one block of KV cache"
        self.num_available_kv_blocks = nb
        self.kv_cache = torch.empty(2, num_layers, nb, self.block_size, num_kv_heads, head_dim,
                                    device=self.device, dtype=dtype)
        self._attach_pool(self.kv_cache)

    # ----------------------------------------------------------- metadata --
    def _pad_tables(self, seqs: list[Sequence]) -> torch.Tensor:
        width = max(len(s.block_table) for s in seqs)
        rows = [s.block_table + [-1] * (width - len(s.block_table)) for s in seqs]
        return torch.tensor(rows, dtype=torch.int32, pin_memory=True).to(self.device, non_blocking=True)

    def prepare_prefill(self, seqs: list[Sequence]):
        m = prefill_metadata(seqs, self.block_size)
        pin = dict(pin_memory=True)

        def dev(x, dtype):
            return torch.tensor(x, dtype=dtype, **pin).to(self.device, non_blocking=True)

        block_tables = self._pad_tables(seqs) if m["cu_seqlens_q"][-1] < m["cu_seqlens_k"][-1] else None
        set_context(True, dev(m["cu_seqlens_q"], torch.int32), dev(m["cu_seqlens_k"], torch.int32),
                    m["max_seqlen_q"], m["max_seqlen_k"], dev(m["slot_mapping"], torch.int64),
                    None, block_tables)
        return dev(m["input_ids"], torch.int64), dev(m["positions"], torch.int64)

    def prepare_decode(self, seqs: list[Sequence]):
        m = decode_metadata(seqs, self.block_size)
        pin = dict(pin_memory=True)

        def dev(x, dtype):
            return torch.tensor(x, dtype=dtype, **pin).to(self.device, non_blocking=True)

        set_context(False, None, None, 0, 0, dev(m["slot_mapping"], torch.int64),
                    dev(m["context_lens"], torch.int64), self._pad_tables(seqs))
        return dev(m["input_ids"], torch.int64), dev(m["positions"], torch.int64)

    def prepare_sample(self, seqs: list[Sequence]) -> torch.Tensor:
        return torch.tensor([s.temperature for s in seqs], dtype=torch.float32,
                            pin_memory=True).to(self.device, non_blocking=True)

    # --------------------------------------------------------------- run ---
    @torch.inference_mode()
    def run_model(self, input_ids: torch.Tensor, positions: torch.Tensor, is_prefill: bool) -> torch.Tensor:
        bs = input_ids.size(0)
        if is_prefill or self.enforce_eager or bs > self.max_graph_bs():
            return self.model.compute_logits(self.model(input_ids, positions))
        ctx = get_context()
        graph_bs = next(b for b in sorted(self.graphs) if b >= bs)
        v = self.graph_vars
        v["input_ids"][:bs] = input_ids
        v["positions"][:bs] = positions
        v["slot_mapping"].fill_(-1)
        v["slot_mapping"][:bs] = ctx.slot_mapping
        v["context_lens"].zero_()
        v["context_lens"][:bs] = ctx.context_lens
        v["block_tables"].fill_(-1)
        v["block_tables"][:bs, :ctx.block_tables.size(1)] = ctx.block_tables
        self.graphs[graph_bs].replay()
        return self.graph_logits(bs)

    def graph_logits(self, bs: int) -> torch.Tensor:
        """Logits of the first bs rows of the last replay of the graph that
        serves batch size bs.  A model with forward_q (its output's act_quant
        from the final norm's own launch) captured that, and its lm_head
        skips its own act_quant (the same codes and scales, so the same
        logits)."""
        graph_bs = next(b for b in sorted(self.graphs) if b >= bs)
        h, hq, hs = self.graph_outputs[graph_bs]
        if hq is not None:
            return self.model.compute_logits_q(hq[:bs], hs[:bs])
        return self.model.compute_logits(h[:bs])

    def run(self, seqs: list[Sequence], is_prefill: bool,
            generator: Optional[torch.Generator] = None) -> list[int]:
        input_ids, positions = self.prepare_prefill(seqs) if is_prefill else self.prepare_decode(seqs)
        logits = self.run_model(input_ids, positions, is_prefill)
        if is_prefill:
            # one logit row per sequence: the last prompt token
            last = get_context().cu_seqlens_q[1:] - 1
            logits = logits[last]
        token_ids = self.sampler(logits, self.prepare_sample(seqs), generator).tolist()
        reset_context()
        return token_ids

    # ------------------------------------------------------ graph capture --
    def max_graph_bs(self) -> int:
        return max(self.graphs) if self.graphs else 0

    @torch.inference_mode()
    def capture_cudagraph(self) -> None:
        cfg = self.config
        max_bs = min(cfg.get("max_num_seqs", 128), 512)
        max_blocks = math.ceil(cfg.get("max_model_length", 4096) / self.block_size)
        dev = self.device
        input_ids = torch.zeros(max_bs, dtype=torch.int64, device=dev)
        positions = torch.zeros(max_bs, dtype=torch.int64, device=dev)
        slot_mapping = torch.full((max_bs,), -1, dtype=torch.int64, device=dev)
        context_lens = torch.zeros(max_bs, dtype=torch.int64, device=dev)
        block_tables = torch.full((max_bs, max_blocks), -1, dtype=torch.int32, device=dev)
        sizes = [b for b in [1, 2, 4, 8] + list(range(16, max_bs + 1, 16)) if b <= max_bs]
        self.graph_outputs = {}
        pool = None
        for bs in reversed(sizes):
            graph = torch.cuda.CUDAGraph()
            set_context(False, slot_mapping=slot_mapping[:bs], context_lens=context_lens[:bs],
                        block_tables=block_tables[:bs])
            fwd = getattr(self.model, "forward_q", None)
            run = (lambda: fwd(input_ids[:bs], positions[:bs])) if fwd is not None else \
                (lambda: (self.model(input_ids[:bs], positions[:bs]), None, None))
            run()  # warm up outside capture
            with torch.cuda.graph(graph, pool):
                # the graph's own output tensors (in its pool), read after each
                # replay: no copy into a shared buffer
                self.graph_outputs[bs] = run()
            if pool is None:
                pool = graph.pool()
            self.graphs[bs] = graph
            torch.cuda.synchronize()
            reset_context()
        self.graph_vars = dict(input_ids=input_ids, positions=positions, slot_mapping=slot_mapping,
                               context_lens=context_lens, block_tables=block_tables)

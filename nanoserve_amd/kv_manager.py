"""Paged KV manager: how the scheduler and the engine get KV blocks for requests (host-side integers).

Decisions follow nanoserve/kv_manager.py:70-202 (PagedKVManager), pinned step by step by
tests/golden/host_traces.json:
  * admission needs the request's uncached tokens in whole blocks, less cached prefix hits, plus the hits
    that must be taken back from the parked (cached, unheld) set, within the free blocks minus a 1%
    watermark (:116-121);
  * with prefix caching a request starts from the longest cached prefix, leaving at least one token to
    compute, i.e. at most (len - 1) // block_size hit blocks (:101-107, :123-138);
  * per step: the slot of every scheduled token, the decode rows (one new token on a stored context,
    context length ctx + 1 including it), and at commit the registration of newly full blocks (:153-196).

Design (this build's own): one call, batch(plan), turns a StepPlan into a StepBatch -- the flattened token
ids, positions and slots, one SeqInput per sequence, and the decode rows' indices, tables and context
lengths as plain lists -- which the executor stages straight into its pinned buffers (graph steps) or
turns into tensors (eager steps). Every prefill sequence carries its block table, a fresh one included:
the HIP prefill attention reads its pages in place (the reference's SDPA path needs none for ctx = 0).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
from nanoserve_amd.model import DecodeMeta, ModelConfig, SeqInput


@dataclass
class StepBatch:
    """Everything the model needs for one step, host side."""
    token_ids: list[int] = field(default_factory=list)
    positions: list[int] = field(default_factory=list)
    slots: list[int] = field(default_factory=list)
    seqs: list[SeqInput] = field(default_factory=list)
    tables: list[list[int]] = field(default_factory=list)   # per sequence: its block list (the live list)
    dec_idx: list[int] = field(default_factory=list)        # decode rows: index in the flattened step
    dec_tables: list[list[int]] = field(default_factory=list)
    dec_lens: list[int] = field(default_factory=list)       # context incl. this step's token
    n_prefill: int = 0                                      # sequences that are prefilling

    @property
    def n_tokens(self) -> int:
        return len(self.token_ids)

    @property
    def pure_decode(self) -> bool:
        return len(self.dec_idx) == len(self.seqs)


class PagedKVManager:
    kind = "paged"

    def __init__(self, cfg: ModelConfig, budget_tokens: int, block_size: int = 16, device="cuda",
                 dtype=torch.bfloat16, watermark: float = 0.01, prefix_caching: bool = False):
        self.pool = PagedKVCache.from_token_budget(cfg, budget_tokens, block_size, device, dtype, prefix_caching)
        self.alloc = self.pool.allocator
        self.block_size = block_size
        self.device = device
        self.prefix_caching = prefix_caching
        self.prefix_query_tokens = 0     # prompt tokens looked up at admission
        self.prefix_hit_tokens = 0       # ... of which were found cached (prefill skipped)
        self.watermark_blocks = math.floor(watermark * self.pool.num_blocks)

    @property
    def num_free_blocks(self) -> int:
        return self.alloc.num_free

    def refcount(self, block: int) -> int:
        return self.alloc.refcount(block)

    def reset_stats(self) -> None:
        self.prefix_query_tokens = self.prefix_hit_tokens = 0

    def _prefix_hits(self, seq) -> list[int]:
        if not self.prefix_caching:
            return []
        return self.alloc.lookup(seq.tokens, max_blocks=(seq.num_tokens - 1) // self.block_size)

    # ------------------------------------------------------------------------- scheduler interface
    def can_ever_fit(self, n_tokens: int) -> bool:
        return -(-n_tokens // self.block_size) <= self.pool.num_blocks

    def can_admit(self, seq) -> bool:
        hits = self._prefix_hits(seq)
        parked = sum(1 for b in hits if self.alloc.refcount(b) == 0)   # taking them back uses free capacity
        need = -(-seq.step_cost // self.block_size) - len(hits) + parked
        return need <= self.alloc.num_free - self.watermark_blocks

    def admit(self, seq) -> None:
        table = BlockTable(self.block_size)
        if self.prefix_caching:
            self.prefix_query_tokens += seq.num_tokens
            hits = self._prefix_hits(seq)
            if hits:
                self.alloc.pin(hits)
                table.blocks = list(hits)
                table.num_hashed = len(hits)
                table.num_tokens = seq.num_cached = len(hits) * self.block_size
                table.prefix_node = self.alloc.node_of(hits[-1])
                self.prefix_hit_tokens += table.num_tokens
        seq.block_table = table
        table.reserve(seq.step_cost, self.alloc)

    def try_append(self, seq) -> bool:
        """Room for one more token; False if the pool cannot provide the block it needs."""
        t = seq.block_table
        if t.blocks_needed(1) > self.alloc.num_free:
            return False
        t.reserve(1, self.alloc)
        return True

    def free(self, seq) -> None:
        if seq.block_table is not None:
            seq.block_table.release(self.alloc)
            seq.block_table = None

    # ---------------------------------------------------------------------------- engine interface
    def batch(self, plan) -> StepBatch:
        """The step's model inputs, in plan order."""
        sb = StepBatch()
        for seq, n in zip(plan.scheduled, plan.chunks):
            t = seq.block_table
            ctx = t.num_tokens
            toks, pos = seq.step_tokens(n)
            row = len(sb.token_ids)
            sb.token_ids += toks
            sb.positions += pos
            sb.slots += t.slots(n)
            sb.tables.append(t.blocks)
            if n == 1 and ctx > 0:
                sb.dec_idx.append(row)
                sb.dec_tables.append(t.blocks)
                sb.dec_lens.append(ctx + 1)
                sb.seqs.append(SeqInput(1, ctx_len=ctx, use_kernel=True))
            else:
                sb.seqs.append(SeqInput(n, block_table=t.blocks, ctx_len=ctx))
            sb.n_prefill += seq.is_prefill
        return sb

    def decode_meta(self, sb: StepBatch, width: int | None = None) -> DecodeMeta | None:
        """Device tensors of the decode rows (tables padded with 0 to `width`, default the widest row)."""
        if not sb.dec_idx:
            return None
        w = width or max(len(t) for t in sb.dec_tables)
        rows = [t + [0] * (w - len(t)) for t in sb.dec_tables]
        dev = self.device
        return DecodeMeta(token_idx=torch.tensor(sb.dec_idx, device=dev),
                          block_tables=torch.tensor(rows, dtype=torch.int32, device=dev),
                          context_lens=torch.tensor(sb.dec_lens, dtype=torch.int32, device=dev),
                          all_rows=sb.pure_decode)

    def commit(self, seq, n_tokens: int) -> None:
        t = seq.block_table
        t.commit(n_tokens)
        if self.prefix_caching and t.num_tokens // self.block_size > t.num_hashed:
            self.alloc.register(t, seq.tokens)      # newly full blocks become reusable

    def usage(self, running) -> tuple[int, int]:
        """(tokens actually stored, tokens reserved = blocks held x block_size)."""
        used = held = 0
        for s in running:
            if s.block_table is not None:
                used += s.block_table.num_tokens
                held += len(s.block_table.blocks)
        return used, held * self.block_size

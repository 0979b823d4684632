"""Paged KV manager: the scheduler's and engine's interface to the block pool (host-side integers).

Semantics follow nanoserve/kv_manager.py:70-202 (PagedKVManager):
  * admission by an explicit token budget, keeping a 1% watermark of blocks free (:116-121);
  * with prefix caching, admission starts from the longest cached prefix, leaving at least one token to
    compute, i.e. at most (len - 1) // block_size hit blocks (:101-107, :123-138);
  * per step: slot mapping of every scheduled token, DecodeMeta for one-token decodes on a context
    (ctx + 1 including the new token, tables as int32 padded with 0 to the step's widest), graph inputs,
    and registration of newly full blocks at commit (:153-196).
The contiguous manager of the reference (M1/M2 A/B comparisons) is not part of the decode loop.
"""
from __future__ import annotations

import math

import torch

from nanoserve_amd.kv_cache import BlockTable, PagedKVCache, PrefixCachingAllocator
from nanoserve_amd.model import DecodeMeta, ModelConfig, SeqInput


class PagedKVManager:
    kind = "paged"

    def __init__(self, cfg: ModelConfig, budget_tokens: int, block_size: int = 16, device="cuda",
                 dtype=torch.bfloat16, watermark: float = 0.01, attn_backend: str = "hip",
                 prefix_caching: bool = False):
        self.pool = PagedKVCache.from_token_budget(cfg, budget_tokens, block_size, device, dtype)
        self.block_size = block_size
        self.device = device
        self.attn_backend = attn_backend
        self.prefix_caching = prefix_caching
        self.alloc = (PrefixCachingAllocator(self.pool.allocator, block_size) if prefix_caching
                      else self.pool.allocator)
        self.prefix_query_tokens = 0     # prompt tokens looked up at admission
        self.prefix_hit_tokens = 0       # ... of which were found cached (prefill skipped)
        self.watermark_blocks = math.floor(watermark * self.pool.num_blocks)
        self._slots: list[int] = []
        self._offset = 0
        self._dec_idx: list[int] = []
        self._dec_tables: list[list[int]] = []
        self._dec_lens: list[int] = []

    @property
    def num_free_blocks(self) -> int:
        return self.alloc.num_free

    def refcount(self, block: int) -> int:
        """How many block tables hold `block` (1 for an allocated block without prefix caching)."""
        ref = getattr(self.alloc, "ref", None)
        if ref is not None:
            return ref.get(block, 0)
        return int(block in self.alloc._used)

    def _blocks_for(self, n_tokens: int) -> int:
        return math.ceil(n_tokens / self.block_size)

    def _hits(self, seq) -> list[int]:
        """Cached blocks of the longest known prefix, leaving >= 1 token to compute (its logits are needed)."""
        if not self.prefix_caching:
            return []
        toks = seq.prompt_ids + seq.output_ids
        return self.alloc.lookup(toks, max_blocks=(len(toks) - 1) // self.block_size)

    def reset_stats(self) -> None:
        self.prefix_query_tokens = self.prefix_hit_tokens = 0

    # --- scheduler interface
    def can_ever_fit(self, n_tokens: int) -> bool:
        return self._blocks_for(n_tokens) <= self.pool.num_blocks

    def can_admit(self, seq) -> bool:
        hits = self._hits(seq)
        parked = sum(1 for b in hits if self.alloc.ref.get(b, 0) == 0)   # pinning them uses free capacity
        need = self._blocks_for(seq.step_cost) - len(hits) + parked
        return need <= self.num_free_blocks - self.watermark_blocks

    def admit(self, seq) -> None:
        table = BlockTable(self.block_size)
        if self.prefix_caching:
            hits = self._hits(seq)
            self.prefix_query_tokens += seq.num_tokens
            if hits:
                self.alloc.pin(hits)
                table.blocks = list(hits)
                table.num_hashed = len(hits)
                table.num_tokens = len(hits) * self.block_size
                table.prefix_node = self.alloc.node_of[hits[-1]]
                seq.num_cached = table.num_tokens
                self.prefix_hit_tokens += table.num_tokens
        seq.block_table = table
        table.reserve(seq.step_cost, self.alloc)

    def try_append(self, seq) -> bool:
        """Room for one more token (a decode step); False if the pool is out of blocks."""
        if seq.block_table.blocks_needed(1) > self.num_free_blocks:
            return False
        seq.block_table.reserve(1, self.alloc)
        return True

    def free(self, seq) -> None:
        if seq.block_table is not None:
            seq.block_table.release(self.alloc)
            seq.block_table = None

    # --- engine interface
    def begin_step(self) -> None:
        self._slots = []
        self._offset = 0
        self._dec_idx, self._dec_tables, self._dec_lens = [], [], []

    def seq_input(self, seq, n_tokens: int) -> SeqInput:
        table = seq.block_table
        self._slots += table.slots(n_tokens)
        ctx = table.num_tokens
        use_kernel = n_tokens == 1 and ctx > 0
        if use_kernel:
            self._dec_idx.append(self._offset)
            self._dec_tables.append(table.blocks)
            self._dec_lens.append(ctx + 1)
        self._offset += n_tokens
        # the HIP attention reads every prefill token's pages in place: give it the table (also ctx == 0)
        bt = None if use_kernel else torch.tensor(table.blocks, dtype=torch.int32, device=self.device)
        return SeqInput(n_tokens, block_table=bt, ctx_len=ctx, use_kernel=use_kernel)

    def decode_meta(self) -> DecodeMeta | None:
        """Kernel inputs of this step's one-token decodes (None if there are none)."""
        if not self._dec_idx:
            return None
        width = max(len(t) for t in self._dec_tables)
        tables = [t + [0] * (width - len(t)) for t in self._dec_tables]
        all_rows = self._dec_idx == list(range(self._offset))
        return DecodeMeta(token_idx=torch.tensor(self._dec_idx, device=self.device),
                          block_tables=torch.tensor(tables, dtype=torch.int32, device=self.device),
                          context_lens=torch.tensor(self._dec_lens, dtype=torch.int32, device=self.device),
                          all_rows=all_rows)

    def forward_kwargs(self) -> dict:
        kw = {"paged": self.pool, "slot_mapping": torch.tensor(self._slots, device=self.device)}
        meta = self.decode_meta()
        if meta is not None:
            kw["decode_meta"] = meta
        return kw

    def graph_inputs(self) -> tuple[list[int], list[list[int]], list[int]]:
        """(slots, block tables, context lens) of this step's decodes, for the graph path."""
        return self._slots, self._dec_tables, self._dec_lens

    def commit(self, seq, n_tokens: int) -> None:
        table = seq.block_table
        table.commit(n_tokens)
        if self.prefix_caching and table.num_tokens // self.block_size > table.num_hashed:
            self.alloc.register(table, seq.prompt_ids + seq.output_ids)

    def usage(self, running) -> tuple[int, int]:
        """(tokens actually stored, tokens reserved = blocks held x block_size)."""
        used = sum(s.block_table.num_tokens for s in running if s.block_table)
        held = sum(len(s.block_table.blocks) for s in running if s.block_table)
        return used, held * self.block_size

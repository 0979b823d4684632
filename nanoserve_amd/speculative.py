"""Greedy speculative decoding with a draft model, on the HIP decode path.

Behaviour of nanoserve/speculative.py:64-305 (SpeculativeEngine): the draft proposes k tokens one step at a
time; the target checks all of them in ONE pass over [newest token, d1 .. dk] and yields its own greedy
choice t0 .. tk at every position; the longest prefix with d_{i+1} == t_i is accepted, followed by the
target's token at the first mismatch (or the bonus tk when all k match). Every emitted token is the
target's greedy choice given the tokens before it, so the output equals plain greedy decoding with the
target. KV bookkeeping: both models' tables are reserved up front for prompt + max_new + k + 1 tokens; the
target's KV covers every token but the newest and is rewound past rejected drafts after each round; the
draft may lag one token and catches up in its next round (a 2-token step).

Design (this build's own): each model runs in a Lane -- its pool, its decode graph runner and one
`greedy(items)` call that feeds each item's new tokens on top of its table and returns the greedy token at
every fed position. A lane turns every new token into its own decode row that shares the sequence's block
table with context length ctx + j + 1, so the paged decode kernel applies causality by itself and a
verification of k + 1 tokens, or the draft's catch-up, is one ordinary graph replay (the argmax runs inside
the graph). Rows beyond the largest graph bucket, and prefills, run the eager HIP forward.
"""
from __future__ import annotations

import math
import time
from collections import deque

import torch

from nanoserve_amd.engine import StepOutput
from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
from nanoserve_amd.model import Qwen2Model, SeqInput


class SpecSeq:
    __slots__ = ("seq_id", "tokens", "n_prompt", "max_new_tokens", "ignore_eos", "arrival_time", "tables")

    def __init__(self, seq_id, prompt_ids, max_new_tokens, ignore_eos, arrival_time):
        self.seq_id = seq_id
        self.tokens = list(prompt_ids)
        self.n_prompt = len(self.tokens)
        self.max_new_tokens, self.ignore_eos, self.arrival_time = max_new_tokens, ignore_eos, arrival_time
        self.tables: list[BlockTable] | None = None      # [target table, draft table]

    @property
    def prompt_ids(self) -> list[int]:
        return self.tokens[:self.n_prompt]

    @property
    def output_ids(self) -> list[int]:
        return self.tokens[self.n_prompt:]


class Lane:
    """One model of the pair: pool, graphs, and greedy tokens for tokens fed on top of tables."""

    def __init__(self, model: Qwen2Model, kv_tokens: int, block_size: int, span: int, cuda_graphs: bool):
        if model.device.type != "cuda":
            raise ValueError("speculative decoding runs the HIP kernels: put both models on the GPU")
        self.model = model
        self.pool = PagedKVCache.from_token_budget(model.cfg, kv_tokens, block_size, model.device, model.dtype)
        self.graphs = None
        if cuda_graphs:
            from nanoserve_amd.hip_graphs import DecodeGraphRunner
            self.graphs = DecodeGraphRunner(model, self.pool, span, pair_rows=True)
        self.graph_steps = 0
        self.forwards = 0

    def greedy(self, items: list[tuple[BlockTable, list[int]]], last_only: bool = False) -> list[list[int]]:
        """Feed each item's tokens after its table's stored ones (K/V written, tables committed); returns the
        greedy next token at every fed position (only the last one with last_only), per item."""
        self.forwards += 1
        n_rows = sum(len(t) for _, t in items)
        fresh = any(tab.num_tokens == 0 for tab, _ in items)
        if self.graphs is not None and not fresh and n_rows <= self.graphs.max_bucket:
            toks = self._rows(items)
            self.graph_steps += 1
        else:
            toks = self._eager(items, last_only)
        out, i = [], 0
        for tab, t in items:
            n = 1 if last_only and len(toks) == len(items) else len(t)
            out.append(toks[i:i + n][-1:] if last_only else toks[i:i + n])
            i += n
            tab.commit(len(t))
        return out

    def _rows(self, items) -> list[int]:
        tokens, positions, slots, tables, lens = [], [], [], [], []
        for tab, t in items:
            c = tab.num_tokens
            tokens += t
            positions += range(c, c + len(t))
            slots += tab.slots(len(t))
            tables += [tab.blocks] * len(t)
            lens += range(c + 1, c + len(t) + 1)
        self.graphs.run(tokens, positions, slots, tables, lens)
        return self.graphs.greedy_tokens(len(tokens))

    def _eager(self, items, last_only: bool) -> list[int]:
        from nanoserve_amd.kernels.sampling import argmax_rows
        tokens, positions, slots, seqs = [], [], [], []
        for tab, t in items:
            c = tab.num_tokens
            tokens += t
            positions += range(c, c + len(t))
            slots += tab.slots(len(t))
            seqs.append(SeqInput(len(t), block_table=tab.blocks, ctx_len=c))
        dev, m = self.model.device, self.model
        logits = m.forward_batch(torch.tensor(tokens, device=dev), torch.tensor(positions, device=dev), seqs,
                                 logits="last" if last_only else "all", paged=self.pool,
                                 slot_mapping=torch.tensor(slots, device=dev))
        return argmax_rows(logits).tolist()


class SpeculativeEngine:
    def __init__(self, target: Qwen2Model, draft: Qwen2Model, eos_token_ids: list[int],
                 num_speculative_tokens: int = 4, max_seq_len: int = 2048, max_num_seqs: int = 8,
                 max_num_batched_tokens: int = 4096, target_kv_tokens: int | None = None,
                 draft_kv_tokens: int | None = None, block_size: int = 16, cuda_graphs: bool | None = None):
        if target.cfg.vocab_size != draft.cfg.vocab_size:
            raise ValueError("draft and target must share a vocabulary")
        self.k = int(num_speculative_tokens)
        if self.k < 1:
            raise ValueError("num_speculative_tokens must be >= 1")
        self._eos = frozenset(eos_token_ids)
        self.eos_token_ids = list(eos_token_ids)
        self.max_seq_len, self.max_num_seqs, self.block_size = max_seq_len, max_num_seqs, block_size
        self.max_num_batched_tokens = max(max_num_batched_tokens, max_seq_len)
        span = max_seq_len + self.k + 1
        t_tokens = target_kv_tokens or 8 * span
        graphs = True if cuda_graphs is None else bool(cuda_graphs)
        self.lanes = [Lane(target, t_tokens, block_size, span, graphs),
                      Lane(draft, draft_kv_tokens or t_tokens, block_size, span, graphs)]
        self.waiting: deque[SpecSeq] = deque()
        self.running: list[SpecSeq] = []
        self.sequences: dict[int, SpecSeq] = {}
        self._next_id = 0
        self.reset_stats()

    @property
    def target(self) -> Qwen2Model:
        return self.lanes[0].model

    @property
    def draft(self) -> Qwen2Model:
        return self.lanes[1].model

    def reset_stats(self) -> None:
        self._stats = {"steps": 0, "proposed": 0, "accepted": 0, "emitted_by_verification": 0, "peak_running": 0}
        self._verifications = 0
        for lane in self.lanes:
            lane.graph_steps = lane.forwards = 0

    @property
    def stats(self) -> dict:
        s = dict(self._stats)
        tl, dl = self.lanes
        s.update(target_forwards=tl.forwards, draft_forwards=dl.forwards, graph_verify_steps=tl.graph_steps,
                 graph_draft_steps=dl.graph_steps, num_speculative_tokens=self.k, cuda_graphs=tl.graphs is not None)
        s["acceptance_rate"] = s["accepted"] / s["proposed"] if s["proposed"] else None
        s["tokens_per_target_forward"] = (s["emitted_by_verification"] / self._verifications
                                          if self._verifications else None)
        return s

    # ---------------------------------------------------------------------------------------- requests
    def _span(self, seq: SpecSeq) -> int:
        return seq.n_prompt + seq.max_new_tokens + self.k + 1

    def add_request(self, prompt_ids: list[int], max_new_tokens: int, ignore_eos: bool = False,
                    arrival_time: float | None = None, sampling=None) -> int:
        if sampling is not None and not getattr(sampling, "greedy", False):
            raise ValueError("speculative decoding here is greedy only")
        if len(prompt_ids) + max_new_tokens > self.max_seq_len:
            raise ValueError(f"prompt + max_new_tokens exceeds max_seq_len ({self.max_seq_len})")
        seq = SpecSeq(self._next_id, prompt_ids, max_new_tokens, ignore_eos,
                      time.perf_counter() if arrival_time is None else arrival_time)
        blocks = math.ceil(self._span(seq) / self.block_size)
        if blocks > min(lane.pool.num_blocks for lane in self.lanes):
            raise ValueError("request can never fit in the KV pools")
        self.waiting.append(seq)
        self.sequences[seq.seq_id] = seq
        self._next_id += 1
        return seq.seq_id

    def has_unfinished(self) -> bool:
        return bool(self.waiting) or bool(self.running)

    def _release(self, seq: SpecSeq) -> None:
        if seq.tables is not None:
            for tab, lane in zip(seq.tables, self.lanes):
                tab.release(lane.pool.allocator)
            seq.tables = None
        self.sequences.pop(seq.seq_id, None)

    def abort(self, seq_id: int) -> None:
        seq = self.sequences.get(seq_id)
        if seq is None:
            return
        if seq in self.running:
            self.running.remove(seq)
        elif seq in self.waiting:
            self.waiting.remove(seq)
        self._release(seq)

    def _admit(self) -> list[SpecSeq]:
        """FCFS while seats, the prefill budget and both pools allow (tables reserved for the whole span)."""
        out, budget = [], self.max_num_batched_tokens
        while self.waiting and len(self.running) + len(out) < self.max_num_seqs:
            seq = self.waiting[0]
            blocks = math.ceil(self._span(seq) / self.block_size)
            if seq.n_prompt > budget or any(blocks > lane.pool.allocator.num_free for lane in self.lanes):
                break
            self.waiting.popleft()
            seq.tables = []
            for lane in self.lanes:
                tab = BlockTable(self.block_size)
                tab.reserve(self._span(seq), lane.pool.allocator)
                seq.tables.append(tab)
            budget -= seq.n_prompt
            out.append(seq)
        self.running.extend(out)
        return out

    # -------------------------------------------------------------------------------------------- step
    def step(self) -> list[StepOutput]:
        admitted = self._admit()
        new = set(id(s) for s in admitted)
        decoding = [s for s in self.running if id(s) not in new]
        if not admitted and not decoding:
            return []
        st = self._stats
        st["steps"] += 1
        st["peak_running"] = max(st["peak_running"], len(self.running))
        target, draft = self.lanes

        # draft: prefill the newcomers; the others catch up on what they have not seen and propose k tokens
        if admitted:
            draft.greedy([(s.tables[1], s.prompt_ids) for s in admitted], last_only=True)
        proposals: list[list[int]] = [[] for _ in decoding]
        if decoding:
            firsts = draft.greedy([(s.tables[1], s.tokens[s.tables[1].num_tokens:]) for s in decoding])
            for p, f in zip(proposals, firsts):
                p.append(f[-1])
            for _ in range(self.k - 1):
                nxt = draft.greedy([(s.tables[1], [p[-1]]) for s, p in zip(decoding, proposals)])
                for p, f in zip(proposals, nxt):
                    p.append(f[0])

        # target: the newcomers' first token, and the verification of [newest token, d1 .. dk]
        outputs = []
        if admitted:
            firsts = target.greedy([(s.tables[0], s.prompt_ids) for s in admitted], last_only=True)
            for s, f in zip(admitted, firsts):
                outputs += self._emit(s, [f[-1]])
        if decoding:
            self._verifications += 1
            checks = target.greedy([(s.tables[0], s.tokens[s.tables[0].num_tokens:] + p)
                                    for s, p in zip(decoding, proposals)])
            for s, p, c in zip(decoding, proposals, checks):
                t = c[-(self.k + 1):]
                n = 0
                while n < self.k and p[n] == t[n]:
                    n += 1
                st["proposed"] += self.k
                st["accepted"] += n
                st["emitted_by_verification"] += n + 1
                outputs += self._emit(s, p[:n] + [t[n]])
        return outputs

    def _emit(self, s: SpecSeq, new_tokens: list[int]) -> list[StepOutput]:
        out = []
        for tok in new_tokens:
            s.tokens.append(tok)
            done = (tok in self._eos and not s.ignore_eos) or len(s.tokens) - s.n_prompt >= s.max_new_tokens
            out.append(StepOutput(s.seq_id, tok, done))
            if done:
                self.running.remove(s)
                self._release(s)
                return out
        # keep KV only for accepted tokens: everything but the newest is stored, rejected drafts are dropped
        keep = len(s.tokens) - 1
        for tab in s.tables:
            tab.rewind(min(tab.num_tokens, keep))
        return out

"""Continuous / static batching: which requests run in each engine step (host-side integer logic).

Semantics follow nanoserve/scheduler.py:25-200, so a step sees exactly the batch the reference would
build:

  * budget order per step: (1) every running decode, 1 token each; (2) running requests part-way through
    a chunked prefill, min(remaining, budget) tokens; (3) first-come-first-served admissions, which never
    skip the head of the queue;
  * before that, every running request reserves KV room for this step's token; if the pool is out of
    blocks, the most recently admitted request is preempted (LIFO) and recomputes prompt + outputs later;
  * policy "static" admits only between batches, once the batch is full or has waited batch_wait_s.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from enum import Enum


class SeqStatus(Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


@dataclass(eq=False)
class Sequence:
    """One request inside the engine."""
    seq_id: int
    prompt_ids: list[int]
    max_new_tokens: int
    ignore_eos: bool = False
    arrival_time: float = 0.0
    output_ids: list[int] = field(default_factory=list)
    status: SeqStatus = SeqStatus.WAITING
    cache: object | None = None        # unused by the paged path (kept for interface parity)
    block_table: object | None = None  # paged KV, set on admission
    num_cached: int = 0                # tokens whose K/V are stored; 0 => must (re)prefill
    sampling: object | None = None     # SamplingParams (None = greedy)
    seed: int = 0                      # this request's random stream

    @property
    def num_tokens(self) -> int:
        return len(self.prompt_ids) + len(self.output_ids)

    @property
    def remaining(self) -> int:
        """Known tokens whose K/V is not stored yet."""
        return self.num_tokens - self.num_cached

    @property
    def is_prefill(self) -> bool:
        """Prefilling = new, preempted (recomputing), or part-way through a chunked prefill. Decoding =
        exactly one uncached token (the newest output)."""
        return self.num_cached == 0 or self.remaining > 1

    def step_tokens(self, n: int | None = None) -> tuple[list[int], list[int]]:
        """(token ids, positions) of the next n uncached tokens (default: all of them)."""
        n = self.remaining if n is None else n
        if n == 1 and self.remaining == 1 and self.output_ids:
            return [self.output_ids[-1]], [self.num_tokens - 1]
        start = self.num_cached
        known = self.prompt_ids + self.output_ids
        return known[start:start + n], list(range(start, start + n))

    @property
    def step_cost(self) -> int:
        return self.remaining


@dataclass
class SchedulerOutput:
    scheduled: list[Sequence]   # everyone running this step, in batch order
    admitted: list[Sequence]    # the subset newly admitted this step
    chunks: list[int] = field(default_factory=list)   # tokens each scheduled sequence processes


class Scheduler:
    def __init__(self, policy: str = "continuous", max_num_seqs: int = 8, max_num_batched_tokens: int = 8192,
                 batch_wait_s: float = 0.02, kv=None, chunked_prefill: bool = False):
        if policy not in ("static", "continuous"):
            raise ValueError(f"unknown policy {policy!r}")
        self.policy = policy
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.batch_wait_s = batch_wait_s
        self.kv = kv
        self.chunked_prefill = chunked_prefill
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []
        self.num_preemptions = 0

    def add(self, seq: Sequence) -> None:
        n_prompt = len(seq.prompt_ids)
        if not self.chunked_prefill and n_prompt > self.max_num_batched_tokens:
            raise ValueError(f"prompt of {n_prompt} tokens exceeds the per-step token budget "
                             f"({self.max_num_batched_tokens}) and chunked prefill is off")
        if self.kv is not None and not self.kv.can_ever_fit(n_prompt + seq.max_new_tokens):
            raise ValueError(f"request needs up to {n_prompt + seq.max_new_tokens} tokens of KV, more than the "
                             f"whole KV budget: it could never finish")
        seq.status = SeqStatus.WAITING
        self.waiting.append(seq)

    def finish(self, seq: Sequence) -> None:
        seq.status = SeqStatus.FINISHED
        self.running.remove(seq)
        if self.kv is not None:
            self.kv.free(seq)

    def abort(self, seq: Sequence) -> None:
        """Drop a request wherever it is."""
        if seq in self.running:
            self.finish(seq)
        elif seq in self.waiting:
            self.waiting.remove(seq)
            seq.status = SeqStatus.FINISHED

    def _preempt(self, seq: Sequence) -> None:
        """Free a running request's KV, keep its outputs, put it back at the front of the queue."""
        self.running.remove(seq)
        self.kv.free(seq)
        seq.num_cached = 0
        seq.status = SeqStatus.WAITING
        self.waiting.appendleft(seq)
        self.num_preemptions += 1

    def _reserve_decode_slots(self) -> None:
        """Room for this step's token for every running request; preempt the newest while blocks run out."""
        i = 0
        while i < len(self.running):
            if self.kv.try_append(self.running[i]):
                i += 1
            else:
                self._preempt(self.running[-1])   # may be running[i] itself: the loop then moves on

    def has_unfinished(self) -> bool:
        return bool(self.waiting or self.running)

    def _may_admit(self, now: float) -> bool:
        if self.policy == "continuous":
            return True
        if self.running or not self.waiting:
            return False
        return len(self.waiting) >= self.max_num_seqs or now - self.waiting[0].arrival_time >= self.batch_wait_s

    def schedule(self, now: float) -> SchedulerOutput:
        if self.kv is not None:
            self._reserve_decode_slots()
        budget = self.max_num_batched_tokens
        scheduled: list[Sequence] = []
        chunks: list[int] = []
        partial: list[Sequence] = []
        for seq in self.running:
            if seq.is_prefill:
                partial.append(seq)
            else:
                scheduled.append(seq)
                chunks.append(1)
                budget -= 1
        for seq in partial:
            n = min(seq.remaining, budget) if self.chunked_prefill else seq.remaining
            if n > 0:
                scheduled.append(seq)
                chunks.append(n)
                budget -= n
        admitted: list[Sequence] = []
        if self._may_admit(now):
            while self.waiting and len(self.running) + len(admitted) < self.max_num_seqs:
                head = self.waiting[0]
                fits = budget > 0 if self.chunked_prefill else head.step_cost <= budget
                if not fits or (self.kv is not None and not self.kv.can_admit(head)):
                    break
                seq = self.waiting.popleft()
                if self.kv is not None:
                    self.kv.admit(seq)   # may start from cached prefix blocks: admit before sizing the chunk
                n = min(seq.step_cost, budget) if self.chunked_prefill else seq.step_cost
                budget -= n
                seq.status = SeqStatus.RUNNING
                admitted.append(seq)
                scheduled.append(seq)
                chunks.append(n)
            self.running.extend(admitted)
        return SchedulerOutput(scheduled=scheduled, admitted=admitted, chunks=chunks)

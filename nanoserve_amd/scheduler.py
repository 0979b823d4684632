"""Which requests run in each engine step (host-side integer logic).

The decisions are nanoserve/scheduler.py:25-200's, so every step schedules the batch the reference would
(pinned step by step by tests/golden/host_traces.json):

  * budget order: every running decode (1 token each), then running requests part-way through a chunked
    prefill (min(remaining, budget) tokens), then admissions first come first served -- the head of the
    queue is never skipped (scheduler.py:161-200);
  * before that, every running request reserves KV room for this step's token; when the pool runs dry the
    most recently admitted running request is preempted (LIFO) and later recomputes prompt + outputs
    (scheduler.py:128-146);
  * policy "static" admits only between batches, once the batch is full or has waited batch_wait_s.

Design (this build's own): a Sequence keeps one list of all its known token ids (prompt, then outputs),
so step inputs and prefix-cache keys slice it instead of concatenating prompt and outputs every step; a
step's plan is a StepPlan of parallel lists whose decode rows always come first, which the engine's
mixed-step graph relies on (decode rows are rows 0 .. n_decode-1 of the flattened step). With the
engine's one-step-ahead launch (LLMEngine.overlap_host), a request added between step() calls is planned
one step later than the reference would; with it off the plans are identical.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from enum import Enum


class SeqStatus(Enum):
    WAITING = "waiting"
    RUNNING = "running"
    FINISHED = "finished"


class Sequence:
    """One request inside the engine: its token ids, its KV (block table) and how much of it is stored."""

    __slots__ = ("seq_id", "tokens", "n_prompt", "max_new_tokens", "ignore_eos", "arrival_time", "status",
                 "block_table", "num_cached")

    def __init__(self, seq_id: int, prompt_ids: list[int], max_new_tokens: int, ignore_eos: bool = False,
                 arrival_time: float = 0.0):
        self.seq_id = seq_id
        self.tokens: list[int] = list(prompt_ids)     # prompt, then every generated token
        self.n_prompt = len(self.tokens)
        self.max_new_tokens = max_new_tokens
        self.ignore_eos = ignore_eos
        self.arrival_time = arrival_time
        self.status = SeqStatus.WAITING
        self.block_table = None                       # set on admission (paged KV)
        self.num_cached = 0                           # tokens whose K/V are stored; 0 -> (re)prefill

    @property
    def prompt_ids(self) -> list[int]:
        return self.tokens[:self.n_prompt]

    @property
    def output_ids(self) -> list[int]:
        return self.tokens[self.n_prompt:]

    @property
    def num_outputs(self) -> int:
        return len(self.tokens) - self.n_prompt

    @property
    def num_tokens(self) -> int:
        return len(self.tokens)

    @property
    def remaining(self) -> int:
        """Known tokens whose K/V is not stored yet."""
        return len(self.tokens) - self.num_cached

    @property
    def is_prefill(self) -> bool:
        """New, preempted (recomputing) or part-way through a chunked prefill; decoding means exactly one
        uncached token, the newest output."""
        return self.num_cached == 0 or len(self.tokens) - self.num_cached > 1

    @property
    def step_cost(self) -> int:
        return len(self.tokens) - self.num_cached

    def step_tokens(self, n: int | None = None) -> tuple[list[int], range]:
        """(token ids, positions) of the next n uncached tokens (default: all of them)."""
        a = self.num_cached
        b = len(self.tokens) if n is None else a + n
        return self.tokens[a:b], range(a, b)


@dataclass
class StepPlan:
    """One step: the sequences that run, in batch order (decode rows first), and how many tokens each
    feeds; `admitted` is the subset admitted this step."""
    scheduled: list[Sequence] = field(default_factory=list)
    chunks: list[int] = field(default_factory=list)
    admitted: list[Sequence] = field(default_factory=list)
    n_decode: int = 0


_POLICIES = ("continuous", "static")


class Scheduler:
    """Plans each step from two queues: `waiting` (FIFO, preempted requests re-enter at the front) and
    `running` (admission order, so its tail is the newest). The constructor's parameters are the reference's
    (scheduler.py:88-89); kv is the KV manager, or None for unlimited KV (host-logic tests)."""

    def __init__(self, policy: str = "continuous", max_num_seqs: int = 8, max_num_batched_tokens: int = 8192,
                 batch_wait_s: float = 0.02, kv=None, chunked_prefill: bool = False):
        if policy not in _POLICIES:
            raise ValueError(f"scheduler policy must be one of {', '.join(_POLICIES)}; got {policy!r}")
        self.policy, self.kv, self.chunked_prefill = policy, kv, chunked_prefill
        self.max_num_seqs, self.max_num_batched_tokens = max_num_seqs, max_num_batched_tokens
        self.batch_wait_s = batch_wait_s
        self.waiting: deque[Sequence] = deque()
        self.running: list[Sequence] = []
        self.num_preemptions = 0

    # ---------------------------------------------------------------------------- request lifetime
    def add(self, seq: Sequence) -> None:
        """Queue a request; reject at once one that no step could take (a prompt over the token budget when
        prompts cannot be split) or that could not finish even with the whole KV pool to itself."""
        budget = self.max_num_batched_tokens
        if seq.n_prompt > budget and not self.chunked_prefill:
            raise ValueError(f"cannot schedule a {seq.n_prompt}-token prompt: steps carry at most {budget} tokens "
                             "and prompts are not split (chunked_prefill=False)")
        need = seq.n_prompt + seq.max_new_tokens
        if self.kv is not None and not self.kv.can_ever_fit(need):
            raise ValueError(f"cannot schedule a request that may reach {need} tokens: the KV pool holds fewer, "
                             "so it could never finish")
        seq.status = SeqStatus.WAITING
        self.waiting.append(seq)

    def finish(self, seq: Sequence) -> None:
        seq.status = SeqStatus.FINISHED
        self.running.remove(seq)
        if self.kv is not None:
            self.kv.free(seq)

    def abort(self, seq: Sequence) -> None:
        """Drop a request wherever it is (client went away)."""
        if seq.status is SeqStatus.RUNNING and seq in self.running:
            self.finish(seq)
        elif seq in self.waiting:
            self.waiting.remove(seq)
            seq.status = SeqStatus.FINISHED

    def has_unfinished(self) -> bool:
        return bool(self.waiting) or bool(self.running)

    # ------------------------------------------------------------------------------------ planning
    def _evict_newest(self) -> None:
        """Recompute-preemption of the most recently admitted running request: its KV is freed, its outputs
        kept, and it waits at the head of the queue."""
        victim = self.running.pop()
        self.kv.free(victim)
        victim.num_cached = 0
        victim.status = SeqStatus.WAITING
        self.waiting.appendleft(victim)
        self.num_preemptions += 1

    def _grow_running(self) -> None:
        """Room for this step's token for every running request, evicting from the back as needed."""
        i = 0
        while i < len(self.running):
            if self.kv.try_append(self.running[i]):
                i += 1
            else:
                self._evict_newest()   # possibly running[i] itself: then i == len(running) and the loop ends

    def _admission_open(self, now: float) -> bool:
        """Continuous batching admits every step. Static batching forms a batch only once the previous one has
        drained, and only when a full batch is queued or its oldest request has waited batch_wait_s."""
        if self.policy != "static":
            return True
        idle = not self.running and bool(self.waiting)
        full = len(self.waiting) >= self.max_num_seqs
        return idle and (full or now - self.waiting[0].arrival_time >= self.batch_wait_s)

    def _head_fits(self, budget: int, n_admitted: int) -> bool:
        if not self.waiting or len(self.running) + n_admitted >= self.max_num_seqs:
            return False
        head = self.waiting[0]
        if not (budget > 0 if self.chunked_prefill else head.step_cost <= budget):
            return False
        return self.kv is None or self.kv.can_admit(head)

    def schedule(self, now: float) -> StepPlan:
        if self.kv is not None:
            self._grow_running()
        plan = StepPlan()
        budget = self.max_num_batched_tokens
        partial = []
        for seq in self.running:                       # (1) decodes, one token each, always
            if seq.is_prefill:
                partial.append(seq)
            else:
                plan.scheduled.append(seq)
                plan.chunks.append(1)
                budget -= 1
        plan.n_decode = len(plan.scheduled)
        for seq in partial:                            # (2) chunked prefills already under way
            n = min(seq.remaining, budget) if self.chunked_prefill else seq.remaining
            if n > 0:
                plan.scheduled.append(seq)
                plan.chunks.append(n)
                budget -= n
        if self._admission_open(now):                  # (3) admissions, first come first served
            while self._head_fits(budget, len(plan.admitted)):
                seq = self.waiting.popleft()
                if self.kv is not None:
                    self.kv.admit(seq)                 # may start from cached prefix blocks
                n = min(seq.step_cost, budget) if self.chunked_prefill else seq.step_cost
                budget -= n
                seq.status = SeqStatus.RUNNING
                plan.admitted.append(seq)
                plan.scheduled.append(seq)
                plan.chunks.append(n)
            self.running.extend(plan.admitted)
        return plan

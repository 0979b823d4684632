"""hipGraph capture of the decode step (torch.cuda.CUDAGraph records hipGraphs on ROCm).

Contract of nanoserve/cuda_graphs.py:42-126 (DecodeGraphRunner):
  * batch buckets 1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128; a batch of n replays the smallest bucket >= n;
  * padding rows use token 0, slot garbage_block * block_size, table row [garbage_block, 0, ...] and
    ctx 1, so they write and read only the block reserved at start-up (the first block handed out);
  * inputs are overwritten in static buffers before each replay; the logits view stays valid until the
    bucket's next replay.

Design (this build's own): every bucket is a StepGraph -- one packed device buffer holding all of a step's
inputs (tokens, positions, slots int64 [B]; context lengths int32 [B]; block tables int32 [B, W]) with TWO
pinned host twins, so a step is staged by numpy writes into the twin the previous step's copy is not
reading and arrives in ONE host-to-device copy; the captured forward ends in the HIP argmax, which writes
the greedy tokens straight into pinned host memory (no device-to-host copy after the replay). A table row
is staged incrementally: block lists only grow between steps (truncation and release rebind them), so a
row staged from the same list needs only its new tail. The next step can be staged while the current one
runs (prestage / launch_prestaged), which the engine uses for steady greedy decode. Captures share one
side stream; a runner's graphs share one memory pool.
"""
from __future__ import annotations

import math

import torch

from nanoserve_amd.kv_cache import PagedKVCache
from nanoserve_amd.model import DecodeMeta, Qwen2Model, SeqInput

BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128)


_SIDE: torch.cuda.Stream | None = None


def _side_stream() -> torch.cuda.Stream:
    """One warm-up stream for every capture in the process (default priority)."""
    global _SIDE
    if _SIDE is None:
        _SIDE = torch.cuda.Stream()
    return _SIDE


def capture(fn, pool):
    """Warm fn up twice on the side stream, then record it into a graph drawing on memory pool `pool`;
    returns (graph, fn's output). Capture always begins outside inference mode (fn may enter it): the
    graph-safe RNG state torch registers at the first capture is then an ordinary tensor, which later
    captures and replays may update whether or not they run under inference mode."""
    side = _side_stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.inference_mode(False), torch.cuda.graph(graph, pool=pool):
        out = fn()
    return graph, out


class StepGraph:
    """One decode bucket: packed static inputs, two pinned twins, the captured step and its outputs."""

    def __init__(self, runner: "DecodeGraphRunner", B: int):
        self.B, self.W = B, runner.max_blocks
        self.garbage_slot = runner.garbage_block * runner.block_size
        self.garbage_block = runner.garbage_block
        nbytes = 28 * B + 4 * B * self.W
        dev = runner.model.device
        self.dev_buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        self.twins = [torch.zeros(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self.np = [self._views(t, numpy=True) for t in self.twins]
        self.staged_rows: list[list] = [[None] * B for _ in range(2)]
        self.greedy = torch.empty(B, dtype=torch.int64, pin_memory=True)
        self.par = 1                                  # twin of the last staged step
        for v in self.np:
            self._pad(v, 0)
        self.dev_buf.copy_(self.twins[0])
        tok, pos, slots, lens, tables = self._views(self.dev_buf)
        meta = DecodeMeta(runner.token_idx[:B], tables, lens, all_rows=True)
        seqs = [SeqInput(1, ctx_len=1, use_kernel=True)] * B

        def forward():
            from nanoserve_amd.kernels.sampling import argmax_rows
            logits = runner.model.forward_batch(tok, pos, seqs, logits="all", paged=runner.pool,
                                                slot_mapping=slots, decode_meta=meta)
            argmax_rows(logits, self.greedy)
            return logits

        # warm-up and capture run on padding rows only: they read and write nothing but the garbage block
        self.graph, self.logits = capture(forward, runner.mempool)

    def _views(self, buf: torch.Tensor, numpy: bool = False):
        """tokens, positions, slots (int64 [B]); context lengths (int32 [B]); tables (int32 [B, W])."""
        B = self.B
        o = (0, 8 * B, 16 * B, 24 * B, 28 * B)
        v = (buf[o[0]:o[1]].view(torch.int64), buf[o[1]:o[2]].view(torch.int64), buf[o[2]:o[3]].view(torch.int64),
             buf[o[3]:o[4]].view(torch.int32), buf[o[4]:].view(torch.int32).view(B, self.W))
        return tuple(x.numpy() for x in v) if numpy else v

    def _pad(self, views, lo: int) -> None:
        tok, pos, slots, lens, tables = views
        tok[lo:] = 0
        pos[lo:] = 0
        slots[lo:] = self.garbage_slot
        lens[lo:] = 1
        tables[lo:] = 0
        tables[lo:, 0] = self.garbage_block

    def stage(self, par: int, tokens, positions, slots, tables, lens) -> None:
        """Write a step into pinned twin `par` (tokens None: left for later)."""
        n = len(positions)
        tok, pos, sl, ln, tb = self.np[par]
        if tokens is not None:
            tok[:n] = tokens
        pos[:n] = positions
        sl[:n] = slots
        ln[:n] = lens
        rows = self.staged_rows[par]
        for i, t in enumerate(tables):
            L = len(t)
            if L > self.W:
                raise ValueError(f"block table of {L} blocks exceeds the graph width {self.W} (max_seq_len)")
            prev = rows[i]
            if prev is not None and prev[0] is t and prev[1] <= L:
                if prev[1] < L:
                    tb[i, prev[1]:L] = t[prev[1]:L]
            else:
                tb[i, :L] = t
                tb[i, L:] = 0
            rows[i] = (t, L)
        for i in range(n, self.B):
            rows[i] = None
        self._pad(self.np[par], n)

    def launch(self, par: int) -> None:
        self.par = par
        self.dev_buf.copy_(self.twins[par], non_blocking=True)
        self.graph.replay()


class DecodeGraphRunner:
    def __init__(self, model: Qwen2Model, pool: PagedKVCache, max_seq_len: int, max_batch: int = BUCKETS[-1]):
        self.model, self.pool = model, pool
        self.block_size = pool.block_size
        self.buckets = [b for b in BUCKETS if b <= max_batch]
        self.max_bucket = self.buckets[-1]
        self.max_blocks = math.ceil(max_seq_len / pool.block_size)
        self.garbage_block = pool.allocator.allocate()
        self.token_idx = torch.arange(self.max_bucket, device=model.device)
        self.graphs: dict[int, StepGraph] = {}
        self._pending: tuple[StepGraph, int, int] | None = None    # prestaged step: (graph, twin, rows)
        self.last: StepGraph | None = None
        self.mempool = torch.cuda.graph_pool_handle()                 # shared by this runner's graphs

    @property
    def captured_buckets(self) -> list[int]:
        return sorted(self.graphs)

    def bucket_for(self, n: int) -> int | None:
        for b in self.buckets:
            if b >= n:
                return b
        return None

    def _graph(self, n: int) -> StepGraph:
        B = self.bucket_for(n)
        if B is None:
            raise ValueError(f"batch of {n} exceeds the largest graph bucket ({self.max_bucket})")
        g = self.graphs.get(B)
        if g is None:
            g = self.graphs[B] = StepGraph(self, B)
        return g

    def has_graph_for(self, n: int) -> bool:
        B = self.bucket_for(n)
        return B is not None and B in self.graphs

    def capture_all(self, max_batch: int) -> None:
        """Capture every bucket a batch of up to max_batch requests can use."""
        top = self.bucket_for(min(max_batch, self.max_bucket))
        for B in self.buckets:
            if B <= top:
                self._graph(B)

    def run(self, tokens: list[int], positions: list[int], slots: list[int], block_tables: list[list[int]],
            context_lens: list[int]) -> torch.Tensor:
        """One decode step of n requests through the bucket's graph; logits [n, vocab] (a view of the graph's
        output, valid until the bucket's next replay). The greedy tokens are in greedy_tokens(n)."""
        g = self._graph(len(tokens))
        par = g.par ^ 1
        torch.cuda.current_stream().synchronize()   # the twin about to be rewritten may still be copying
        g.stage(par, tokens, positions, slots, block_tables, context_lens)
        g.launch(par)
        self.last = g
        return g.logits[:len(tokens)]

    def prestage(self, positions: list[int], slots: list[int], block_tables: list[list[int]],
                 context_lens: list[int]) -> None:
        """Stage the next step except its tokens (not known until the running step ends) into the twin the
        running step's copy is not reading; launch_prestaged() completes and launches it."""
        g = self._graph(len(positions))
        par = g.par ^ 1
        g.stage(par, None, positions, slots, block_tables, context_lens)
        self._pending = (g, par, len(positions))

    def launch_prestaged(self, tokens: list[int]) -> torch.Tensor:
        g, par, n = self._pending
        self._pending = None
        if len(tokens) != n:
            raise ValueError(f"{len(tokens)} tokens for a prestaged step of {n} rows")
        g.np[par][0][:n] = tokens
        g.launch(par)
        self.last = g
        return g.logits[:n]

    def greedy_tokens(self, n: int) -> list[int]:
        """Argmax of the first n rows of the last replay (written into pinned memory inside the graph):
        waits for the replay, then reads the host buffer."""
        torch.cuda.current_stream().synchronize()
        return self.last.greedy[:n].tolist()

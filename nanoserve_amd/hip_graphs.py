"""hipGraph capture of the decode step and of mixed steps (torch.cuda.CUDAGraph records hipGraphs on ROCm).

Contract of nanoserve/cuda_graphs.py:42-126 (DecodeGraphRunner):
  * batch buckets 1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128; a batch of n replays the smallest bucket >= n;
  * padding rows use token 0, slot garbage_block * block_size, table row [garbage_block, 0, ...] and
    ctx 1, so they write and read only the block reserved at start-up (the first block handed out);
  * inputs are overwritten in static buffers before each replay; the logits view stays valid until the
    bucket's next replay.

Design (this build's own): every bucket is a StepGraph -- one packed device buffer holding all of a step's
inputs (tokens, positions, slots int64 [B]; context lengths int32 [B]; block tables int32 [B, W]) with TWO
pinned host twins, so a step is staged by numpy writes into the twin the previous step's copy is not
reading and arrives in ONE host-to-device copy; the captured forward ends in the LM head with the argmax
fused (one launch), which writes the greedy tokens straight into pinned host memory (no device-to-host copy
after the replay). A table row
is staged incrementally: block lists only grow between steps (truncation and release rebind them), so a
row staged from the same list needs only its new tail. The next step can be staged while the current one
runs (prestage / launch_prestaged), which the engine uses for steady greedy decode. Captures share one
side stream; a runner's graphs share one memory pool.

Mixed steps (prefill chunks + decode rows; the role of nanoserve/cuda_graphs.py:151-259, PiecewiseGraphRunner,
in this build's own design): the whole step is one graph, attention included -- the chunked-prefill kernel
reads the pages in place, so nothing has to run eagerly between pieces. A MixedStepGraph is keyed by a row
bucket N (a multiple of 128, the tiled GEMM's row tile) and by the prefill-sequence capacity S (1, 2, 4, 8);
it holds N + 1 rows, the last always padding. Its packed static inputs: token ids, positions and slots of
every row; the prefill kernel's seq_info [S, 4] and tables [S, W]; the decode rows' indices, tables and
context lengths [D] (D = the runner's decode capacity); and the rows whose logits are wanted (each
sequence's last token). Unused prefill entries have no new tokens (their workgroups exit at once), unused
decode entries attend over the garbage block from the padding row, and padding rows write their K/V into
the garbage block. The greedy tokens go into pinned host memory inside the graph, as in the decode graph.
A runner made with capture=False stages the same padded rows and runs the same forward without recording
it, so an engine without graphs computes its mixed steps exactly as one with them (the kernels' tilings and
K slices depend on the row count, so an unpadded step may round differently). Steps above the graph bound are
never recorded by either, so they run tight: their n rows plus one padding row (at index n), not the bucket's
N + 1, which saves the GEMM work of up to 127 padding rows.
"""
from __future__ import annotations

import gc
import itertools
import math
import struct
import time

import numpy as np
import torch

from nanoserve_amd.kernels.paged_attention import pair_rows
from nanoserve_amd.kv_cache import PagedKVCache
from nanoserve_amd.model import DecodeMeta, Qwen2Model, SeqInput

BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128)
POLL_S = 0.05   # longest host poll for a decode replay's tokens before a stream synchronisation


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
    captures and replays may update whether or not they run under inference mode. Python's cyclic garbage
    collector is run first and held off while recording: graphs are captured mid-run, and a collection
    inside the capture would free earlier graphs' pinned buffers, which a stream capture does not allow."""
    side = _side_stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
        fn()
    torch.cuda.current_stream().wait_stream(side)
    gc.collect()
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        graph = torch.cuda.CUDAGraph()
        with torch.inference_mode(False), torch.cuda.graph(graph, pool=pool):
            out = fn()
    finally:
        if was_enabled:
            gc.enable()
    return graph, out


class StepGraph:
    """One decode bucket: packed static inputs, two pinned twins, the captured step and its outputs."""

    def __init__(self, runner: "DecodeGraphRunner", B: int):
        self.B, self.W = B, runner.max_blocks
        self.garbage_slot = runner.garbage_block * runner.block_size
        self.garbage_block = runner.garbage_block
        nbytes = 32 * B + 4 * B * self.W
        dev = runner.model.device
        self.dev_buf = torch.zeros(nbytes, dtype=torch.uint8, device=dev)
        self.twins = [torch.zeros(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self.np = [self._views(t, numpy=True) for t in self.twins]
        self.staged_rows: list[list] = [[None] * B for _ in range(2)]
        self.greedy = torch.empty(B, dtype=torch.int64, pin_memory=True)
        self.greedy_np = self.greedy.numpy()
        self.par = 1                                  # twin of the last staged step
        for v in self.np:
            self._pad(v, 0)
        self.dev_buf.copy_(self.twins[0])
        tok, pos, slots, lens, pairs, tables = self._views(self.dev_buf)
        # the row pairing only where rows can share a table (speculative verification): the paired attention
        # kernel costs a plain decode step ~0.4 us per layer
        self.pairing = runner.pair_rows
        meta = DecodeMeta(runner.token_idx[:B], tables, lens, all_rows=True, pairs=pairs if self.pairing else None)
        seqs = [SeqInput(1, ctx_len=1, use_kernel=True)] * B

        def forward():
            return runner.model.forward_batch(tok, pos, seqs, logits="all", paged=runner.pool, slot_mapping=slots,
                                              decode_meta=meta, greedy_out=self.greedy)

        # warm-up and capture run on padding rows only: they read and write nothing but the garbage block
        self.graph, self.logits = capture(forward, runner.mempool)

    def _views(self, buf: torch.Tensor, numpy: bool = False):
        """tokens, positions, slots (int64 [B]); context lengths, row pairing (int32 [B]); tables (int32 [B, W])."""
        B = self.B
        o = (0, 8 * B, 16 * B, 24 * B, 28 * B, 32 * B)
        v = (buf[o[0]:o[1]].view(torch.int64), buf[o[1]:o[2]].view(torch.int64), buf[o[2]:o[3]].view(torch.int64),
             buf[o[3]:o[4]].view(torch.int32), buf[o[4]:o[5]].view(torch.int32),
             buf[o[5]:].view(torch.int32).view(B, self.W))
        return tuple(x.numpy() for x in v) if numpy else v

    def _pad(self, views, lo: int) -> None:
        tok, pos, slots, lens, pairs, tables = views
        pairs[lo:] = 0
        tok[lo:] = 0
        pos[lo:] = 0
        slots[lo:] = self.garbage_slot
        lens[lo:] = 1
        tables[lo:] = 0
        tables[lo:, 0] = self.garbage_block

    def stage(self, par: int, tokens, positions, slots, tables, lens) -> None:
        """Write a step into pinned twin `par` (tokens None: left for later)."""
        n = len(positions)
        tok, pos, sl, ln, pr, tb = self.np[par]
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
        if self.pairing:
            pair_rows(tables, pr)   # rows of one sequence (speculative verification) share its table
        self._pad(self.np[par], n)

    def launch(self, par: int) -> None:
        self.par = par
        self.greedy_np.fill(-1)                       # no token yet: the replay's argmax overwrites every row
        self.dev_buf.copy_(self.twins[par], non_blocking=True)
        self.graph.replay()


class DecodeGraphRunner:
    def __init__(self, model: Qwen2Model, pool: PagedKVCache, max_seq_len: int, max_batch: int = BUCKETS[-1],
                 pair_rows: bool = False):
        """pair_rows: stage the row pairing (rows that share a block table run as one attention workgroup
        row) -- for speculative verification, whose rows of one sequence share its table."""
        self.model, self.pool = model, pool
        self.pair_rows = pair_rows
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
        self.captured_up_front = False
        self.captures_in_run = 0    # buckets captured by a step after capture_all (a step paid for a capture)

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
            self.captures_in_run += self.captured_up_front
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
        self.captured_up_front = True

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
        """Argmax of the first n rows of the last replay. The graph's last kernel (the LM head with the argmax)
        stores each row's token once, as one 8-byte store, into pinned host memory that launch() filled with
        -1; the host polls that memory instead of waiting for the stream, so it sees the tokens as soon as
        they land. A value outside [0, vocab) is not a token yet. After POLL_S without every row the wait
        falls back to a stream synchronisation."""
        buf = self.last.greedy_np[:n]
        vocab = self.model.cfg.vocab_size
        deadline = time.perf_counter() + POLL_S
        while not ((buf >= 0) & (buf < vocab)).all():
            if time.perf_counter() > deadline:
                torch.cuda.current_stream().synchronize()
                break
        return buf.tolist()


MIXED_ROW_STEP = 128
MIXED_SEQ_BUCKETS = (1, 2, 4, 8)


class MixedStepGraph:
    """One mixed-step bucket: N + 1 rows, S prefill entries, D decode entries (see the module docstring)."""

    def __init__(self, runner: "MixedGraphRunner", N: int, S: int, record: bool, tight: bool = False):
        self.N, self.S, self.D, self.W = N, S, runner.max_decode, runner.max_blocks
        self.tight = tight and not record   # unrecorded, sized per step: n rows + padding row n
        self.rows_run = N + 1
        R, D, W = N + 1, self.D, self.W
        self.garbage_block = runner.garbage_block
        self.garbage_slot = runner.garbage_block * runner.block_size
        # int64 section: tokens, positions, slots [R]; decode row index [D]; logit rows [S + D]
        # int32 section: seq_info [S, 4]; decode context lengths [D]; prefill tables [S, W]; decode tables [D, W]
        n64 = 3 * R + D + (S + D)
        n32 = 4 * S + D + S * W + D * W
        self.nbytes = 8 * n64 + 4 * n32
        dev = runner.model.device
        self.dev_buf = torch.zeros(self.nbytes, dtype=torch.uint8, device=dev)
        self.twins = [torch.zeros(self.nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        self.np = [self._views(t, numpy=True) for t in self.twins]
        self.greedy = torch.empty(S + D, dtype=torch.int64, pin_memory=True)
        self.par = 1
        for v in self.np:
            self._pad_all(v)
        self.dev_buf.copy_(self.twins[0])
        tok, pos, slots, dec_idx, rows, info, dec_lens, pf_tab, dec_tab = self._views(self.dev_buf)
        meta = DecodeMeta(dec_idx, dec_tab, dec_lens)
        # a sequence's new tokens fit both the rows and its table
        prefill = ("chunks", pf_tab, info, min(N, W * runner.block_size), W * runner.block_size)

        def forward(r: int = R):
            return runner.model.forward_batch(tok[:r], pos[:r], [SeqInput(r)], logits=rows, paged=runner.pool,
                                              slot_mapping=slots[:r], decode_meta=meta, prefill_meta=prefill,
                                              greedy_out=self.greedy)

        self.forward = forward
        self.graph, self.logits = None, None
        if record:
            # warm-up and capture run on padding only: no new prefill tokens, decode entries on the garbage block
            self.graph, self.logits = capture(forward, runner.mempool)

    @property
    def host_bytes(self) -> int:
        return 2 * self.nbytes + self.greedy.numel() * 8

    def _views(self, buf: torch.Tensor, numpy: bool = False):
        R, S, D, W = self.N + 1, self.S, self.D, self.W
        o, out = 0, []
        for n in (R, R, R, D, S + D):
            out.append(buf[o:o + 8 * n].view(torch.int64))
            o += 8 * n
        for shape in ((S, 4), (D,), (S, W), (D, W)):
            n = 1
            for d in shape:
                n *= d
            out.append(buf[o:o + 4 * n].view(torch.int32).view(*shape))
            o += 4 * n
        return tuple(x.numpy() for x in out) if numpy else tuple(out)

    def _pad_all(self, v) -> None:
        tok, pos, slots, dec_idx, rows, info, dec_lens, pf_tab, dec_tab = v
        tok[:] = 0
        pos[:] = 0
        slots[:] = self.garbage_slot
        dec_idx[:] = self.N
        rows[:] = self.N
        info[:] = 0
        dec_lens[:] = 1
        pf_tab[:] = 0
        dec_tab[:] = 0
        dec_tab[:, 0] = self.garbage_block

    def stage(self, par: int, sb) -> None:
        """Write StepBatch sb into pinned twin `par` (everything past its rows and entries is padding)."""
        v = self.np[par]
        self._pad_all(v)
        tok, pos, slots, dec_idx, rows, info, dec_lens, pf_tab, dec_tab = v
        n = len(sb.token_ids)
        _put_int64(tok, sb.token_ids)
        _put_int64(pos, sb.positions)
        _put_int64(slots, sb.slots)
        start, j = 0, 0
        for i, s in enumerate(sb.seqs):
            T = s.n_tokens
            rows[i] = start + T - 1
            if not s.use_kernel:
                t = sb.tables[i]
                info[j] = (start, T, s.ctx_len, 0)
                pf_tab[j, :len(t)] = t
                j += 1
            start += T
        nd = len(sb.dec_idx)
        dec_idx[:nd] = sb.dec_idx
        dec_lens[:nd] = sb.dec_lens
        if nd:   # the decode rows' tables through one conversion (zeros past each table's end)
            dec_tab[:nd] = 0
            flat = np.frombuffer(struct.pack(f"{sum(len(t) for t in sb.dec_tables)}i",
                                             *itertools.chain.from_iterable(sb.dec_tables)), dtype=np.int32)
            o = 0
            for i, t in enumerate(sb.dec_tables):
                dec_tab[i, :len(t)] = flat[o:o + len(t)]
                o += len(t)
        self.rows_run = self.N + 1
        if self.tight:   # the padding row is row n: unused decode entries and logit rows point there
            dec_idx[nd:] = n
            rows[len(sb.seqs):] = n
            self.rows_run = n + 1

    def launch(self, par: int) -> None:
        self.par = par
        self.dev_buf.copy_(self.twins[par], non_blocking=True)
        if self.graph is not None:
            self.graph.replay()
        else:
            self.logits = self.forward(self.rows_run)


def _put_int64(dst, values) -> None:
    """values (Python ints) into the head of the int64 array dst. A long list goes through one struct.pack (about
    12 ns per value against 28 for numpy's list assignment, token-sized values; a 1552-row step stages three
    such lists)."""
    n = len(values)
    if n > 64 and isinstance(values, list):
        dst[:n] = np.frombuffer(struct.pack(f"{n}q", *values), dtype=np.int64)
    else:
        dst[:n] = values


MIXED_GRAPH_MAX_ROWS = 512   # default bound: mixed steps of more rows run staged, unrecorded (launches are a
                             # small share of a step that size)


class MixedGraphRunner:
    """Mixed-step graphs of one model and pool. The recorded set is bounded: row buckets up to
    max_graph_rows times the prefill capacities a step of at most max_decode sequences can need
    (graph_keys); capture_all records all of them up front (largest first, so the smaller ones reuse the shared
    pool's segments), a key of that set met before capture_all is recorded on first use, and bigger steps run
    the same staged forward without a graph, on their own rows plus one padding row. With capture=False
    nothing is recorded (steps up to max_graph_rows still run their whole padded bucket)."""

    def __init__(self, model: Qwen2Model, pool: PagedKVCache, max_seq_len: int, max_decode: int,
                 max_rows: int, garbage_block: int, capture: bool = True, max_graph_rows: int = MIXED_GRAPH_MAX_ROWS):
        self.model, self.pool = model, pool
        self.capture = capture
        self.max_graph_rows = max_graph_rows
        self.block_size = pool.block_size
        self.max_blocks = math.ceil(max_seq_len / pool.block_size)
        self.max_decode = max_decode
        self.max_rows = max_rows
        self.garbage_block = garbage_block
        self.graphs: dict[tuple[int, int], MixedStepGraph] = {}    # recorded
        self.staged: dict[tuple[int, int], MixedStepGraph] = {}    # run unrecorded
        self.mempool = torch.cuda.graph_pool_handle()
        self.last: MixedStepGraph | None = None
        self.captured_up_front = False
        self.captures_in_run = 0
        self.device_bytes = 0    # device memory the recorded graphs took (pool segments and input buffers)

    @staticmethod
    def bucket(n_rows: int) -> int:
        return max(MIXED_ROW_STEP, -(-n_rows // MIXED_ROW_STEP) * MIXED_ROW_STEP)

    def graph_keys(self) -> list[tuple[int, int]]:
        """The (row bucket, prefill capacity) pairs this runner records, smallest first."""
        top_rows = min(self.bucket(self.max_rows), self.max_graph_rows)
        top_seqs = next(s for s in MIXED_SEQ_BUCKETS if s >= min(self.max_decode, MIXED_SEQ_BUCKETS[-1]))
        return [(n, s) for n in range(MIXED_ROW_STEP, top_rows + 1, MIXED_ROW_STEP)
                for s in MIXED_SEQ_BUCKETS if s <= top_seqs]

    @property
    def host_bytes(self) -> int:
        """Pinned host memory of the recorded graphs' input twins and token outputs."""
        return sum(g.host_bytes for g in self.graphs.values())

    def _record(self, key: tuple[int, int]) -> MixedStepGraph:
        before = torch.cuda.memory_reserved(self.model.device)
        g = self.graphs[key] = MixedStepGraph(self, *key, record=True)
        self.device_bytes += torch.cuda.memory_reserved(self.model.device) - before
        return g

    def capture_all(self) -> None:
        """Record every key of graph_keys() not recorded yet (no-op with capture=False)."""
        if self.capture:
            for key in reversed(self.graph_keys()):
                if key not in self.graphs:
                    self._record(key)
            self.captured_up_front = True

    def fits(self, sb) -> bool:
        n_pf = len(sb.seqs) - len(sb.dec_idx)
        return (self.model.dtype == torch.bfloat16 and 0 < n_pf <= MIXED_SEQ_BUCKETS[-1]
                and len(sb.token_ids) <= self.max_rows and len(sb.dec_idx) <= self.max_decode
                and all(len(t) <= self.max_blocks for t in sb.tables))

    def run(self, sb) -> torch.Tensor:
        n_pf = len(sb.seqs) - len(sb.dec_idx)
        key = (self.bucket(len(sb.token_ids)), next(s for s in MIXED_SEQ_BUCKETS if s >= n_pf))
        g = self.graphs.get(key) or self.staged.get(key)
        if g is None:
            if self.capture and key[0] <= self.max_graph_rows:
                g = self._record(key)
                self.captures_in_run += self.captured_up_front
            else:
                g = self.staged[key] = MixedStepGraph(self, *key, record=False, tight=key[0] > self.max_graph_rows)
        par = g.par ^ 1
        torch.cuda.current_stream().synchronize()   # the twin about to be rewritten may still be copying
        g.stage(par, sb)
        g.launch(par)
        self.last = g
        return g.logits[:len(sb.seqs)]

    def greedy_tokens(self, n: int) -> list[int]:
        torch.cuda.current_stream().synchronize()
        return self.last.greedy[:n].tolist()

"""hipGraph runners for the decode loop (torch.cuda.CUDAGraph records hipGraphs on ROCm).

DecodeGraphRunner — one graph per batch bucket for pure-decode steps; contract of
nanoserve/cuda_graphs.py:42-126:
  * buckets (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128); a batch of n replays the smallest bucket >= n;
  * inputs live in static device buffers overwritten before each replay (tokens, positions, slots int64;
    block tables int32 [B, W]; context lengths int32), W = ceil(max_seq_len / block_size); here each bucket
    packs them into one buffer with a pinned host twin, so staging a step is one H2D copy;
  * padding rows use token 0, slot garbage_block * block_size, table row [garbage_block, 0, ...] and
    ctx 1: they write and read only the reserved garbage block;
  * capture is lazy (first use of a bucket) after two eager warm-ups on a shared side stream, and every
    graph shares one memory pool; run() returns a view of the graph's logits, valid until the next replay.
Every capture and replay runs under torch.inference_mode (as forward_batch does): the graph-safe RNG
state torch registers at capture must be created and updated in one mode. All HIP kernels take the
capture stream from torch and allocate nothing, so the whole step — embedding,
28 layers of GEMMs / fused ops / split-K attention, final norm and LM head — is one graph launch.

PiecewiseGraphRunner — mixed prefill + decode steps (nanoserve/cuda_graphs.py:151-259): per token
bucket, L+1 graph pieces (embed + layer 0 _pre; layer j-1 _post + layer j _pre; last _post + final
norm) with attention run eagerly between them through the same HIP kernels.
"""
from __future__ import annotations

import math

import torch

from nanoserve_amd.kv_cache import PagedKVCache
from nanoserve_amd.model import DecodeMeta, Qwen2Model, SeqInput

BUCKETS = (1, 2, 4, 8, 16, 24, 32, 48, 64, 96, 128)

_SIDE_STREAM = None


def _capture_stream() -> torch.cuda.Stream:
    """One warm-up stream for every capture in the process (default priority)."""
    global _SIDE_STREAM
    if _SIDE_STREAM is None:
        _SIDE_STREAM = torch.cuda.Stream()
    return _SIDE_STREAM


class DecodeGraphRunner:
    def __init__(self, model: Qwen2Model, pool: PagedKVCache, max_seq_len: int, max_batch: int = BUCKETS[-1]):
        self.model, self.pool = model, pool
        self.buckets = [b for b in BUCKETS if b <= max_batch]
        self.max_bucket = self.buckets[-1]
        self.max_blocks = math.ceil(max_seq_len / pool.block_size)
        self.garbage_block = pool.allocator.allocate()
        dev, mb = model.device, self.max_bucket
        self.token_idx = torch.arange(mb, device=dev)
        self.inputs: dict[int, tuple] = {}     # bucket -> (device buffer, pinned twin, device views, host views)
        self.graphs: dict[int, torch.cuda.CUDAGraph] = {}
        self.outputs: dict[int, torch.Tensor] = {}
        self._np: dict[tuple, tuple] = {}              # numpy views of the pinned host inputs
        self._staged_rows: dict[tuple, list] = {}      # per (bucket, buffer) row: (block list, entries staged)
        self._host2: dict[int, torch.Tensor] = {}      # second pinned host buffer per bucket
        self._par: dict[int, int] = {}                 # host buffer of the bucket's last staged step
        self._pending = None                           # (bucket, buffer, rows) of a prestaged step
        # in-graph argmax of each row's logits (int64), written by the kernel straight into pinned host
        # memory: reading it after the step's synchronisation needs no device-to-host copy
        self.greedy: dict[int, torch.Tensor] = {}
        self.mempool = None

    @property
    def captured_buckets(self) -> list[int]:
        return sorted(self.graphs)

    def _views(self, buf: torch.Tensor, B: int):
        """tokens, positions, slots (int64 [B]); context lengths (int32 [B]); block tables (int32 [B, W])."""
        o1, o2, o3, o4 = 8 * B, 16 * B, 24 * B, 28 * B
        return (buf[0:o1].view(torch.int64), buf[o1:o2].view(torch.int64), buf[o2:o3].view(torch.int64),
                buf[o3:o4].view(torch.int32), buf[o4:].view(torch.int32).view(B, self.max_blocks))

    def _buffers(self, B: int) -> tuple:
        """Bucket B's static inputs: one packed device buffer with a pinned host twin, so a step's inputs
        arrive in a single H2D copy of 28 B + 4 B W bytes."""
        if B not in self.inputs:
            n = 28 * B + 4 * B * self.max_blocks
            dev = torch.zeros(n, dtype=torch.uint8, device=self.model.device)
            host = torch.zeros(n, dtype=torch.uint8, pin_memory=True)
            self.inputs[B] = (dev, host, self._views(dev, B), self._views(host, B))
        return self.inputs[B]

    def bucket_for(self, n: int) -> int | None:
        return next((b for b in self.buckets if b >= n), None)

    def _fill_padding(self, views, lo: int) -> None:
        """Rows lo.. of the (host) views become padding rows."""
        tokens, positions, slots, lens, tables = views
        tokens[lo:] = 0
        positions[lo:] = 0
        slots[lo:] = self.garbage_block * self.pool.block_size
        lens[lo:] = 1
        tables[lo:] = 0
        tables[lo:, 0] = self.garbage_block

    def _reset_to_padding(self, B: int) -> None:
        dev, host, _, hv = self._buffers(B)
        self._fill_padding(hv, 0)
        self._staged_rows[(B, 0)] = [None] * B
        dev.copy_(host)

    def _host_buf(self, B: int, par: int) -> torch.Tensor:
        """Pinned host buffer `par` (0 or 1) of bucket B."""
        if par == 0:
            return self._buffers(B)[1]
        if B not in self._host2:
            self._host2[B] = torch.zeros_like(self._buffers(B)[1], pin_memory=True)
            self._fill_padding(self._views(self._host2[B], B), 0)
        return self._host2[B]

    def _host_np(self, B: int, par: int = 0) -> tuple:
        """numpy views of bucket B's pinned host buffer `par` (list assignment into them skips torch.tensor)."""
        if (B, par) not in self._np:
            self._np[(B, par)] = tuple(v.numpy() for v in self._views(self._host_buf(B, par), B))
            self._staged_rows.setdefault((B, par), [None] * B)
        return self._np[(B, par)]

    def _forward(self, B: int) -> tuple[torch.Tensor, torch.Tensor]:
        from nanoserve_amd.kernels.sampling import argmax_rows
        tokens, positions, slots, lens, tables = self._buffers(B)[2]
        meta = DecodeMeta(self.token_idx[:B], tables, lens, all_rows=True)
        seqs = [SeqInput(1, ctx_len=1, use_kernel=True)] * B
        logits = self.model.forward_batch(tokens, positions, seqs, logits="all", paged=self.pool,
                                          slot_mapping=slots, decode_meta=meta)
        if B not in self.greedy:
            self.greedy[B] = torch.empty(B, dtype=torch.int64, pin_memory=True)
        return logits, argmax_rows(logits, self.greedy[B])

    def _capture(self, B: int) -> None:
        # warm-up and capture run on padding inputs only, so they cannot overwrite real K/V
        self._reset_to_padding(B)
        side = _capture_stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                self._forward(B)
        torch.cuda.current_stream().wait_stream(side)
        if self.mempool is None:
            self.mempool = torch.cuda.graph_pool_handle()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, pool=self.mempool):
            out, _ = self._forward(B)
        self.graphs[B], self.outputs[B] = graph, out

    def _stage_host(self, B: int, par: int, tokens: list[int] | None, positions: list[int], slots: list[int],
                    block_tables: list[list[int]], context_lens: list[int]) -> None:
        """Write one step's inputs into pinned host buffer `par` of bucket B (tokens None: left for later)."""
        n = len(positions)
        W = self.max_blocks
        for t in block_tables:
            if len(t) > W:
                raise ValueError(f"block table of {len(t)} blocks exceeds the graph width {W} (max_seq_len)")
        ht, hp, hs, hl, hb = self._host_np(B, par)
        if tokens is not None:
            ht[:n] = tokens
        hp[:n] = positions
        hs[:n] = slots
        hl[:n] = context_lens
        # Table rows: a block list only grows between steps (every other change rebinds the sequence's
        # list), so a row whose list is the one staged last time needs only its new tail written.
        staged = self._staged_rows[(B, par)]
        for i, t in enumerate(block_tables):
            c, L = staged[i], len(t)
            if c is not None and c[0] is t and c[1] <= L:
                if c[1] < L:
                    hb[i, c[1]:L] = t[c[1]:L]
            else:
                hb[i, :L] = t
                hb[i, L:] = 0
            staged[i] = (t, L)
        for i in range(n, B):
            staged[i] = None
        self._fill_padding((ht, hp, hs, hl, hb), n)

    def _bucket(self, n: int) -> int:
        B = self.bucket_for(n)
        if B is None:
            raise ValueError(f"batch of {n} exceeds the largest graph bucket ({self.max_bucket})")
        return B

    def stage(self, tokens: list[int], positions: list[int], slots: list[int], block_tables: list[list[int]],
              context_lens: list[int]) -> int:
        """Write one step's inputs into the static buffers (padding rows point at the garbage block);
        returns the bucket. The pinned host side alternates between two buffers, so a step can be staged
        while the previous step's copy may still be reading the other one."""
        B = self._bucket(len(tokens))
        par = self._par.get(B, 1) ^ 1
        self._par[B] = par
        self._stage_host(B, par, tokens, positions, slots, block_tables, context_lens)
        self._buffers(B)[0].copy_(self._host_buf(B, par), non_blocking=True)
        return B

    def prestage(self, positions: list[int], slots: list[int], block_tables: list[list[int]],
                 context_lens: list[int]) -> int:
        """Stage the next step's inputs except its tokens (unknown until the running step ends) into the
        host buffer the running step does not use; launch_prestaged() adds the tokens and replays."""
        B = self._bucket(len(positions))
        par = self._par.get(B, 1) ^ 1
        self._stage_host(B, par, None, positions, slots, block_tables, context_lens)
        self._pending = (B, par, len(positions))
        return B

    @torch.inference_mode()
    def launch_prestaged(self, tokens: list[int]) -> torch.Tensor:
        """Complete the prestaged step with its tokens, copy it in and replay its bucket's graph (the caller
        has waited for the previous step); returns the logits view as run() does."""
        B, par, n = self._pending
        self._pending = None
        assert len(tokens) == n and B in self.graphs
        self._host_np(B, par)[0][:n] = tokens
        self._par[B] = par
        self._buffers(B)[0].copy_(self._host_buf(B, par), non_blocking=True)
        self.graphs[B].replay()
        self.last_bucket = B
        return self.outputs[B][:n]

    @torch.inference_mode()
    def run(self, tokens: list[int], positions: list[int], slots: list[int], block_tables: list[list[int]],
            context_lens: list[int]) -> torch.Tensor:
        """One decode step for n requests via the bucket's graph; logits [n, vocab] (a view of the graph's
        output buffer, valid until the next replay of that bucket)."""
        n = len(tokens)
        B = self.bucket_for(n)
        if B is None:
            raise ValueError(f"batch of {n} exceeds the largest graph bucket ({self.max_bucket})")
        if B not in self.graphs:
            self._capture(B)
        torch.cuda.current_stream().synchronize()   # a pinned staging buffer is reused every other step
        self.stage(tokens, positions, slots, block_tables, context_lens)
        self.graphs[B].replay()
        self.last_bucket = B
        return self.outputs[B][:n]

    def greedy_tokens(self, n: int) -> list[int]:
        """Argmax of the first n rows of the last replay (computed inside the graph into pinned host memory):
        waits for the replay, then reads the host buffer."""
        torch.cuda.current_stream().synchronize()
        return self.greedy[self.last_bucket][:n].tolist()

    @torch.inference_mode()
    def capture_all(self, max_batch: int) -> None:
        """Capture every bucket a batch of up to max_batch requests can use."""
        top = self.bucket_for(min(max_batch, self.max_bucket))
        for B in self.buckets:
            if B <= top and B not in self.graphs:
                self._capture(B)


PIECEWISE_CAP = 512


def piecewise_buckets(max_tokens: int, cap: int = PIECEWISE_CAP) -> list[int]:
    """Token-count buckets for mixed steps: every 16 up to 256, then every 32, up to min(max_tokens, cap)."""
    top = min(max_tokens, cap)
    grid = list(range(16, 256, 16)) + list(range(256, cap + 1, 32))
    return [b for b in grid if b < top] + [top]


class PiecewiseGraphRunner:
    def __init__(self, model: Qwen2Model, pool: PagedKVCache, garbage_block: int, max_tokens: int = PIECEWISE_CAP,
                 buckets: list[int] | None = None):
        self.model, self.pool, self.garbage_block = model, pool, garbage_block
        self.buckets = sorted(buckets) if buckets else piecewise_buckets(max_tokens)
        self.max_tokens = self.buckets[-1]
        cfg, dev, dt, Tm = model.cfg, model.device, model.dtype, self.max_tokens
        self.gslot = garbage_block * pool.block_size
        self.tokens = torch.zeros(Tm, dtype=torch.long, device=dev)
        self.positions = torch.zeros(Tm, dtype=torch.long, device=dev)
        self.slots = torch.full((Tm,), self.gslot, dtype=torch.long, device=dev)

        def z(*shape):
            return torch.zeros(1, Tm, *shape, dtype=dt, device=dev)

        self.x = z(cfg.hidden_size)
        self.q, self.k, self.v = z(cfg.n_heads, cfg.head_dim), z(cfg.n_kv_heads, cfg.head_dim), z(cfg.n_kv_heads, cfg.head_dim)
        self.o = z(cfg.n_heads * cfg.head_dim)
        self.cos, self.sin = z(cfg.head_dim), z(cfg.head_dim)
        self.graphs: dict[int, list[torch.cuda.CUDAGraph]] = {}
        self.mempool = None

    @property
    def captured_buckets(self) -> list[int]:
        return sorted(self.graphs)

    def bucket_for(self, n: int) -> int | None:
        return next((b for b in self.buckets if b >= n), None)

    def _piece(self, j: int, B: int) -> None:
        m, L = self.model, self.model.cfg.n_layers
        if j == 0:
            x = torch.nn.functional.embedding(self.tokens[:B], m.embed)[None]
            cos, sin = m.rope(self.positions[:B])
            self.cos[:, :B].copy_(cos)
            self.sin[:, :B].copy_(sin)
        else:
            x = m._post(j - 1, self.x[:, :B], self.o[:, :B])
        if j < L:
            q, k, v = m._pre(j, x, self.cos[:, :B], self.sin[:, :B], self.pool, self.slots[:B])
            self.q[:, :B].copy_(q)
            self.k[:, :B].copy_(k)
            self.v[:, :B].copy_(v)
            self.x[:, :B].copy_(x)
        else:
            self.x[:, :B].copy_(m.final_norm(x))

    def _capture(self, B: int) -> None:
        self.tokens.zero_()
        self.positions.zero_()
        self.slots.fill_(self.gslot)
        L = self.model.cfg.n_layers
        side = _capture_stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                for j in range(L + 1):
                    self._piece(j, B)
        torch.cuda.current_stream().wait_stream(side)
        if self.mempool is None:
            self.mempool = torch.cuda.graph_pool_handle()
        graphs = []
        for j in range(L + 1):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, pool=self.mempool):
                self._piece(j, B)
            graphs.append(g)
        self.graphs[B] = graphs

    @torch.inference_mode()
    def capture_all(self) -> None:
        for B in reversed(self.buckets):   # largest first: its temporaries carve the shared pool once
            if B not in self.graphs:
                self._capture(B)

    @torch.inference_mode()
    def run(self, tokens: list[int], positions: list[int], slots: list[int], seqs: list[SeqInput],
            decode_meta: DecodeMeta | None, rows: torch.Tensor | None = None) -> torch.Tensor:
        """One mixed step of T tokens: logits of each sequence's last token, or of `rows` if given."""
        T = len(tokens)
        B = self.bucket_for(T)
        if B is None:
            raise ValueError(f"step of {T} tokens exceeds the largest piecewise bucket ({self.max_tokens})")
        if B not in self.graphs:
            self._capture(B)
        pad = B - T
        self.tokens[:B].copy_(torch.tensor(tokens + [0] * pad))
        self.positions[:B].copy_(torch.tensor(positions + [0] * pad))
        self.slots[:B].copy_(torch.tensor(slots + [self.gslot] * pad))
        m, graphs = self.model, self.graphs[B]
        q, k, v, o = self.q[:, :T], self.k[:, :T], self.v[:, :T], self.o[:, :T]
        m._rows_cache = None
        slot_view = self.slots[:T]
        for i in range(m.cfg.n_layers):
            graphs[i].replay()
            m._attend(i, q, k, v, seqs, self.pool, decode_meta, out=o, slot_mapping=slot_view)
        graphs[-1].replay()
        m._rows_cache = None
        return m.lm_head_rows(self.x[:, :T], seqs, "last" if rows is None else rows)

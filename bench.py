"""Headline benchmark: decode tokens/s of the HIP decode loop on one MI355X, plus the paged-attention
roofline and the CPU oracle timed beside it.

    python bench.py [--steps K] [--warmup W] [--gpus 1]

Workload: Qwen2.5-1.5B-architecture decoder, random-init bf16 weights (N(0, 0.02),
norms 1, tied embeddings), 32 sequences whose 1024-token random prompts are prefilled into the paged KV
cache through the engine (not timed), then W untimed and K timed greedy decode steps at batch 32. A step
is one LLMEngine.step(): schedule, stage inputs, replay the bucket-32 hipGraph (embedding, 28 layers,
final norm, LM head), argmax + the step's single device->host sync, KV commit. value = 32 * K / (time of
the K steps); inputs and weights are resident in HBM before timing starts.

roofline: the paged-attention decode op alone at BASELINE config 2 (B=32, 14 q / 2 kv heads, hd 64,
ctx U[512, 4096], 16-token pages scattered over a 64k-block pool, 8 disjoint draws used round-robin so the
256 MB Infinity Cache cannot serve them). Algorithmic bytes per call = sum_b ctx_b*n_kv*hd*2(K,V)*2B +
Q and O (2*B*n_heads*hd*2B) + block-table entries read (4B per page) + context lengths (4B per row);
duration = (time between two HIP events bracketing 400 back-to-back calls on the launch stream) / 400,
each call one launch (partitions and their merge).
step_roofline: the decode step's algorithmic HBM bytes (every weight once, the KV cache of every row, the
new K/V and the logits) over the measured step time.
mixed_step: BASELINE config 4 (one 1536-token chunk on 512 cached tokens + 16 decode rows, eager) --
step time and algorithmic TFLOP/s against the bf16 MFMA peak, and the chunked-prefill attention kernel
alone at that shape (FLOPs = sum_j (512 + j + 1) * n_heads * hd * 4 per layer).
fused_ops: the standalone RMSNorm+residual, SiLU*mul and RoPE+KV-write kernels at 32 and 1552 rows of the
1.5B shapes: algorithmic HBM bytes per launch over the HIP-event time (`--ops-only` runs these and the
chunked-prefill kernel alone, for rocprofv3 --pmc passes).
spec_verify: speculative verification through the decode graph -- k + 1 rows per sequence sharing its
block table (k = 2: 32 sequences, k = 4: 24 sequences, 1024-token contexts): ms per verify step.
prefix_sharing: BASELINE config 5 (3B shape, a 1024-token prefix shared by 32 requests through the prefix
cache, 211-token suffixes): decode tokens/s and the step's HBM roofline, logical (a shared block counted
once per row that reads it) and unique bytes.

cpu_baseline: the CPU oracle (oracle/, the reference algorithm restated in PyTorch) on this process's
physical cores (torch threads set to that count; the count, the logical CPUs and the CPU model are recorded):
value = one fp32 decode step of the same 1.5B shape at batch 32 with 1024-token contexts (random-valued
caches), median of 3 timed steps after 1 warm-up; `configs` holds bounded samples of configs 1, 2 (gather +
SDPA per call, fp32 and bf16, also copied beside the roofline), 4 and 5.
"""
from __future__ import annotations

import argparse
import dataclasses
import json
import math
import os
import statistics
import sys
import time

import torch

PEAK_HBM_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0   # dense bf16 MFMA


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def gated_event_times(fn, n: int) -> list[float]:
    """Duration (ms) of each of n calls of fn, from events recorded right before and after it. A sleep
    kernel first keeps the GPU behind the host, so no call waits on Python to be enqueued."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2e8))
    for e0, e1 in evs:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return [e0.elapsed_time(e1) for e0, e1 in evs]


def gated_region_time(fn, n: int) -> float:
    """Time (ms) of n back-to-back calls of fn between one pair of events on the launch stream, behind a
    sleep kernel so the GPU never waits on Python to enqueue the next call."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2e8))
    e0.record()
    for _ in range(n):
        fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


def _attention_draws(B: int, NH: int, NKV: int, HD: int, ctx_lo: int, ctx_hi: int, W: int, R: int = 8,
                     NB: int = 65536, seed: int = 2):
    """R disjoint draws of a decode-attention call: contexts U[ctx_lo, ctx_hi], 16-token pages scattered by one
    random permutation of an NB-block pool (the draws never share a page, so round-robin calls cannot be
    served from the Infinity Cache). Returns the pools and [(q, tables, ctx, algorithmic bytes)]."""
    g = torch.Generator().manual_seed(seed)
    dev = "cuda"
    k = torch.randn(NB, 16, NKV, HD, device=dev, dtype=torch.bfloat16)
    v = torch.randn(NB, 16, NKV, HD, device=dev, dtype=torch.bfloat16)
    perm = torch.randperm(NB, generator=g)
    draws, used = [], 0
    for _ in range(R):
        ctx = torch.randint(ctx_lo, ctx_hi + 1, (B,), generator=g).tolist()
        t = torch.zeros(B, W, dtype=torch.int32)
        for i, c in enumerate(ctx):
            n = -(-c // 16)
            t[i, :n] = perm[used:used + n].int()
            used += n
        q = torch.randn(B, NH, HD, generator=g).to(torch.bfloat16)
        nbytes = (sum(ctx) * NKV * HD * 2 * 2 + 2 * B * NH * HD * 2 + 4 * sum(-(-c // 16) for c in ctx) + 4 * B)
        draws.append((q.to(dev), t.to(dev), torch.tensor(ctx, dtype=torch.int32, device=dev), nbytes))
    return k, v, draws


def _attention_us(k, v, draws, HD: int, products: str = "mfma", n: int = 400) -> float:
    """us per call of n back-to-back calls over the draws (round robin), after one warm pass."""
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    scale = HD ** -0.5
    for q, t, c, _ in draws:
        paged_attention_decode(q, k, v, t, c, scale, products=products)
    it = iter(range(10 ** 9))

    def call():
        q, t, c, _ = draws[next(it) % len(draws)]
        paged_attention_decode(q, k, v, t, c, scale, products=products)

    for _ in range(2 * len(draws)):
        call()
    return gated_region_time(call, n) / n * 1e3


def paged_attention_roofline() -> dict:
    HD = 64
    k, v, draws = _attention_draws(32, 14, 2, HD, 512, 4096, 256)
    us = _attention_us(k, v, draws, HD)
    avg_bytes = sum(d[3] for d in draws) / len(draws)
    achieved = avg_bytes / (us * 1e-6) / 1e9
    del k, v
    return {"bound": "hbm", "kernel": "paged_attention_decode (split-K partitions merged in the same launch), BASELINE config 2",
            "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": pmc_traffic(),
            "bytes_per_launch": int(avg_bytes), "us_per_launch": round(us, 2)}


def attention_ab() -> dict:
    """The decode-attention kernel with its two products on the matrix cores (the product) and on the vector
    ALUs (ns_paged_attn_decode_valu: same partitions, loads and merge), alternating three times (best of
    three per side), at BASELINE config 2 (14 q / 2 kv heads, hd 64, ctx U[512, 4096], table width 256) and at
    config 3's attention (the 1.5B decode step: 12 / 2 heads, hd 128, ctx U[1025, 1152], table width 73): us
    per call and fraction of HBM peak."""
    out = {}
    for name, (NH, NKV, HD, lo, hi, W) in (("config2", (14, 2, 64, 512, 4096, 256)),
                                           ("config3", (12, 2, 128, 1025, 1152, 73))):
        k, v, draws = _attention_draws(32, NH, NKV, HD, lo, hi, W)
        avg_bytes = sum(d[3] for d in draws) / len(draws)
        t = {"mfma": [], "valu": []}
        for _ in range(3):
            for prod in ("mfma", "valu"):
                t[prod].append(_attention_us(k, v, draws, HD, prod))
        out[name] = {prod: {"us_per_call": round(min(x), 2),
                            "frac": round(avg_bytes / (min(x) * 1e-6) / 1e9 / PEAK_HBM_GBS, 4)} for prod, x in t.items()}
        del k, v, draws
        torch.cuda.empty_cache()
    return out


def decode_run(model, prompts: list[list[int]], K: int, W: int, prefix_caching: bool = False,
               first_alone: bool = False) -> dict:
    """Prefill `prompts` through the engine (not timed), W warm-up and K timed greedy decode steps at the full
    batch (every timed step must be a graph replay of the full bucket). first_alone: the first prompt is
    prefilled (and its blocks registered with the prefix cache) before the others are admitted. Returns
    tokens/s, ms/step and the step's algorithmic HBM bytes (every weight once, the KV of every row --
    logical, a shared block counted per row -- and the logits), plus the unique KV bytes."""
    from nanoserve_amd.engine import LLMEngine
    cfg, B = model.cfg, len(prompts)
    # Sequences are admitted a few per prefill step, so the first ones start decoding early: max_new_tokens
    # leaves room for that, and no sequence finishes inside the timed window.
    max_new = W + K + B + 8
    max_seq = max(len(p) for p in prompts) + max_new
    eng = LLMEngine(model, eos_token_ids=[], max_seq_len=max_seq, max_num_seqs=B, max_num_batched_tokens=2048,
                    batch_wait_s=0.0, kv_cache_tokens=B * (max_seq + 16), piecewise_graphs=False,
                    prefix_caching=prefix_caching)
    log(f"prefilling {B} prompts of {len(prompts[0])}..{max(len(p) for p in prompts)} tokens (not timed)")
    t0 = time.perf_counter()
    rest = prompts
    if first_alone:
        eng.add_request(prompts[0], max_new, ignore_eos=True)
        while any(s.is_prefill for s in eng.scheduler.running) or eng.scheduler.waiting:
            eng.step()
        rest = prompts[1:]
    for p in rest:
        eng.add_request(p, max_new, ignore_eos=True)
    while any(s.is_prefill for s in eng.scheduler.running) or eng.scheduler.waiting:
        eng.step()
    torch.cuda.synchronize()
    hits = eng.stats.get("prefix_hit_tokens", 0) if prefix_caching else 0
    log(f"prefill done in {time.perf_counter() - t0:.1f} s (prefix hits {hits} tokens); {W} warm-up decode steps "
        f"(captures bucket {B})")
    for _ in range(W):
        eng.step()
    assert eng.last_step.n_decode == B and eng.last_step.n_prefill == 0
    g0 = eng.stats["graph_steps"]
    ctx_sum = sum(s.num_tokens for s in eng.scheduler.running)   # context of the first timed step (incl. new)
    produced = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(K):
        produced += len(eng.step())
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    assert eng.stats["graph_steps"] - g0 == K, "every timed step must be a graph replay"
    assert produced == B * K and len(eng.scheduler.running) == B, "every timed step must decode the full batch"
    wbytes = sum(t.numel() * t.element_size() for name, t in model.named_weights().items()
                 if name != "model.embed_tokens.weight")
    wbytes += model.lm_head.numel() * model.lm_head.element_size()           # LM head reads the whole table
    kv_tok = cfg.kv_bytes_per_token(model.dtype)
    mean_ctx_total = ctx_sum + B * (K - 1) / 2                                 # sum_b ctx_b averaged over steps
    shared = hits // (B - 1) if prefix_caching and B > 1 else 0              # tokens every row shares
    step_bytes = wbytes + mean_ctx_total * kv_tok + B * cfg.vocab_size * 2
    unique_bytes = step_bytes - (B - 1) * shared * kv_tok
    del eng
    torch.cuda.empty_cache()
    return {"tok_s": produced / elapsed, "ms_step": elapsed / K * 1e3, "step_bytes": step_bytes,
            "unique_bytes": unique_bytes, "prefix_hit_tokens": hits}


def prefix_sharing_bench(K: int, W: int) -> dict:
    """Qwen2.5-3B shape, bf16, random-init weights (drawn on the GPU: the CPU oracle does
    not run this config), one 1024-token random prefix shared by 32 requests, each with its own 211-token
    random suffix; prefix caching on, so the other 31 requests reuse the prefix's 64 blocks (read by every
    row's decode attention through its block table). K greedy decode steps at batch 32."""
    from nanoserve_amd.model import QWEN25_3B, Qwen2Model, random_state_dict
    cfg, B = QWEN25_3B, 32
    log("generating random-init 3B weights (seeded)")
    model = Qwen2Model(cfg, random_state_dict(cfg, seed=0, dtype=torch.bfloat16, device="cuda"))
    g = torch.Generator().manual_seed(5)
    prefix = torch.randint(0, cfg.vocab_size, (1024,), generator=g).tolist()
    prompts = [prefix + torch.randint(0, cfg.vocab_size, (211,), generator=g).tolist() for _ in range(B)]
    run = decode_run(model, prompts, K, W, prefix_caching=True, first_alone=True)
    del model
    ms, nbytes, ubytes = run["ms_step"], run["step_bytes"], run["unique_bytes"]
    return {"workload": "BASELINE config 5: Qwen2.5-3B-shape bf16 greedy decode, batch 32, a shared 1024-token "
                        "prefix (64 blocks) + 32 distinct 211-token suffixes, prefix caching, hipGraph bucket 32",
            "value": round(run["tok_s"], 1), "unit": "tokens/s", "ms_per_step": round(ms, 4),
            "prefix_hit_tokens": run["prefix_hit_tokens"],
            "step_roofline": {"bound": "hbm", "achieved": round(nbytes / (ms * 1e-3) / 1e9, 1), "peak": PEAK_HBM_GBS,
                              "unit": "GB/s", "frac": round(nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
                              "bytes_per_step": int(nbytes), "unique_bytes_per_step": int(ubytes),
                              "unique_frac": round(ubytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}}


def mixed_step_bench(model, cfg, reps: int = 5) -> dict:
    """one engine-sized mixed step on the 1.5B model -- sequence A continues a 1536-token
    chunk on 512 cached tokens while 16 sequences (contexts U[256, 2048], seed 2) decode one token each
    (1552 rows: the tiled HIP GEMMs for the projections, the chunked-prefill kernel for A, the paged decode kernel
    for the 16 rows, LM head on the 17 last rows). The step is repeated `reps` times on the same inputs (it
    rewrites the same K/V slots with the same values); median time. Also the chunked-prefill attention
    alone at this step's shape, against the bf16 MFMA peak."""
    from nanoserve_amd.kernels.paged_attention import paged_attention_prefill, prefill_seq_info
    from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
    from nanoserve_amd.model import DecodeMeta, SeqInput
    dev = "cuda"
    g = torch.Generator().manual_seed(2)
    ctxs = torch.randint(256, 2049, (16,), generator=g).tolist()
    toks_a = torch.randint(0, cfg.vocab_size, (2048,), generator=g).tolist()
    pool = PagedKVCache.from_token_budget(cfg, 2048 + sum(ctxs) + 16 * 17 + 64, 16, dev, torch.bfloat16)
    ta = BlockTable(16)
    ta.reserve(2048, pool.allocator)
    model.forward_batch(torch.tensor(toks_a[:512], device=dev), torch.arange(512, device=dev), [SeqInput(512)],
                        paged=pool, slot_mapping=torch.tensor(ta.slots(512), device=dev))
    ta.commit(512)
    dec_tables, last = [], []
    for c in ctxs:                                     # the decode rows' contexts (prefilled, not timed)
        t = BlockTable(16)
        t.reserve(c + 1, pool.allocator)
        ids = torch.randint(0, cfg.vocab_size, (c,), generator=g).tolist()
        model.forward_batch(torch.tensor(ids, device=dev), torch.arange(c, device=dev), [SeqInput(c)],
                            paged=pool, slot_mapping=torch.tensor(t.slots(c), device=dev))
        t.commit(c)
        dec_tables.append(t)
        last.append(ids[-1])
    T = 1536
    tokens = toks_a[512:] + last
    positions = list(range(512, 2048)) + ctxs
    slots = ta.slots(T) + [s for t in dec_tables for s in t.slots(1)]
    W = max(len(t.blocks) for t in dec_tables)
    seqs = [SeqInput(T, block_table=torch.tensor(ta.blocks, device=dev), ctx_len=512)] + \
           [SeqInput(1, ctx_len=c, use_kernel=True) for c in ctxs]
    meta = DecodeMeta(token_idx=torch.arange(T, T + 16, device=dev),
                      block_tables=torch.tensor([t.blocks + [0] * (W - len(t.blocks)) for t in dec_tables],
                                                dtype=torch.int32, device=dev),
                      context_lens=torch.tensor([c + 1 for c in ctxs], dtype=torch.int32, device=dev))
    tok_t, pos_t, slot_t = (torch.tensor(x, device=dev) for x in (tokens, positions, slots))

    def step():
        return model.forward_batch(tok_t, pos_t, seqs, logits="last", paged=pool, slot_mapping=slot_t,
                                   decode_meta=meta)
    step()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        step()
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    ms = statistics.median(times) * 1e3

    # the same step as the engine runs it: MixedGraphRunner stages the rows and launches the forward; steps
    # above MIXED_GRAPH_MAX_ROWS (512) rows are not recorded as a graph (their launches are a small share of
    # the step), so this one launches its kernels eagerly, on its 1552 rows + a padding row (a recorded step
    # would run its whole 128-row bucket + a padding row)
    from nanoserve_amd.hip_graphs import MixedGraphRunner
    from nanoserve_amd.kv_manager import StepBatch
    sb = StepBatch()
    sb.token_ids, sb.positions, sb.slots = tokens, positions, slots
    sb.seqs = [SeqInput(T, block_table=ta.blocks, ctx_len=512)] + seqs[1:]
    sb.tables = [ta.blocks] + [t.blocks for t in dec_tables]
    sb.dec_idx = list(range(T, T + 16))
    sb.dec_tables = [t.blocks for t in dec_tables]
    sb.dec_lens = [c + 1 for c in ctxs]
    runner = MixedGraphRunner(model, pool, 2048 + 16, 16, 2048, pool.allocator.allocate())
    runner.run(sb)
    runner.greedy_tokens(17)
    gtimes = []
    for _ in range(reps):
        t0 = time.perf_counter()
        runner.run(sb)
        torch.cuda.synchronize()
        gtimes.append(time.perf_counter() - t0)
    g_ms = statistics.median(gtimes) * 1e3
    rows_run = runner.last.rows_run
    recorded = runner.last.graph is not None
    del runner
    H, I, L, V = cfg.hidden_size, cfg.intermediate_size, cfg.n_layers, cfg.vocab_size
    qkv_n = (cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim
    rows = T + 16
    gemm_flops = 2 * rows * L * H * (qkv_n + cfg.n_heads * cfg.head_dim + 2 * I) + 2 * rows * L * I * H
    attn_pf = sum(512 + j + 1 for j in range(T)) * cfg.n_heads * cfg.head_dim * 4 * L
    attn_dec = sum(c + 1 for c in ctxs) * cfg.n_heads * cfg.head_dim * 4 * L
    lm = 2 * 17 * H * V
    flops = gemm_flops + attn_pf + attn_dec + lm

    # the chunked-prefill kernel alone at this step's shape (one layer's call)
    q = torch.randn(T, cfg.n_heads, cfg.head_dim, device=dev, dtype=torch.bfloat16)
    info = prefill_seq_info([0], [T], [512], dev)
    tab = torch.tensor([ta.blocks], dtype=torch.int32, device=dev)
    out = torch.empty_like(q)

    def pf():
        paged_attention_prefill(q, pool.k[0], pool.v[0], tab, info, T, 512 + T, cfg.head_dim ** -0.5, out=out)
    pf()
    pf_ms = gated_region_time(pf, 50) / 50
    pf_flops = attn_pf / L
    del pool
    return {"workload": "BASELINE config 4: 1.5B bf16 mixed step, a 1536-token chunk on 512 cached tokens + 16 "
                        "decode rows (ctx U[256, 2048]), 1552 rows; ms_per_step: the engine's mixed-step path "
                        f"(MixedGraphRunner: {rows_run - 1} rows + 1 padding row, host staging and the H2D copy "
                        f"included; {'a graph replay' if recorded else 'above its 512-row graph bound, so launched eagerly'}); "
                        "eager_ms_per_step: the unpadded eager forward",
            "ms_per_step": round(g_ms, 3), "eager_ms_per_step": round(ms, 3), "tflop_per_step": round(flops / 1e12, 3),
            "achieved_tflops": round(flops / (g_ms * 1e-3) / 1e12, 1), "peak_tflops": PEAK_BF16_TFLOPS,
            "frac": round(flops / (g_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
            "prefill_attention": {"bound": "mfma", "achieved": round(pf_flops / (pf_ms * 1e-3) / 1e12, 1),
                                  "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                  "frac": round(pf_flops / (pf_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4),
                                  "flop_per_launch": int(pf_flops), "us_per_launch": round(pf_ms * 1e3, 2)}}


def fused_ops_bench(reps: int = 100) -> dict:
    """The standalone token-wise kernels -- RMSNorm with the residual add, SiLU*mul, RoPE with the paged KV
    write (the reference's fused.py entry points) -- on the 1.5B shapes at the config-3 decode row count (32)
    and the config-4 step's row count (1552). Algorithmic HBM bytes per launch (every input read once, every
    output written once) over the HIP-event time of `reps` back-to-back launches cycling over 8 input sets
    (the 1552-row sets total 0.2-0.9 GB, beyond the 256 MB Infinity Cache). In the decode step these ops run
    inside the GEMM epilogues; these are the drop-in entry points' own numbers."""
    from nanoserve_amd.kernels.fused import rms_norm, rope_qkv, silu_mul
    dev, bf = "cuda", torch.bfloat16
    H, I, NH, NKV, HD, R = 1536, 8960, 12, 2, 128, 8
    g = torch.Generator().manual_seed(3)
    out = {}
    for rows in (32, 1552):
        xs = [torch.randn(rows, H, generator=g).to(dev, bf) for _ in range(R)]
        rs = [torch.randn(rows, H, generator=g).to(dev, bf) for _ in range(R)]
        w = torch.ones(H, device=dev, dtype=bf)
        gus = [torch.randn(rows, 2 * I, generator=g).to(dev, bf) for _ in range(R)]
        qkvs = [torch.randn(rows, (NH + 2 * NKV) * HD, generator=g).to(dev, bf) for _ in range(R)]
        cos = torch.randn(rows, HD, generator=g).to(dev, bf)
        sin = torch.randn(rows, HD, generator=g).to(dev, bf)
        kc = torch.zeros(rows // 16 + 8, 16, NKV, HD, device=dev, dtype=bf)
        vc = torch.zeros_like(kc)
        slots = torch.randperm(kc.shape[0] * 16, generator=g)[:rows].to(dev)
        it = iter(range(10 ** 9))
        cases = {
            "rms_norm_residual": (lambda: rms_norm(xs[next(it) % R], w, 1e-6, residual=rs[0]),
                                  (4 * rows * H + H) * 2),
            "silu_mul": (lambda: silu_mul(gus[next(it) % R]), 3 * rows * I * 2),
            "rope_qkv_kv_write": (lambda: rope_qkv(qkvs[next(it) % R], cos, sin, NH, NKV, HD, kc, vc, slots),
                                  2 * rows * (NH + 2 * NKV) * HD * 2 + 2 * rows * HD * 2 + 2 * rows * NKV * HD * 2
                                  + 8 * rows),
        }
        for name, (fn, nbytes) in cases.items():
            for _ in range(2 * R):
                fn()
            us = gated_region_time(fn, reps) / reps * 1e3
            gbs = nbytes / (us * 1e-6) / 1e9
            out[f"{name}_{rows}rows"] = {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS,
                                         "unit": "GB/s", "frac": round(gbs / PEAK_HBM_GBS, 4),
                                         "bytes_per_launch": int(nbytes), "us_per_launch": round(us, 2)}
        del xs, rs, gus, qkvs
    return out


def spec_verify_bench(model, cfg, ctx: int = 1024, reps: int = 20) -> dict:
    """Speculative verification through the decode graph (nanoserve/speculative.py:193-211): each sequence's
    k draft tokens plus its last accepted token are k + 1 decode rows sharing the sequence's block table, with
    context lengths ctx + 1 .. ctx + k + 1, in one graph replay. 1.5B shape, bf16, `ctx`-token contexts of
    random K/V; k = 2 with 32 sequences (96 rows) and k = 4 with 24 sequences (120 rows, the largest bucket
    that holds them). Returns ms per verify step and rows (tokens checked) per second."""
    from nanoserve_amd.hip_graphs import DecodeGraphRunner
    from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
    out = {}
    for k, nseq in ((2, 32), (4, 24)):
        k1 = k + 1
        pool = PagedKVCache.from_token_budget(cfg, nseq * (ctx + k1 + 16) + 64, 16, "cuda", torch.bfloat16)
        g = torch.Generator(device="cuda").manual_seed(5)
        pool.k.normal_(generator=g)
        pool.v.normal_(generator=g)
        runner = DecodeGraphRunner(model, pool, max_seq_len=ctx + k1 + 16, pair_rows=True)
        tables = []
        for _ in range(nseq):
            t = BlockTable(16)
            t.reserve(ctx + k1, pool.allocator)
            t.commit(ctx)
            tables.append(t)
        gt = torch.Generator().manual_seed(6)
        toks = torch.randint(0, cfg.vocab_size, (nseq * k1,), generator=gt).tolist()
        args = dict(tokens=toks, positions=[ctx + j for _ in tables for j in range(k1)],
                    slots=[x for t in tables for x in t.slots(k1)],
                    block_tables=[t.blocks for t in tables for _ in range(k1)],
                    context_lens=[ctx + j + 1 for _ in tables for j in range(k1)])
        for _ in range(3):
            runner.run(**args)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            runner.run(**args)
        torch.cuda.synchronize()
        ms = (time.perf_counter() - t0) / reps * 1e3
        out[f"k{k}"] = {"sequences": nseq, "rows": nseq * k1, "ctx": ctx, "ms_per_verify_step": round(ms, 3),
                        "rows_per_s": round(nseq * k1 / (ms * 1e-3), 1)}
        del runner, pool
        torch.cuda.empty_cache()
    return out


def prefill_attention_bench(reps: int = 50) -> dict:
    """The chunked-prefill attention kernel alone at BASELINE config 4's shape with synthetic pages: one
    sequence, a 1536-token chunk on 512 cached tokens (2048 keys), 12 q / 2 kv heads, hd 128, its 128 blocks
    scattered by a random permutation over a 4096-block pool. FLOPs = sum_j (512 + j + 1) * n_heads * hd * 4
    (QK^T and PV, causal) against the bf16 MFMA peak."""
    from nanoserve_amd.kernels.paged_attention import paged_attention_prefill, prefill_seq_info
    dev, bf = "cuda", torch.bfloat16
    T, C, NH, NKV, HD, NB = 1536, 512, 12, 2, 128, 4096
    g = torch.Generator().manual_seed(4)
    k = torch.randn(NB, 16, NKV, HD, generator=g).to(dev, bf)
    v = torch.randn(NB, 16, NKV, HD, generator=g).to(dev, bf)
    q = torch.randn(T, NH, HD, generator=g).to(dev, bf)
    tab = torch.randperm(NB, generator=g)[:(T + C) // 16].int().view(1, -1).to(dev)
    info = prefill_seq_info([0], [T], [C], dev)
    out = torch.empty_like(q)

    def pf():
        paged_attention_prefill(q, k, v, tab, info, T, C + T, HD ** -0.5, out=out)
    for _ in range(3):
        pf()
    us = gated_region_time(pf, reps) / reps * 1e3
    flops = sum(C + j + 1 for j in range(T)) * NH * HD * 4
    tf = flops / (us * 1e-6) / 1e12
    return {"bound": "mfma", "achieved": round(tf, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / PEAK_BF16_TFLOPS, 4), "flop_per_launch": int(flops), "us_per_launch": round(us, 2)}


def copy_calibration(nbytes: int = 512 << 20, reps: int = 4) -> float:
    """A plain device copy of known size (nbytes read + nbytes written per launch): under rocprofv3 --pmc its
    FETCH_SIZE / WRITE_SIZE per dispatch give the scale from counter units to bytes. Returns GB/s."""
    src = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    times = gated_event_times(lambda: dst.copy_(src), reps)
    del src, dst
    return 2 * nbytes / (min(times) * 1e-3) / 1e9


def pmc_traffic() -> int | None:
    """HBM bytes per paged-attention call (one launch) measured by rocprofv3 --pmc FETCH_SIZE
    and WRITE_SIZE runs of `bench.py --attention-only`, scaled by the copy calibration, as committed in
    profiles/paged_attention_decode_config2_pmc.md (None when that summary is absent)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                        "paged_attention_decode_config2_pmc.md")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_call:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def host_cpu() -> dict:
    """This process's CPU share: physical cores (distinct package/core pairs among the CPUs it may run on),
    capped by a cgroup CPU quota and by OMP_NUM_THREADS when those are set; the logical CPU count; the model
    name from /proc/cpuinfo."""
    aff = set(os.sched_getaffinity(0))
    phys, model = set(), None
    try:
        for blk in open("/proc/cpuinfo").read().split("\n\n"):
            d = dict((k.strip(), v.strip()) for k, v in (ln.split(":", 1) for ln in blk.splitlines() if ":" in ln))
            if "processor" not in d:
                continue
            model = model or d.get("model name")
            if int(d["processor"]) in aff:
                phys.add((d.get("physical id", "0"), d.get("core id", d["processor"])))
    except OSError:
        pass
    cores = len(phys) or len(aff)
    caps = {}
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            caps["cgroup_quota_cpus"] = math.ceil(int(quota) / int(period))
    except (OSError, ValueError):
        pass
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        caps["OMP_NUM_THREADS"] = int(os.environ["OMP_NUM_THREADS"])
    threads = min([cores] + [v for v in caps.values() if v > 0])
    return {"threads": threads, "physical_cores": cores, "logical_cpus": os.cpu_count(), "affinity_cpus": len(aff),
            "caps": caps, "model": model}


def _timed(fn, reps: int = 3) -> float:
    """Median seconds of `reps` calls after one warm-up call."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def _filled_cache(orc, ctx: int, room: int, g) -> "object":
    c = orc.new_cache(ctx + room)
    c.k[:, :, :ctx].normal_(generator=g)
    c.v[:, :, :ctx].normal_(generator=g)
    c.length = ctx
    return c


def cpu_baseline(sd_cpu: dict, cfg, B: int, ctx: int) -> dict:
    """The CPU oracle (oracle/, the reference's algorithm restated in PyTorch) on this host's physical cores,
    for every BASELINE config, each a bounded sample timed with perf_counter (one warm-up, median of 3):
      config 1: 0.5B shape fp32, batch 4, 128-token prompts: batched prefill time and decode tok/s over the
                31 batched greedy steps that follow it;
      config 2: gather + SDPA per call (oracle/ops.py paged_attention_reference), fp32 and bf16, on the
                roofline's seeded draws (B 32, 14/2 heads, hd 64, contexts U[512, 4096]);
      config 3: one fp32 decode step of the 1.5B shape, batch B, ctx-token contexts (random-valued caches);
      config 4: one fp32 mixed step of the 1.5B shape (a 1536-token chunk on 512 cached tokens + 16 decode
                rows, contexts U[256, 2048]);
      config 5: fp32 decode step of the 3B shape at batch 32 with 1235-token contexts, from 2- and 4-layer
                slices (time = a + b * layers, extrapolated to 36 layers); the oracle keeps one cache per
                sequence, so prefix sharing changes nothing it computes.
    The headline value is config 3's tokens/s (the bench's own workload)."""
    from nanoserve_amd.model import QWEN25_0_5B, QWEN25_3B, random_state_dict
    from oracle.model import OracleModel
    from oracle.ops import paged_attention_reference
    host = host_cpu()
    torch.set_num_threads(host["threads"])
    g = torch.Generator().manual_seed(11)
    out = {"host": host}

    # config 3 (headline): the bench's decode step
    orc = OracleModel(cfg, sd_cpu, dtype=torch.float32)
    caches = [_filled_cache(orc, ctx, 8, g) for _ in range(B)]
    toks = torch.randint(0, cfg.vocab_size, (B,), generator=g).tolist()

    def step3():
        for c in caches:
            c.length = ctx
        orc.step([(c, [t]) for c, t in zip(caches, toks)])
    s3 = _timed(step3)
    out["config3"] = {"ms_per_step": round(s3 * 1e3, 1), "tok_s": round(B / s3, 2)}
    log(f"cpu config 3: {s3 * 1e3:.0f} ms/step")

    # config 4: one mixed step on the same weights
    g4 = torch.Generator().manual_seed(2)
    ctxs = torch.randint(256, 2049, (16,), generator=g4).tolist()
    ca = _filled_cache(orc, 512, 1536, g)
    dec = [_filled_cache(orc, c, 1, g) for c in ctxs]
    chunk = torch.randint(0, cfg.vocab_size, (1536,), generator=g4).tolist()
    last = torch.randint(0, cfg.vocab_size, (16,), generator=g4).tolist()

    def step4():
        ca.length = 512
        for c, n in zip(dec, ctxs):
            c.length = n
        orc.step([(ca, chunk)] + [(c, [t]) for c, t in zip(dec, last)])
    s4 = _timed(step4)
    out["config4"] = {"ms_per_mixed_step": round(s4 * 1e3, 1), "rows": 1552}
    log(f"cpu config 4: {s4 * 1e3:.0f} ms/mixed step")
    del orc, caches, ca, dec

    # config 2: gather + SDPA per call
    NB, NKV, HD, NH = 65536, 2, 64, 14
    g2 = torch.Generator().manual_seed(2)
    kf = torch.randn(NB, 16, NKV, HD, generator=g2)
    vf = torch.randn(NB, 16, NKV, HD, generator=g2)
    perm = torch.randperm(NB, generator=g2)
    cl = torch.randint(512, 4097, (32,), generator=g2)
    tab = torch.zeros(32, 256, dtype=torch.int32)
    used = 0
    for i, c in enumerate(cl.tolist()):
        n = -(-c // 16)
        tab[i, :n] = perm[used:used + n].int()
        used += n
    qf = torch.randn(32, NH, HD, generator=g2)
    c2 = {}
    for name, dt in (("fp32", torch.float32), ("bf16", torch.bfloat16)):
        kk, vv, qq = kf.to(dt), vf.to(dt), qf.to(dt)
        t2 = _timed(lambda: paged_attention_reference(qq, kk, vv, tab, cl, HD ** -0.5))
        nbytes = int(cl.sum()) * NKV * HD * 2 * kk.element_size() + 2 * 32 * NH * HD * kk.element_size()
        c2[name] = {"ms_per_call": round(t2 * 1e3, 2), "effective_GBs": round(nbytes / t2 / 1e9, 2)}
        del kk, vv, qq
    out["config2"] = c2
    log(f"cpu config 2: gather+SDPA {c2['fp32']['ms_per_call']} ms (fp32), {c2['bf16']['ms_per_call']} ms (bf16)")
    del kf, vf

    # config 1: 0.5B fp32, batch 4, 128-token prompts, prefill + 31 decode steps
    orc1 = OracleModel(QWEN25_0_5B, random_state_dict(QWEN25_0_5B, seed=0, dtype=torch.float32))
    g1 = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, QWEN25_0_5B.vocab_size, (128,), generator=g1).tolist() for _ in range(4)]
    cs1 = [orc1.new_cache(160) for _ in prompts]
    res = {}

    def run1():
        for c in cs1:
            c.length = 0
            c.tokens = []
        t0 = time.perf_counter()
        lg = orc1.step([(c, p) for c, p in zip(cs1, prompts)])
        t1 = time.perf_counter()
        nxt = lg.argmax(-1).tolist()
        for _ in range(31):
            nxt = orc1.step([(c, [t]) for c, t in zip(cs1, nxt)]).argmax(-1).tolist()
        res.setdefault("prefill", []).append(t1 - t0)
        res.setdefault("decode", []).append(time.perf_counter() - t1)
    for _ in range(4):
        run1()
    pre, decs = statistics.median(res["prefill"][1:]), statistics.median(res["decode"][1:])
    out["config1"] = {"prefill_ms": round(pre * 1e3, 1), "decode_tok_s": round(4 * 31 / decs, 2)}
    log(f"cpu config 1: prefill {pre * 1e3:.0f} ms, decode {4 * 31 / decs:.1f} tok/s")
    del orc1, cs1

    # config 5: 3B shape from 2- and 4-layer slices
    t5 = {}
    for L in (2, 4):
        c5 = dataclasses.replace(QWEN25_3B, n_layers=L)
        o5 = OracleModel(c5, random_state_dict(c5, seed=5, dtype=torch.float32))
        cc = [_filled_cache(o5, 1235, 2, g) for _ in range(32)]
        tk = torch.randint(0, c5.vocab_size, (32,), generator=g).tolist()

        def step5():
            for c in cc:
                c.length = 1235
            o5.step([(c, [t]) for c, t in zip(cc, tk)])
        t5[L] = _timed(step5)
        del o5, cc
    per_layer = (t5[4] - t5[2]) / 2
    s5 = t5[2] + per_layer * (QWEN25_3B.n_layers - 2)
    out["config5"] = {"ms_per_step": round(s5 * 1e3, 1), "tok_s": round(32 / s5, 2),
                      "sliced_ms": {str(k): round(v * 1e3, 1) for k, v in t5.items()}}
    log(f"cpu config 5: {s5 * 1e3:.0f} ms/step (extrapolated)")

    return {"value": round(B / s3, 2), "unit": "tokens/s", "cores": host["threads"], "kind": "port",
            "sample": f"CPU oracle (fp32 PyTorch restatement of the reference) on {host['threads']} threads = "
                      f"physical cores of this process's CPU share ({host['model']}): config-3 decode step, 1.5B "
                      f"shape, batch {B}, {ctx}-token random-valued contexts, median of 3 steps after 1 "
                      f"warm-up: {s3 * 1e3:.0f} ms/step; per-config samples under 'configs'",
            "configs": out}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=128)
    ap.add_argument("--warmup", type=int, default=4)
    ap.add_argument("--batch", type=int, default=32)
    ap.add_argument("--prompt-len", type=int, default=1024)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-mixed-step", action="store_true", help="skip the config-4 mixed-step measurement")
    ap.add_argument("--no-prefix-sharing", action="store_true", help="skip the config-5 prefix-sharing decode run")
    ap.add_argument("--attention-only", action="store_true",
                    help="only the paged-attention roofline and the copy calibration (for rocprofv3 --pmc passes)")
    ap.add_argument("--attention-ab", action="store_true",
                    help="only the decode-attention kernel with MFMA vs VALU products at configs 2 and 3")
    ap.add_argument("--mixed-only", action="store_true",
                    help="only the config-4 mixed step, engine path and eager (for rocprofv3 kernel traces)")
    ap.add_argument("--ops-only", action="store_true",
                    help="only the fused token-wise ops, the chunked-prefill kernel alone and the copy calibration "
                         "(for rocprofv3 --pmc passes)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (data-parallel replicas would "
              "scale the per-GPU number with no exchange); run it with --gpus 1", file=sys.stderr)
        return 2
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    if args.attention_ab:
        ab = attention_ab()
        log("attention A/B (us per call, mfma vs valu): " + ", ".join(
            f"{k}: {v['mfma']['us_per_call']} vs {v['valu']['us_per_call']}" for k, v in ab.items()))
        print(json.dumps({"attention_ab": ab}), flush=True)
        return 0
    if args.attention_only:
        roof = paged_attention_roofline()
        log(f"paged attention: {roof['us_per_launch']} us/call, {roof['achieved']} GB/s")
        log(f"copy calibration: {copy_calibration():.0f} GB/s")
        print(json.dumps({"roofline": roof}), flush=True)
        return 0
    if args.ops_only:
        ops = fused_ops_bench()
        pfa = prefill_attention_bench()
        log(f"prefill attention alone: {pfa['us_per_launch']} us/launch, {pfa['achieved']} TFLOP/s")
        log(f"copy calibration: {copy_calibration():.0f} GB/s")
        print(json.dumps({"fused_ops": ops, "prefill_attention": pfa}), flush=True)
        return 0
    from nanoserve_amd.model import QWEN25_1_5B, QWEN25_3B, Qwen2Model, random_state_dict

    cfg, B, P, K, W = QWEN25_1_5B, args.batch, args.prompt_len, args.steps, args.warmup
    torch.manual_seed(0)
    log("generating random-init 1.5B weights (CPU, fp32, seeded)")
    sd_cpu = random_state_dict(cfg, seed=0, dtype=torch.float32)
    model = Qwen2Model(cfg, {n: t.to("cuda", torch.bfloat16) for n, t in sd_cpu.items()})
    if args.mixed_only:
        mixed = mixed_step_bench(model, cfg)
        log(f"mixed step: {mixed['ms_per_step']} ms engine path, {mixed['eager_ms_per_step']} ms eager")
        print(json.dumps({"mixed_step": mixed}), flush=True)
        return 0
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, cfg.vocab_size, (P,), generator=g).tolist() for _ in range(B)]
    run = decode_run(model, prompts, K, W)
    tok_s, ms_step, step_bytes = run["tok_s"], run["ms_step"], run["step_bytes"]
    step_gbs = step_bytes / (ms_step * 1e-3) / 1e9
    log(f"decode: {tok_s:.0f} tok/s, {ms_step:.3f} ms/step, {step_gbs:.0f} GB/s algorithmic")

    log("speculative verification rows (k = 2, 4)")
    spec = spec_verify_bench(model, cfg)
    log(f"verify steps: k=2 {spec['k2']['ms_per_verify_step']} ms ({spec['k2']['rows']} rows), "
        f"k=4 {spec['k4']['ms_per_verify_step']} ms ({spec['k4']['rows']} rows)")

    mixed = None
    if not args.no_mixed_step:
        log("mixed step (config 4 shape)")
        mixed = mixed_step_bench(model, cfg)
        torch.cuda.empty_cache()
        log(f"mixed step: {mixed['ms_per_step']} ms engine path, {mixed['eager_ms_per_step']} ms eager "
            f"({mixed['achieved_tflops']} TFLOP/s); chunked-prefill attention "
            f"{mixed['prefill_attention']['us_per_launch']} us/layer ({mixed['prefill_attention']['achieved']} TFLOP/s)")
    log("paged-attention roofline (config 2 shape)")
    roof = paged_attention_roofline()
    log(f"paged attention: {roof['us_per_launch']} us/call, {roof['achieved']} GB/s")
    log("fused token-wise ops alone (32 and 1552 rows)")
    ops = fused_ops_bench()

    prefix = None
    if not args.no_prefix_sharing:
        del model
        torch.cuda.empty_cache()
        log("prefix sharing (config 5: 3B shape)")
        prefix = prefix_sharing_bench(K, W)
        torch.cuda.empty_cache()
        log(f"prefix sharing: {prefix['value']} tok/s, {prefix['ms_per_step']} ms/step")
    cpu = None
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle, fp32)")
        model = None
        torch.cuda.empty_cache()
        cpu = cpu_baseline(sd_cpu, cfg, B, P)
        log(f"cpu: {cpu['value']} tok/s on {cpu['cores']} threads")
        roof["cpu_gather_sdpa"] = cpu["configs"]["config2"]

    out = {
        "metric": "decode tok/s, Qwen2.5-1.5B-shape b=32; paged-attn HBM GB/s as % of peak",
        "value": round(tok_s, 1), "unit": "tokens/s", "n_gpus": 1, "steps": K, "warmup": W,
        "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: random-init weights N(0,0.02), random 1024-token prompts",
        "config": {"workload": "BASELINE config 3: Qwen2.5-1.5B-shape bf16 greedy decode, batch 32, "
                               "1024-token prompts in the paged KV cache, hipGraph bucket 32",
                   "batch": B, "prompt_len": P, "block_size": 16},
        "roofline": roof,
        "step_roofline": {"bound": "hbm", "achieved": round(step_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(step_gbs / PEAK_HBM_GBS, 4), "bytes_per_step": int(step_bytes),
                          "roofline_tok_s": round(B / (step_bytes / (PEAK_HBM_GBS * 1e9)), 1)},
        "mixed_step": mixed,
        "fused_ops": ops,
        "spec_verify": spec,
        "prefix_sharing": prefix,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())

"""Writes the golden fixtures in this folder by running the REFERENCE (darshanseenivasakumar/nanoserve,
read-only at /root/reference) on the CPU. Run it only where the reference is mounted:

    python tests/golden/make_golden.py [--reference /root/reference]

Nothing else in this repository imports the reference; the tests read only the JSON this script writes.

config1_fp32_streams.json
    BASELINE config 1 through the reference's own engine on its fp32 CPU path (LLMEngine with
    attn_backend="sdpa", fused_ops=False, cuda_graphs=False, device "cpu"; nanoserve/engine.py:195-260):
    Qwen2.5-0.5B architecture with this repo's seeded random-init weights (nanoserve_amd.model
    .random_state_dict, seed 0, fp32), 4 prompts of 128 tokens (torch.Generator seed 1), 32 greedy steps.

host_traces.json
    The reference's host integer state, step by step, for small scenarios that exercise its scheduler
    (nanoserve/scheduler.py:161-200), KV manager (kv_manager.py:70-202) and block allocators / prefix cache
    (kv_cache.py:75-248) as called by LLMEngine.step: chunked prefill mixed with decodes (config 4 in small),
    a shared prefix through the prefix cache (config 5 in small), LIFO preemption with and without chunking,
    prefix-cache eviction, the static policy, EOS finishes and aborts. The model is replaced by a stub whose
    greedy token for a sequence is a fixed function of the tokens and last position it was fed (STUB_VOCAB,
    stub_token), so the trace depends on the host logic alone. Per step it records what the engine scheduled,
    every tensor the model received (tokens, positions, slot mapping, per-sequence tables and context
    lengths, decode metadata), the outputs, free blocks, preemptions, the running sequences' block tables,
    refcounts, the evictable LRU order and the prefix-hit counters.
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

STUB_VOCAB = 64
STUB_EOS = 5


def stub_token(tokens: list[int], last_position: int) -> int:
    """The stub model's greedy choice for one sequence (shared with tests/test_host_traces.py)."""
    return (sum(tokens) * 31 + last_position * 7 + 13) % STUB_VOCAB


SCENARIOS = [
    # name, engine kwargs, requests [(prompt_len, max_new, ignore_eos, prompt_seed, shared_prefix_len)],
    # arrivals [(step, n_requests_added_so_far)], aborts [(step, request index)], reserve_garbage_block
    dict(name="chunked_mixed", engine=dict(max_seq_len=512, max_num_seqs=8, max_num_batched_tokens=96,
                                           kv_cache_tokens=4096, chunked_prefill=True),
         requests=[(23, 12, True), (40, 9, True), (17, 14, False), (60, 7, True), (33, 12, True), (300, 5, True),
                   (90, 6, True), (45, 8, False)],
         arrivals=[(0, 5), (3, 6), (5, 8)], aborts=[], garbage=True),
    dict(name="prefix_sharing", engine=dict(max_seq_len=512, max_num_seqs=8, max_num_batched_tokens=256,
                                            kv_cache_tokens=4096, prefix_caching=True),
         requests=[(64 + 21, 10, True, 64), (64 + 13, 10, True, 64), (64 + 40, 10, True, 64),
                   (64 + 16, 10, True, 64), (64 + 5, 10, True, 64), (64 + 33, 10, True, 64),
                   (64 + 21, 10, True, 64, "dup0"), (64 + 27, 10, True, 64)],
         arrivals=[(0, 1), (2, 6), (6, 8)], aborts=[], garbage=True),
    dict(name="preemption_chunked", engine=dict(max_seq_len=256, max_num_seqs=6, max_num_batched_tokens=64,
                                                kv_cache_tokens=256, chunked_prefill=True),
         requests=[(40, 30, True), (38, 30, True), (41, 30, True), (35, 30, True), (44, 30, True), (30, 30, True)],
         arrivals=[(0, 4), (2, 6)], aborts=[], garbage=False),
    dict(name="preemption_unchunked", engine=dict(max_seq_len=256, max_num_seqs=6, max_num_batched_tokens=128,
                                                  kv_cache_tokens=320, chunked_prefill=False),
         requests=[(50, 40, True), (47, 40, True), (52, 40, True), (45, 40, True), (33, 40, True)],
         arrivals=[(0, 5)], aborts=[], garbage=False),
    dict(name="prefix_eviction", engine=dict(max_seq_len=256, max_num_seqs=4, max_num_batched_tokens=256,
                                             kv_cache_tokens=384, prefix_caching=True),
         requests=[(48 + 20, 6, True, 48), (48 + 9, 6, True, 48), (80, 6, True), (70, 6, True),
                   (48 + 20, 6, True, 48, "dup0"), (48 + 31, 5, True, 48), (90, 5, True), (48 + 9, 4, True, 48, "dup1")],
         arrivals=[(0, 2), (4, 4), (12, 6), (20, 8)], aborts=[], garbage=True),
    dict(name="static_policy", engine=dict(max_seq_len=256, policy="static", max_num_seqs=3,
                                           max_num_batched_tokens=512, kv_cache_tokens=2048, batch_wait_s=0.0),
         requests=[(20, 5, True), (31, 8, True), (12, 3, True), (25, 6, True), (18, 4, True)],
         arrivals=[(0, 5)], aborts=[], garbage=True),
    dict(name="eos_and_abort", engine=dict(max_seq_len=256, max_num_seqs=8, max_num_batched_tokens=128,
                                           kv_cache_tokens=2048),
         requests=[(30, 40, False), (22, 40, False), (41, 40, True), (19, 40, False), (27, 40, False),
                   (35, 12, True)],
         arrivals=[(0, 4), (7, 6)], aborts=[(5, 2), (9, 4)], garbage=True),
]


def make_prompts(scn: dict) -> list[list[int]]:
    """Prompt token ids of a scenario's requests (seeded; a shared prefix comes from one generator)."""
    g = torch.Generator().manual_seed(1000 + len(scn["name"]))
    shared = torch.randint(0, STUB_VOCAB, (512,), generator=g).tolist()
    out = []
    for r in scn["requests"]:
        n, pre = r[0], (r[3] if len(r) > 3 else 0)
        if len(r) > 4:                                   # an exact repeat of an earlier prompt
            out.append(list(out[int(r[4][3:])]))
            continue
        own = torch.randint(0, STUB_VOCAB, (n - pre,), generator=g).tolist()
        out.append(shared[:pre] + own)
    return out


def reference_trace(ref, scn: dict) -> dict:
    """Run one scenario through the reference's LLMEngine with the stub model; returns its records."""
    from nanoserve.engine import LLMEngine
    from nanoserve.model import ModelConfig

    cfg = ModelConfig(vocab_size=STUB_VOCAB, hidden_size=8, n_layers=1, n_heads=1, n_kv_heads=1, head_dim=8,
                      intermediate_size=8, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
    fed: list[dict] = []

    class StubModel:
        def __init__(self):
            self.cfg, self.device, self.dtype, self.fused = cfg, torch.device("cpu"), torch.float32, False

        def forward_batch(self, token_ids, positions, seqs, logits="last", paged=None, slot_mapping=None,
                          decode_meta=None):
            toks, pos = token_ids.tolist(), positions.tolist()
            rec = {"tokens": toks, "positions": pos,
                   "slots": slot_mapping.tolist() if slot_mapping is not None else None,
                   "seqs": [[s.n_tokens, s.ctx_len, bool(s.use_kernel),
                             s.block_table.tolist() if s.block_table is not None else None] for s in seqs],
                   "decode": None}
            if decode_meta is not None:
                rec["decode"] = {"token_idx": decode_meta.token_idx.tolist(),
                                 "tables": decode_meta.block_tables.tolist(),
                                 "lens": decode_meta.context_lens.tolist()}
            fed.append(rec)
            out = torch.zeros(len(seqs), STUB_VOCAB)
            start = 0
            for i, s in enumerate(seqs):
                out[i, stub_token(toks[start:start + s.n_tokens], pos[start + s.n_tokens - 1])] = 1.0
                start += s.n_tokens
            return out

    kw = dict(scn["engine"])
    kw.setdefault("batch_wait_s", 0.0)
    eng = LLMEngine(StubModel(), [STUB_EOS], attn_backend="triton", fused_ops=False, cuda_graphs=False,
                    piecewise_graphs=False, **kw)
    if scn["garbage"]:
        eng.kv.pool.allocator.allocate()            # what DecodeGraphRunner takes at start-up
    plans = []
    orig = eng.scheduler.schedule

    def schedule(now):
        p = orig(now)
        plans.append(p)
        return p

    eng.scheduler.schedule = schedule
    prompts = make_prompts(scn)
    ids: list[int] = []
    arrivals, aborts = list(scn["arrivals"]), list(scn["aborts"])
    records, step = [], 0
    while arrivals or eng.has_unfinished():
        while arrivals and step >= arrivals[0][0]:
            _, upto = arrivals.pop(0)
            for i in range(len(ids), upto):
                n_new, ign = scn["requests"][i][1], scn["requests"][i][2]
                ids.append(eng.add_request(prompts[i], n_new, ignore_eos=ign, arrival_time=0.0))
        for st, i in [a for a in aborts if a[0] == step]:
            eng.abort(ids[i])
        n_fed = len(fed)
        outs = eng.step()
        plan = plans[-1]
        rec = {"sched": [[s.seq_id, c] for s, c in zip(plan.scheduled, plan.chunks)],
               "admitted": [s.seq_id for s in plan.admitted]}
        if len(fed) > n_fed:
            rec.update(fed[-1])
        rec["out"] = [[o.seq_id, o.token, bool(o.finished)] for o in outs]
        kv = eng.kv
        rec["free"] = kv.num_free_blocks
        rec["preempt"] = eng.scheduler.num_preemptions
        rec["tables"] = sorted([s.seq_id, list(s.block_table.blocks), s.block_table.num_tokens]
                               for s in eng.scheduler.running)
        rec["waiting"] = [s.seq_id for s in eng.scheduler.waiting]
        if kv.prefix_caching:
            rec["refs"] = sorted([b, r] for b, r in kv.alloc.ref.items())
            rec["evictable"] = list(kv.alloc.evictable)
            rec["hits"] = [kv.prefix_query_tokens, kv.prefix_hit_tokens]
        records.append(rec)
        step += 1
    return {"name": scn["name"], "engine": scn["engine"], "requests": scn["requests"], "prompts": prompts,
            "arrivals": scn["arrivals"], "aborts": scn["aborts"], "garbage": scn["garbage"],
            "records": records, "stats": {k: eng.stats[k] for k in ("steps", "prefill_chunks", "peak_running",
                                                                     "num_preemptions")}}


def config1_streams() -> dict:
    from nanoserve.engine import LLMEngine
    from nanoserve.model import ModelConfig, Qwen2Model
    from nanoserve_amd.model import QWEN25_0_5B, random_state_dict

    cfg = ModelConfig(**{f: getattr(QWEN25_0_5B, f) for f in QWEN25_0_5B.__dataclass_fields__})
    sd = random_state_dict(QWEN25_0_5B, seed=0, dtype=torch.float32)
    model = Qwen2Model(cfg, sd)
    g = torch.Generator().manual_seed(1)
    prompts = [torch.randint(0, cfg.vocab_size, (128,), generator=g).tolist() for _ in range(4)]
    eng = LLMEngine(model, [], max_seq_len=512, max_num_seqs=8, max_num_batched_tokens=512, batch_wait_s=0.0,
                    kv_cache_tokens=16384, attn_backend="sdpa", fused_ops=False, cuda_graphs=False)
    ids = [eng.add_request(p, 32, ignore_eos=True) for p in prompts]
    outs = {i: [] for i in ids}
    while eng.has_unfinished():
        for o in eng.step():
            outs[o.seq_id].append(o.token)
    return {"config": "Qwen2.5-0.5B architecture, random_state_dict(seed=0, fp32), prompts torch.Generator(1) "
                      "randint(0, 151936, (128,)) x4, 32 greedy steps, reference fp32 CPU path",
            "prompts": prompts, "streams": [outs[i] for i in ids], "steps": eng.stats["steps"]}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    ap.add_argument("--only", choices=["traces", "config1"], default=None)
    args = ap.parse_args()
    sys.path.insert(0, args.reference)
    torch.manual_seed(0)
    if args.only in (None, "traces"):
        traces = {"stub": {"vocab": STUB_VOCAB, "eos": STUB_EOS,
                           "token": "(sum(tokens fed to the sequence this step) * 31 + its last position * 7 + 13) "
                                    "% vocab"},
                  "scenarios": [reference_trace(None, s) for s in SCENARIOS]}
        (HERE / "host_traces.json").write_text(json.dumps(traces, separators=(",", ":")))
        for s in traces["scenarios"]:
            print(s["name"], s["stats"])
    if args.only in (None, "config1"):
        c1 = config1_streams()
        (HERE / "config1_fp32_streams.json").write_text(json.dumps(c1))
        print("config 1:", c1["steps"], "steps;", [s[:6] for s in c1["streams"]])


if __name__ == "__main__":
    main()

"""The host integer layer (Scheduler, PagedKVManager, BlockPool, LLMEngine.step) against the REFERENCE's
own traces (tests/golden/host_traces.json, written by tests/golden/make_golden.py from nanoserve's
LLMEngine on the CPU). Each scenario is replayed through this package's engine with a stand-in executor
that returns the same stub greedy tokens the reference's stub model returned (a fixed function of the
tokens and last position a sequence was fed), so the comparison isolates the host logic. Every step must
match bit for bit: what was scheduled and admitted, the flattened token ids, positions and slot mapping,
each sequence's context length and block table, the decode rows' indices, tables and context lengths,
the outputs, free blocks, preemptions, every running table, the waiting queue and, with prefix caching,
the reference counts, the evictable LRU order and the hit counters.

Deliberate difference: a fresh prefill (ctx 0) carries its block table here (the HIP prefill attention
reads its pages in place); the reference passes none (its SDPA uses the step's own K/V). With prefix
caching, the graph runner's garbage block is held by this pool's reference counts but not by the
reference's caching allocator (it takes it from the base allocator); it is left out of the comparison.
"""
import json
from pathlib import Path

import pytest
import torch

from nanoserve_amd.engine import Launch, LLMEngine
from nanoserve_amd.model import ModelConfig
from tests.golden.make_golden import STUB_EOS, STUB_VOCAB, stub_token

TRACES = json.loads((Path(__file__).resolve().parent / "golden" / "host_traces.json").read_text())


class StubModel:
    def __init__(self):
        self.cfg = ModelConfig(vocab_size=STUB_VOCAB, hidden_size=8, n_layers=1, n_heads=1, n_kv_heads=1, head_dim=8,
                               intermediate_size=8, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
        self.device, self.dtype = torch.device("cpu"), torch.float32


class StubExecutor:
    """Computes the stub tokens from the StepBatch and records what the model would have been fed."""

    def __init__(self):
        self.fed = []
        self.timed = False

    def launch(self, sb):
        rec = {"tokens": list(sb.token_ids), "positions": list(sb.positions), "slots": list(sb.slots),
               "seqs": [[s.n_tokens, s.ctx_len, bool(s.use_kernel),
                         list(s.block_table) if s.block_table is not None else None] for s in sb.seqs],
               "decode": None}
        if sb.dec_idx:
            w = max(len(t) for t in sb.dec_tables)
            rec["decode"] = {"token_idx": list(sb.dec_idx), "tables": [t + [0] * (w - len(t)) for t in sb.dec_tables],
                             "lens": list(sb.dec_lens)}
        self.fed.append(rec)
        toks, start = [], 0
        for s in sb.seqs:
            toks.append(stub_token(sb.token_ids[start:start + s.n_tokens], sb.positions[start + s.n_tokens - 1]))
            start += s.n_tokens
        return Launch("eager", len(toks), toks)

    def tokens(self, h):
        return h.logits

    def can_prestage(self, n):
        return False

    def capture(self):
        pass

    def stats(self):
        return {"cuda_graphs": False, "graph_buckets": []}


def replay(scn):
    ex = StubExecutor()
    kw = dict(scn["engine"])
    kw.setdefault("batch_wait_s", 0.0)
    eng = LLMEngine(StubModel(), [STUB_EOS], executor=ex, **kw)
    garbage = eng.kv.pool.allocator.allocate() if scn["garbage"] else None
    prompts, ids, records, step = scn["prompts"], [], [], 0
    arrivals, aborts = [list(a) for a in scn["arrivals"]], [list(a) for a in scn["aborts"]]
    plans = []
    orig = eng.scheduler.schedule

    def schedule(now):
        p = orig(now)
        plans.append(p)
        return p

    eng.scheduler.schedule = schedule
    while arrivals or eng.has_unfinished():
        while arrivals and step >= arrivals[0][0]:
            _, upto = arrivals.pop(0)
            for i in range(len(ids), upto):
                req = scn["requests"][i]
                ids.append(eng.add_request(prompts[i], req[1], ignore_eos=req[2], arrival_time=0.0))
        for st, i in [a for a in aborts if a[0] == step]:
            eng.abort(ids[i])
        n_fed = len(ex.fed)
        outs = eng.step()
        plan = plans[-1]
        rec = {"sched": [[s.seq_id, c] for s, c in zip(plan.scheduled, plan.chunks)],
               "admitted": [s.seq_id for s in plan.admitted]}
        if len(ex.fed) > n_fed:
            rec.update(ex.fed[-1])
        rec["out"] = [[o.seq_id, o.token, bool(o.finished)] for o in outs]
        kv = eng.kv
        rec["free"] = kv.num_free_blocks
        rec["preempt"] = eng.scheduler.num_preemptions
        rec["tables"] = sorted([s.seq_id, list(s.block_table.blocks), s.block_table.num_tokens]
                               for s in eng.scheduler.running)
        rec["waiting"] = [s.seq_id for s in eng.scheduler.waiting]
        if kv.prefix_caching:
            rec["refs"] = sorted([b, r] for b, r in kv.alloc.held().items() if b != garbage)
            rec["evictable"] = kv.alloc.evictable()
            rec["hits"] = [kv.prefix_query_tokens, kv.prefix_hit_tokens]
        records.append(rec)
        step += 1
    return records, eng


@pytest.mark.parametrize("scn", TRACES["scenarios"], ids=[s["name"] for s in TRACES["scenarios"]])
def test_engine_host_state_matches_the_reference_trace(scn):
    ours, eng = replay(scn)
    ref = scn["records"]
    assert len(ours) == len(ref), f"{len(ours)} steps, the reference took {len(ref)}"
    for k, (a, b) in enumerate(zip(ours, ref)):
        for key, want in b.items():
            got = a.get(key)
            if key == "seqs":
                assert len(got) == len(want), (k, key)
                for g, w in zip(got, want):
                    assert g[:3] == w[:3], (k, key, g, w)
                    if w[3] is not None:
                        assert g[3] == w[3], (k, key, g, w)
                    elif not w[2]:                     # fresh prefill: we carry its table, the reference none
                        assert w[1] == 0 and g[3] is not None
                continue
            assert got == want, f"step {k}: {key} differs:\n ours {got}\n ref  {want}"
    st = eng.stats
    for key, want in scn["stats"].items():
        assert st[key] == want, (key, st[key], want)


def test_traces_cover_the_behaviours_they_pin():
    """The fixture exercises what it claims: chunked prefill, preemption, prefix hits, eviction of cached
    blocks, EOS finishes and aborts."""
    by = {s["name"]: s for s in TRACES["scenarios"]}
    assert by["chunked_mixed"]["stats"]["prefill_chunks"] > 0
    assert by["preemption_chunked"]["stats"]["num_preemptions"] > 0
    assert by["preemption_unchunked"]["stats"]["num_preemptions"] > 0
    assert by["prefix_sharing"]["records"][-1]["hits"][1] > 0
    assert any(r["evictable"] for r in by["prefix_eviction"]["records"])
    eos = [o for r in by["eos_and_abort"]["records"] for o in r["out"] if o[2] and o[1] == STUB_EOS]
    assert eos


def _fails(scenarios) -> list[str]:
    bad = []
    for scn in scenarios:
        try:
            test_engine_host_state_matches_the_reference_trace(scn)
        except (AssertionError, IndexError, ValueError):   # a diverging run may also break an invariant
            bad.append(scn["name"])
    return bad


def test_planted_host_mistakes_fail_the_traces(monkeypatch):
    """Plausible slips in the host integer logic break at least one reference trace: freeing a request's
    blocks head first with prefix caching (the LRU order of cached blocks), and preempting the oldest running
    request instead of the newest. (The prefix-hit cap of (len - 1) // 16 blocks matters only for a fully
    cached prompt of whole blocks, which no trace holds; tests/test_host_logic.py pins it by known answer.)"""
    from nanoserve_amd import kv_cache, scheduler
    assert _fails(TRACES["scenarios"]) == []

    orig_free = kv_cache.BlockPool.free

    def free_head_first(self, blocks):
        pc, self.prefix_caching = self.prefix_caching, False
        try:
            orig_free(self, blocks)
        finally:
            self.prefix_caching = pc

    orig_evict = scheduler.Scheduler._evict_newest

    def evict_oldest(self):
        self.running.append(self.running.pop(0))
        return orig_evict(self)

    for name, (owner, attr, fn) in {"free order": (kv_cache.BlockPool, "free", free_head_first),
                                    "preemption order": (scheduler.Scheduler, "_evict_newest", evict_oldest)}.items():
        with monkeypatch.context() as m:
            m.setattr(owner, attr, fn)
            assert _fails(TRACES["scenarios"]), f"planted mistake '{name}' passes every trace"

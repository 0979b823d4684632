"""The HIP forward and the engine on the GPU vs the CPU oracle (oracle/model.py), on seeded random-init
weights drawn on the CPU (identical values on both sides).

Gates (the reference's own, restated): fp32 logits of a mixed step (fresh prefill + chunk on a cached
context + decodes) within 1e-3 of the oracle (tests/test_model.py:44-52, tests/test_paged_engine.py:66-69);
greedy tokens of the engine identical to the oracle's for the first 32 steps (0.5B shape,
fp32, batch 4, 128-token prompts); bf16 streams teacher-forced against the fp32 oracle with a logit-error
bound (tests/parity.py, the reference's tie rule tests/test_llm_engine.py:72-87 made scale-aware);
a graph step bitwise equal to the eager step at an exact bucket and padding rows touching only the garbage
block (tests/test_cuda_graphs.py:58-86); chunked prefill, preemption and prefix caching leave fp32 tokens
unchanged and leak no blocks (tests/test_chunked_prefill.py, test_paged_engine.py, test_prefix_cache.py).
"""
import json
import random
from pathlib import Path

import pytest
import torch

from nanoserve_amd.model import QWEN25_0_5B, DecodeMeta, ModelConfig, Qwen2Model, SeqInput, random_state_dict
from oracle.model import OracleModel
from tests.parity import DELTA_SMALL128, LogitsRecorder, check_streams

pytestmark = pytest.mark.gpu

SMALL = ModelConfig(vocab_size=2048, hidden_size=256, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=64,
                    intermediate_size=512, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
SMALL128 = ModelConfig(vocab_size=2048, hidden_size=768, n_layers=2, n_heads=6, n_kv_heads=2, head_dim=128,
                       intermediate_size=1024, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
TIE_GAP_FP32 = 1e-3     # fp32 GPU vs CPU: only genuine near-ties may flip


def gpu_model(cfg, dtype, seed=0):
    sd = random_state_dict(cfg, seed=seed, dtype=dtype, device="cuda")
    return Qwen2Model(cfg, sd), sd


def prompts(n, length, vocab, seed=1):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab, (length,), generator=g).tolist() for _ in range(n)]


def first_divergence(a, b):
    return next((k for k in range(min(len(a), len(b))) if a[k] != b[k]), None)


def check_tokens_with_tie_rule(ours, ref, ref_logits, gap_limit, label):
    for i, (a, b) in enumerate(zip(ours, ref)):
        j = first_divergence(a, b)
        if j is None:
            continue
        top2 = ref_logits[i][j].float().topk(2).values
        gap = (top2[0] - top2[1]).item()
        print(f"{label}: request {i} diverges at token {j}, oracle top-2 gap {gap:.2e}")
        assert gap <= gap_limit, f"{label}: request {i} diverged at {j} with a top-2 gap of {gap}"


@pytest.mark.parametrize("cfg", [SMALL, SMALL128], ids=["hd64", "hd128"])
def test_fp32_mixed_step_matches_oracle(hiplib, cfg):
    from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
    model, sd = gpu_model(cfg, torch.float32)
    orc = OracleModel(cfg, sd)
    pool = PagedKVCache.from_token_budget(cfg, 4096, 16, "cuda", torch.float32)
    pool.allocator.shuffle_free(0)                          # fragmented blocks
    A, B, C, D = prompts(4, 64, cfg.vocab_size)
    A, B = A[:40], B[:52]
    tb, tc, td = BlockTable(16), BlockTable(16), BlockTable(16)
    ocache = {}
    for name, t, ids in (("B", tb, B[:30]), ("C", tc, C[:37]), ("D", td, D[:50])):
        t.reserve(len(ids) + 30, pool.allocator)
        model.forward_batch(torch.tensor(ids, device="cuda"), torch.arange(len(ids), device="cuda"),
                            [SeqInput(len(ids))], paged=pool,
                            slot_mapping=torch.tensor(t.slots(len(ids)), device="cuda"))
        t.commit(len(ids))
        ocache[name] = orc.new_cache(256)
        orc.step([(ocache[name], ids)])
    ta = BlockTable(16)
    ta.reserve(40, pool.allocator)
    tokens = A + B[30:] + [C[37], D[50]]
    positions = list(range(40)) + list(range(30, 52)) + [37, 50]
    slots = ta.slots(40) + tb.slots(22) + tc.slots(1) + td.slots(1)
    seqs = [SeqInput(40, ctx_len=0, block_table=torch.tensor(ta.blocks, device="cuda")),
            SeqInput(22, block_table=torch.tensor(tb.blocks, device="cuda"), ctx_len=30),
            SeqInput(1, ctx_len=37, use_kernel=True), SeqInput(1, ctx_len=50, use_kernel=True)]
    width = max(len(tc.blocks), len(td.blocks))
    meta = DecodeMeta(token_idx=torch.tensor([62, 63], device="cuda"),
                      block_tables=torch.tensor([t.blocks + [0] * (width - len(t.blocks)) for t in (tc, td)],
                                                dtype=torch.int32, device="cuda"),
                      context_lens=torch.tensor([38, 51], dtype=torch.int32, device="cuda"))
    out = model.forward_batch(torch.tensor(tokens, device="cuda"), torch.tensor(positions, device="cuda"), seqs,
                              logits="last", paged=pool, slot_mapping=torch.tensor(slots, device="cuda"),
                              decode_meta=meta).cpu()
    ref = orc.step([(orc.new_cache(256), A), (ocache["B"], B[30:]), (ocache["C"], [C[37]]),
                    (ocache["D"], [D[50]])])
    err = (out - ref).abs().max().item()
    print(f"fp32 mixed step ({cfg.head_dim}): max|logit diff| {err:.2e}")
    assert err < 1e-3


@pytest.mark.parametrize("cfg", [SMALL, SMALL128], ids=["hd64", "hd128"])
def test_bf16_mixed_step_chunk_kernel_matches_per_token_rows(hiplib, cfg, monkeypatch):
    """bf16 mixed step (fresh prefill + continuation chunk + decode rows): the chunked-prefill kernel path
    against the same step with every prefill token run as a decode row (the fp32 route, which the fp32
    gate above pins to the oracle), and both against the fp32 oracle on the same bf16 weights."""
    from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
    model, sd = gpu_model(cfg, torch.bfloat16, seed=3)
    orc = OracleModel(cfg, sd, dtype=torch.float32)
    A, B, C = prompts(3, 100, cfg.vocab_size, seed=4)

    def step(force_rows):
        pool = PagedKVCache.from_token_budget(cfg, 4096, 16, "cuda", torch.bfloat16)
        pool.allocator.shuffle_free(2)
        if force_rows:
            monkeypatch.setattr(model, "_prefill_meta",
                                lambda seqs, paged, sm, dtype: Qwen2Model._prefill_meta(model, seqs, paged, sm,
                                                                                        torch.float32))
        tb, tc = BlockTable(16), BlockTable(16)
        for t, ids in ((tb, B[:35]), (tc, C[:70])):
            t.reserve(len(ids) + 40, pool.allocator)
            model.forward_batch(torch.tensor(ids, device="cuda"), torch.arange(len(ids), device="cuda"),
                                [SeqInput(len(ids))], paged=pool,
                                slot_mapping=torch.tensor(t.slots(len(ids)), device="cuda"))
            t.commit(len(ids))
        ta = BlockTable(16)
        ta.reserve(83, pool.allocator)
        tokens = A[:83] + B[35:74] + [C[70]]
        positions = list(range(83)) + list(range(35, 74)) + [70]
        slots = ta.slots(83) + tb.slots(39) + tc.slots(1)
        seqs = [SeqInput(83, block_table=torch.tensor(ta.blocks, device="cuda")),
                SeqInput(39, block_table=torch.tensor(tb.blocks, device="cuda"), ctx_len=35),
                SeqInput(1, ctx_len=70, use_kernel=True)]
        meta = DecodeMeta(token_idx=torch.tensor([122], device="cuda"),
                          block_tables=torch.tensor([tc.blocks], dtype=torch.int32, device="cuda"),
                          context_lens=torch.tensor([71], dtype=torch.int32, device="cuda"))
        out = model.forward_batch(torch.tensor(tokens, device="cuda"), torch.tensor(positions, device="cuda"), seqs,
                                  logits="all", paged=pool, slot_mapping=torch.tensor(slots, device="cuda"),
                                  decode_meta=meta).float().cpu()
        monkeypatch.undo()
        return out

    chunks, rows = step(False), step(True)
    ends = [82, 121, 122]
    ref = orc.step([(orc.new_cache(256), A[:83]), (orc.new_cache(256), B[:74]), (orc.new_cache(256), C[:71])])
    d_paths = (chunks - rows).abs().max().item()
    d_oracle = (chunks[ends] - ref).abs().max().item()
    d_oracle_rows = (rows[ends] - ref).abs().max().item()
    print(f"bf16 mixed step ({cfg.head_dim}): chunks vs rows {d_paths:.3e}; vs oracle {d_oracle:.3e} "
          f"(rows path {d_oracle_rows:.3e})")
    assert d_paths <= 0.05
    assert d_oracle <= max(2 * d_oracle_rows, 0.05)


def test_fresh_prefill_without_table_reads_pages_off_the_slot_mapping(hiplib):
    """SeqInput(n) with no block table (the reference's prefill call shape) == the same with a table."""
    from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
    model, _ = gpu_model(SMALL, torch.float32)
    ids = prompts(1, 45, SMALL.vocab_size)[0]
    outs = []
    for with_table in (False, True):
        pool = PagedKVCache.from_token_budget(SMALL, 1024, 16, "cuda", torch.float32)
        pool.allocator.shuffle_free(1)
        t = BlockTable(16)
        t.reserve(45, pool.allocator)
        s = SeqInput(45, block_table=torch.tensor(t.blocks, device="cuda") if with_table else None)
        outs.append(model.forward_batch(torch.tensor(ids, device="cuda"), torch.arange(45, device="cuda"), [s],
                                        logits="all", paged=pool,
                                        slot_mapping=torch.tensor(t.slots(45), device="cuda")).cpu())
    assert torch.equal(outs[0], outs[1])


def make_engine(model, **kw):
    from nanoserve_amd.engine import LLMEngine
    args = dict(max_seq_len=512, max_num_seqs=8, batch_wait_s=0.0, kv_cache_tokens=16384)
    args.update(kw)
    return LLMEngine(model, [], **args)


def run_all(eng, reqs, waves=None, recorder=None):
    """Add requests (optionally in waves: (step, count)) and step until done; tokens per request. A
    LogitsRecorder, if given, collects each emitted token's logits."""
    outs, idx, steps = {}, {}, 0
    pending = list(waves) if waves else [(0, len(reqs))]
    while pending or eng.has_unfinished():
        while pending and steps >= pending[0][0]:
            _, end = pending.pop(0)
            for i in range(len(idx), end):
                p, n = reqs[i]
                idx[eng.add_request(p, n, ignore_eos=True)] = i
                outs[i] = []
        if recorder is not None:
            recorder.ids = idx
        step_out = eng.step()
        if recorder is not None:
            recorder.commit(step_out)
        for o in step_out:
            outs[idx[o.seq_id]].append(o.token)
        steps += 1
    return [outs[i] for i in range(len(reqs))]


def test_config1_greedy_tokens_identical_to_oracle_fp32(hiplib):
    """Qwen2.5-0.5B architecture, random init, fp32, batch 4, 128-token prompts,
    32 greedy steps, paged KV with 16-token blocks."""
    cfg = QWEN25_0_5B
    sd_cpu = random_state_dict(cfg, seed=0, dtype=torch.float32)
    orc = OracleModel(cfg, sd_cpu)
    ps = prompts(4, 128, cfg.vocab_size, seed=1)
    ref, ref_logits = orc.generate_greedy(ps, 32, return_logits=True)
    model = Qwen2Model(cfg, {k: v.to("cuda") for k, v in sd_cpu.items()})
    del sd_cpu
    eng = make_engine(model, max_num_batched_tokens=512)
    ours = run_all(eng, [(p, 32) for p in ps])
    same = sum(a == b for a, b in zip(ours, ref))
    print(f"config 1 fp32: {same}/4 token streams identical; graph steps {eng.stats['graph_steps']}")
    for i, (a, b) in enumerate(zip(ours, ref)):
        j = first_divergence(a, b)
        if j is not None:
            top2 = ref_logits[i][j].float().topk(2).values
            print(f"config 1 fp32: request {i} diverges at token {j}, oracle top-2 gap {(top2[0] - top2[1]).item():.3e}")
    assert eng.stats["graph_steps"] > 0
    assert ours == ref, "config 1: fp32 greedy streams must be identical for all 32 steps"
    golden = json.loads((Path(__file__).resolve().parent / "golden" / "config1_fp32_streams.json").read_text())
    assert golden["prompts"] == ps
    assert ours == golden["streams"], "config 1: streams differ from the reference engine's own (fixture)"
    assert eng.kv.num_free_blocks == eng.kv.pool.num_blocks - 1     # only the garbage block is held


def test_bf16_greedy_tokens_follow_the_oracle(hiplib):
    """bf16 engine (graphs on) against the fp32 oracle on the same bf16 weights, teacher-forced at every
    position with the shape's logit-error bound (tests/parity.py)."""
    cfg = SMALL128
    sd = random_state_dict(cfg, seed=2, dtype=torch.bfloat16)
    orc = OracleModel(cfg, sd, dtype=torch.float32)          # fp32 oracle on the same bf16 weights
    ps = prompts(6, 70, cfg.vocab_size, seed=3)
    model = Qwen2Model(cfg, {k: v.to("cuda") for k, v in sd.items()})
    eng = make_engine(model, max_num_batched_tokens=256)
    rec = LogitsRecorder(eng)
    ours = run_all(eng, [(p, 24) for p in ps], recorder=rec)
    assert eng.stats["graph_steps"] > 0
    check_streams("bf16 engine (vocab 2048, hd 128)", ps, ours, orc, delta_max=DELTA_SMALL128,
                  min_identical=len(ps) - 1, min_agree=0.98, ours_logits=rec.per_request(len(ps)))


def test_graph_step_bitwise_equals_eager_at_bucket_size(hiplib):
    from nanoserve_amd.hip_graphs import DecodeGraphRunner
    from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
    model, _ = gpu_model(SMALL128, torch.bfloat16)
    pool = PagedKVCache.from_token_budget(SMALL128, 8192, 16, "cuda", torch.bfloat16)
    runner = DecodeGraphRunner(model, pool, max_seq_len=1024, max_batch=8)
    tables = []
    for ids in prompts(4, 300, SMALL128.vocab_size, seed=4):
        ids = ids[:random.Random(len(tables)).randint(100, 300)]
        t = BlockTable(16)
        t.reserve(len(ids) + 8, pool.allocator)
        model.forward_batch(torch.tensor(ids, device="cuda"), torch.arange(len(ids), device="cuda"),
                            [SeqInput(len(ids))], paged=pool, slot_mapping=torch.tensor(t.slots(len(ids)), device="cuda"))
        t.commit(len(ids))
        tables.append(t)
    inp = dict(tokens=[42 + i for i in range(4)], positions=[t.num_tokens for t in tables],
               slots=[t.slots(1)[0] for t in tables], block_tables=[t.blocks for t in tables],
               context_lens=[t.num_tokens + 1 for t in tables])
    width = max(len(b) for b in inp["block_tables"])
    meta = DecodeMeta(token_idx=torch.arange(4, device="cuda"),
                      block_tables=torch.tensor([b + [0] * (width - len(b)) for b in inp["block_tables"]],
                                                dtype=torch.int32, device="cuda"),
                      context_lens=torch.tensor(inp["context_lens"], dtype=torch.int32, device="cuda"))
    ref = model.forward_batch(torch.tensor(inp["tokens"], device="cuda"), torch.tensor(inp["positions"], device="cuda"),
                              [SeqInput(1, ctx_len=t.num_tokens, use_kernel=True) for t in tables], logits="all",
                              paged=pool, slot_mapping=torch.tensor(inp["slots"], device="cuda"),
                              decode_meta=meta).clone()
    real = sorted({b for t in tables for b in t.blocks})
    assert runner.garbage_block not in real
    k_before = pool.k[:, real].clone()
    out = runner.run(**inp).clone()
    assert runner.captured_buckets == [4]
    assert out.shape == ref.shape and torch.equal(out, ref)
    # the same step with 3 rows in the 4-row graph: the padding row touches only the garbage block
    k_before = pool.k[:, real].clone()
    three = {k: v[:3] for k, v in inp.items()}
    runner.run(**three)
    changed = (pool.k[:, real] != k_before).any(dim=(0, 3, 4)).nonzero().tolist()
    assert len(changed) <= 3


def test_speculative_verify_rows_match_token_by_token_decode(hiplib):
    """Speculative verification through the decode graph (nanoserve/speculative.py:193-211): each of k + 1
    new tokens of a sequence is its own decode row with the sequence's block table and context length
    ctx + j + 1, all written and attended in one step. Its logits must equal decoding the same tokens one
    step at a time (eager decode rows), row for row, and pick the same argmax."""
    from nanoserve_amd.hip_graphs import DecodeGraphRunner
    from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
    model, _ = gpu_model(SMALL128, torch.bfloat16)
    pool = PagedKVCache.from_token_budget(SMALL128, 8192, 16, "cuda", torch.bfloat16)
    runner = DecodeGraphRunner(model, pool, max_seq_len=1024, max_batch=16)
    k1 = 4                                                   # k = 3 draft tokens + the last accepted one
    tables, ctxs = [], []
    for i, ids in enumerate(prompts(4, 300, SMALL128.vocab_size, seed=7)):
        ids = ids[:150 + 37 * i]
        t = BlockTable(16)
        t.reserve(len(ids) + k1, pool.allocator)
        model.forward_batch(torch.tensor(ids, device="cuda"), torch.arange(len(ids), device="cuda"),
                            [SeqInput(len(ids))], paged=pool, slot_mapping=torch.tensor(t.slots(len(ids)), device="cuda"))
        t.commit(len(ids))
        tables.append(t)
        ctxs.append(len(ids))
    drafts = [torch.randint(0, SMALL128.vocab_size, (k1,), generator=torch.Generator().manual_seed(30 + i)).tolist()
              for i in range(4)]
    slots = [t.slots(k1) for t in tables]                    # the k1 slots after each context
    # token by token: step j feeds token j of every sequence as one eager decode row each
    seq = torch.empty(4, k1, SMALL128.vocab_size, dtype=torch.bfloat16)
    width = max(len(t.blocks) for t in tables)
    bt = torch.tensor([t.blocks + [0] * (width - len(t.blocks)) for t in tables], dtype=torch.int32, device="cuda")
    for j in range(k1):
        meta = DecodeMeta(token_idx=torch.arange(4, device="cuda"), block_tables=bt,
                          context_lens=torch.tensor([c + j + 1 for c in ctxs], dtype=torch.int32, device="cuda"))
        lg = model.forward_batch(torch.tensor([d[j] for d in drafts], device="cuda"),
                                 torch.tensor([c + j for c in ctxs], device="cuda"),
                                 [SeqInput(1, ctx_len=c + j, use_kernel=True) for c in ctxs], logits="all", paged=pool,
                                 slot_mapping=torch.tensor([s[j] for s in slots], device="cuda"), decode_meta=meta)
        seq[:, j] = lg.cpu()
    # one verify step: 16 rows, rows of a sequence sharing its table
    out = runner.run(tokens=[x for d in drafts for x in d],
                     positions=[c + j for c in ctxs for j in range(k1)],
                     slots=[x for s in slots for x in s],
                     block_tables=[t.blocks for t in tables for _ in range(k1)],
                     context_lens=[c + j + 1 for c in ctxs for j in range(k1)]).cpu().view(4, k1, -1)
    diff = (out.float() - seq.float()).abs().max().item()
    print(f"verify rows vs token by token: max|diff| {diff:.3e}, bitwise equal {torch.equal(out, seq)}")
    assert diff <= 1e-2
    assert torch.equal(out.float().argmax(-1), seq.float().argmax(-1))


def oracle_streams(cfg, sd, reqs):
    """Greedy tokens (and logits) of each request generated alone by the CPU oracle."""
    orc = OracleModel(cfg, {k: v.cpu() for k, v in sd.items()})
    toks, logits = [], []
    for p, n in reqs:
        t, lg = orc.generate_greedy([p], n, return_logits=True)
        toks.append(t[0])
        logits.append(lg[0])
    return toks, logits


def test_engine_graphs_and_eager_steps_match_the_oracle(hiplib):
    model, sd = gpu_model(SMALL, torch.float32, seed=5)
    reqs = [(p, 20) for p in prompts(6, 90, SMALL.vocab_size, seed=6)]
    ref, ref_logits = oracle_streams(SMALL, sd, reqs)
    with_g = make_engine(model, max_num_batched_tokens=256)
    a = run_all(with_g, reqs, waves=((0, 3), (4, 6)))
    b = run_all(make_engine(model, max_num_batched_tokens=256, cuda_graphs=False), reqs, waves=((0, 3), (4, 6)))
    st = with_g.stats
    assert st["graph_steps"] > 0 and st["graph_steps"] < st["steps"]      # both graph and eager steps ran
    check_tokens_with_tie_rule(a, ref, ref_logits, TIE_GAP_FP32, "graphs")
    check_tokens_with_tie_rule(b, ref, ref_logits, TIE_GAP_FP32, "eager")


@pytest.mark.parametrize("budget", [48, 2048])
def test_fp32_chunked_prefill_and_preemption_match_the_oracle(hiplib, budget):
    model, sd = gpu_model(SMALL, torch.float32, seed=7)
    reqs = [(p[:random.Random(i).randint(30, 120)], 40) for i, p in enumerate(prompts(8, 120, SMALL.vocab_size, 8))]
    ref, ref_logits = oracle_streams(SMALL, sd, reqs)
    tight = make_engine(model, max_num_batched_tokens=budget, kv_cache_tokens=700)
    t_out = run_all(tight, reqs, waves=((0, 4), (1, 8)))
    st = tight.stats
    print(f"budget {budget}: preemptions {st['num_preemptions']}, partial chunks {st['prefill_chunks']}")
    assert st["num_preemptions"] > 0
    if budget == 48:
        assert st["prefill_chunks"] > 0
    check_tokens_with_tie_rule(t_out, ref, ref_logits, TIE_GAP_FP32, f"tight budget {budget}")
    assert tight.kv.num_free_blocks == tight.kv.pool.num_blocks - 1


def test_fp32_prefix_caching_matches_the_oracle(hiplib):
    model, sd = gpu_model(SMALL, torch.float32, seed=9)
    g = torch.Generator().manual_seed(10)
    system = torch.randint(0, SMALL.vocab_size, (100,), generator=g).tolist()
    reqs = [(system + torch.randint(0, SMALL.vocab_size, (n,), generator=g).tolist(), 12) for n in (5, 9, 21, 3, 30, 7)]
    ref, ref_logits = oracle_streams(SMALL, sd, reqs)
    cached = make_engine(model, max_num_batched_tokens=2048, prefix_caching=True)
    a = run_all(cached, reqs, waves=((0, 2), (6, 4), (12, 6)))
    st = cached.stats
    print(f"prefix hits {st['prefix_hit_tokens']} of {st['prefix_query_tokens']}")
    assert st["prefix_hit_tokens"] >= 0.3 * st["prefix_query_tokens"]
    check_tokens_with_tie_rule(a, ref, ref_logits, TIE_GAP_FP32, "prefix caching")
    assert cached.kv.num_free_blocks == cached.kv.pool.num_blocks - 1


def test_bf16_prefix_sharing_follows_the_oracle(hiplib):
    """BASELINE config 5 in small: bf16, one shared system prompt (several full blocks) + distinct suffixes,
    prefix caching on, requests admitted after the first has registered its blocks, so the others' decode
    rows read the first request's pages through their block tables; greedy streams against the fp32 oracle
    on the same bf16 weights, teacher-forced with the shape's logit-error bound, and no block leaks."""
    cfg = SMALL128
    sd = random_state_dict(cfg, seed=12, dtype=torch.bfloat16)
    orc = OracleModel(cfg, sd, dtype=torch.float32)
    g = torch.Generator().manual_seed(13)
    system = torch.randint(0, cfg.vocab_size, (96,), generator=g).tolist()
    ps = [system + torch.randint(0, cfg.vocab_size, (n,), generator=g).tolist() for n in (13, 20, 7, 31)]
    model = Qwen2Model(cfg, {k: v.to("cuda") for k, v in sd.items()})
    eng = make_engine(model, max_num_batched_tokens=256, prefix_caching=True)
    rec = LogitsRecorder(eng)
    ours = run_all(eng, [(p, 20) for p in ps], waves=((0, 1), (3, 4)), recorder=rec)
    st = eng.stats
    print(f"bf16 prefix sharing: hits {st['prefix_hit_tokens']} of {st['prefix_query_tokens']}")
    assert st["prefix_hit_tokens"] >= 3 * 96
    check_streams("bf16 prefix sharing (vocab 2048, hd 128)", ps, ours, orc, delta_max=DELTA_SMALL128,
                  min_identical=len(ps) - 1, min_agree=0.98, ours_logits=rec.per_request(len(ps)))
    assert eng.kv.num_free_blocks == eng.kv.pool.num_blocks - 1


def test_engine_rejects_the_oracle_only_backends(hiplib):
    from nanoserve_amd.engine import LLMEngine
    model, _ = gpu_model(SMALL, torch.float32)
    for kw in ({"attn_backend": "sdpa"}, {"fused_ops": False}, {"kv_cache": "contiguous"}):
        with pytest.raises(ValueError):
            LLMEngine(model, [], max_seq_len=256, kv_cache_tokens=1024, **kw)


def test_overlapped_host_staging_matches_plain_steps(hiplib):
    """Steady greedy decode stages the next step while the current one runs and relaunches the graph right
    after the wait. Every request's tokens and finish must equal the engine's with that off: requests
    finishing by length at different steps, one finishing on an EOS token, one aborted while a prelaunched
    step is in flight, and a request arriving mid-run (admitted at most one step later: the step already in
    flight when it arrives runs first). Until that arrival the outputs agree step for step."""
    model, _ = gpu_model(SMALL, torch.bfloat16, seed=7)
    ps = prompts(6, 40, SMALL.vocab_size, seed=8)

    def drive(overlap: bool, eos: list[int]):
        from nanoserve_amd.engine import LLMEngine
        eng = LLMEngine(model, eos, max_seq_len=256, max_num_seqs=8, batch_wait_s=0.0, kv_cache_tokens=8192)
        eng.overlap_host = overlap
        ids = [eng.add_request(p, n, ignore_eos=(i != 2)) for i, (p, n) in enumerate(zip(ps[:5], [30, 12, 40, 25, 33]))]
        log, prelaunched, steps = [], 0, 0
        while eng.has_unfinished():
            if steps == 9:
                eng.abort(ids[3])
            if steps == 15:
                ids.append(eng.add_request(ps[5], 10, ignore_eos=True))
            log.append([(o.seq_id, o.token, o.finished) for o in eng.step()])
            prelaunched += eng._inflight is not None
            steps += 1
        assert eng.kv.num_free_blocks == eng.kv.pool.num_blocks - 1 and not eng.sequences
        return log, prelaunched

    plain, _ = drive(False, [])
    # an EOS id request 2 produces at its 20th token (it alone does not ignore EOS)
    out2 = [t for step in plain for (sid, t, _) in step if sid == 2]
    eos = [out2[19]] if len(out2) > 19 and out2[19] not in out2[:19] else []
    plain, n0 = drive(False, eos)
    fast, n1 = drive(True, eos)
    assert n0 == 0 and n1 > 10
    assert fast[:15] == plain[:15]

    def streams(log):
        toks, fin = {}, {}
        for k, step in enumerate(log):
            for sid, t, f in step:
                toks.setdefault(sid, []).append(t)
                fin.setdefault(sid, (k, f)) if f else None
        return toks, fin
    (ta, fa), (tb, fb) = streams(fast), streams(plain)
    assert ta == tb and fa.keys() == fb.keys()
    assert all(0 <= fa[s][0] - fb[s][0] <= 1 for s in fa)


def test_polled_greedy_tokens_equal_the_stream_wait(hiplib, monkeypatch):
    """Decode graph steps hand their greedy tokens over by host polling of the pinned token buffer; with the
    poll window at zero every read falls back to a stream synchronisation. Both give the same steps."""
    from nanoserve_amd import hip_graphs
    from nanoserve_amd.engine import LLMEngine
    model, _ = gpu_model(SMALL, torch.bfloat16, seed=9)
    ps = prompts(5, 33, SMALL.vocab_size, seed=10)

    def drive():
        eng = LLMEngine(model, [], max_seq_len=256, max_num_seqs=8, batch_wait_s=0.0, kv_cache_tokens=8192)
        for p, n in zip(ps, [20, 7, 31, 16, 25]):
            eng.add_request(p, n, ignore_eos=True)
        log = []
        while eng.has_unfinished():
            log.append([(o.seq_id, o.token, o.finished) for o in eng.step()])
        assert eng.stats["graph_steps"] > 10
        return log

    polled = drive()
    monkeypatch.setattr(hip_graphs, "POLL_S", 0.0)
    assert drive() == polled


@pytest.mark.parametrize("cfg", [SMALL, SMALL128], ids=["hd64", "hd128"])
def test_single_sequence_forward_api(hiplib, cfg):
    """Qwen2Model.forward, the one-sequence API of nanoserve/model.py:364-367 (the reference's bf16 tie-rule
    test computes its logits through it, tests/test_llm_engine.py:82-83), on the paged path, fp32: a fresh
    prompt's last logits within 1e-3 of the oracle (tests/test_model.py:44-52), and prefill + one token at a
    time through a SequenceKVCache equal to the full forward's rows within 1e-4 (tests/test_kv_cache.py:52-68)."""
    from nanoserve_amd.kv_cache import SequenceKVCache
    model, sd = gpu_model(cfg, torch.float32, seed=11)
    ids = prompts(1, 70, cfg.vocab_size, seed=12)[0]
    seq = torch.tensor(ids, device="cuda")
    last = model.forward(seq, torch.arange(70, device="cuda"))
    assert last.shape == (1, cfg.vocab_size)
    orc = OracleModel(cfg, sd)
    ref = orc.step([(orc.new_cache(70), ids)])
    assert (last.cpu() - ref).abs().max().item() < 1e-3
    full = model.forward(seq, torch.arange(70, device="cuda"), logits="all")
    assert full.shape == (70, cfg.vocab_size) and torch.allclose(full[-1], last[0], atol=1e-5)
    cache = SequenceKVCache(cfg, 80, "cuda", torch.float32)
    model.forward(seq[:60], torch.arange(60, device="cuda"), cache)
    assert cache.length == 60
    for t in range(60, 70):
        step = model.forward(seq[t:t + 1], torch.tensor([t], device="cuda"), cache)
        assert (step[0] - full[t]).abs().max().item() < 1e-4, t
    assert cache.length == 70
    with pytest.raises(ValueError):
        model.forward(seq[:11], torch.arange(70, 81, device="cuda"), cache)

"""Mixed-step hipGraphs (prefill chunks + decode rows, attention included; the role of
nanoserve/cuda_graphs.py:151-259, PiecewiseGraphRunner):
  * the replay of a captured mixed step equals, bitwise, the eager forward of the same staged rows; at the
    BASELINE config-4 shape (a 1536-token chunk on 512 cached tokens + 16 decode rows, 2 layers of the 1.5B
    shape) it agrees with the unpadded eager step and with the fp32 oracle as the eager step does, and so does
    the same step run tight (unrecorded, its own rows + one padding row) under the default graph bound;
  * an engine whose steps mix chunked prefills with decoding rows gives the same greedy streams with the
    mixed graphs as with the eager forward, and actually replays them.
"""
import dataclasses

import pytest
import torch

from nanoserve_amd.model import QWEN25_1_5B, DecodeMeta, ModelConfig, Qwen2Model, SeqInput, random_state_dict
from oracle.model import OracleModel
from tests.parity import DELTA_SMALL, LogitsRecorder, check_streams

pytestmark = pytest.mark.gpu


def test_config4_mixed_graph_equals_eager_and_follows_the_oracle(hiplib):
    from nanoserve_amd.hip_graphs import MixedGraphRunner
    from nanoserve_amd.kv_cache import BlockTable, PagedKVCache
    from nanoserve_amd.kv_manager import StepBatch
    cfg = dataclasses.replace(QWEN25_1_5B, n_layers=2)
    sd = random_state_dict(cfg, seed=5, dtype=torch.bfloat16)
    model = Qwen2Model(cfg, {k: v.to("cuda") for k, v in sd.items()})
    g = torch.Generator().manual_seed(2)
    seq_a = torch.randint(0, cfg.vocab_size, (2048,), generator=g).tolist()
    ctxs = torch.randint(256, 2049, (16,), generator=g).tolist()
    decs = [torch.randint(0, cfg.vocab_size, (c + 1,), generator=g).tolist() for c in ctxs]
    pool = PagedKVCache.from_token_budget(cfg, 2048 + sum(ctxs) + 16 * 17 + 128, 16, "cuda", torch.bfloat16)
    pool.allocator.shuffle_free(7)
    garbage = pool.allocator.allocate()
    ta = BlockTable(16)
    ta.reserve(2048, pool.allocator)
    tabs = []
    for ids in [seq_a[:512]] + [d[:-1] for d in decs]:
        t = ta if not tabs else BlockTable(16)
        if tabs:
            t.reserve(len(ids) + 1, pool.allocator)
        model.forward_batch(torch.tensor(ids, device="cuda"), torch.arange(len(ids), device="cuda"),
                            [SeqInput(len(ids))], paged=pool, slot_mapping=torch.tensor(t.slots(len(ids)), device="cuda"))
        t.commit(len(ids))
        tabs.append(t)
    sb = StepBatch()
    sb.token_ids = seq_a[512:] + [d[-1] for d in decs]
    sb.positions = list(range(512, 2048)) + ctxs
    sb.slots = ta.slots(1536) + [t.slots(1)[0] for t in tabs[1:]]
    sb.seqs = [SeqInput(1536, ctx_len=512, block_table=ta.blocks)] + [SeqInput(1, ctx_len=c, use_kernel=True) for c in ctxs]
    sb.tables = [t.blocks for t in tabs]
    sb.dec_idx = list(range(1536, 1552))
    sb.dec_tables = [t.blocks for t in tabs[1:]]
    sb.dec_lens = [c + 1 for c in ctxs]
    runner = MixedGraphRunner(model, pool, 2048 + 16, 16, 2048, garbage, max_graph_rows=2048)
    assert runner.fits(sb)
    graph = runner.run(sb).float().cpu()
    greedy = runner.greedy_tokens(17)
    gr = runner.last
    print(f"mixed graph bucket {gr.N} rows (+1 padding), {gr.S} prefill entries, {gr.D} decode entries", flush=True)
    assert gr.N == 1664 and torch.isfinite(graph).all()
    assert greedy == graph.argmax(-1).tolist()

    # eager forward of exactly the staged rows: bitwise the replay
    tok, pos, slots, dec_idx, rows, info, dec_lens, pf_tab, dec_tab = gr._views(gr.dev_buf)
    eager_same = model.forward_batch(tok, pos, [SeqInput(gr.N + 1)], logits=rows, paged=pool, slot_mapping=slots,
                                     decode_meta=DecodeMeta(dec_idx, dec_tab, dec_lens),
                                     prefill_meta=("chunks", pf_tab, info, min(gr.N, gr.W * 16), gr.W * 16))[:17].float().cpu()
    assert torch.equal(graph, eager_same)

    # the unpadded eager step, and the fp32 oracle
    width = max(len(t.blocks) for t in tabs[1:])
    meta = DecodeMeta(token_idx=torch.arange(1536, 1552, device="cuda"),
                      block_tables=torch.tensor([t.blocks + [0] * (width - len(t.blocks)) for t in tabs[1:]],
                                                dtype=torch.int32, device="cuda"),
                      context_lens=torch.tensor(sb.dec_lens, dtype=torch.int32, device="cuda"))
    seqs = [SeqInput(1536, ctx_len=512, block_table=torch.tensor(ta.blocks, device="cuda"))] + sb.seqs[1:]
    eager = model.forward_batch(torch.tensor(sb.token_ids, device="cuda"), torch.tensor(sb.positions, device="cuda"),
                                seqs, logits="last", paged=pool, slot_mapping=torch.tensor(sb.slots, device="cuda"),
                                decode_meta=meta).float().cpu()
    orc = OracleModel(cfg, sd, dtype=torch.float32)
    ca = orc.new_cache(2048)
    orc.step([(ca, seq_a[:512])])
    cds = []
    for d in decs:
        c = orc.new_cache(len(d))
        orc.step([(c, d[:-1])])
        cds.append(c)
    ref = orc.step([(ca, seq_a[512:])] + [(c, [d[-1]]) for c, d in zip(cds, decs)])
    d_eager, d_graph_ref, d_eager_ref = ((graph - eager).abs().max().item(), (graph - ref).abs().max().item(),
                                         (eager - ref).abs().max().item())
    print(f"config 4 mixed graph: vs unpadded eager {d_eager:.3e}, vs oracle {d_graph_ref:.3e} "
          f"(eager vs oracle {d_eager_ref:.3e})")
    assert d_eager <= 0.05
    assert d_graph_ref <= max(2 * d_eager_ref, 0.05)

    # under the default 512-row graph bound the step is not recorded and runs tight: its 1552 rows + padding row
    # 1552 (the K/V it writes are the chunk's own, rewritten)
    tight_runner = MixedGraphRunner(model, pool, 2048 + 16, 16, 2048, garbage)
    tight = tight_runner.run(sb).float().cpu()
    tg = tight_runner.last
    assert tg.graph is None and tg.rows_run == 1553
    assert tight_runner.greedy_tokens(17) == tight.argmax(-1).tolist()
    d_tight, d_tight_ref = (tight - eager).abs().max().item(), (tight - ref).abs().max().item()
    print(f"config 4 tight staged step: vs unpadded eager {d_tight:.3e} (bitwise {torch.equal(tight, eager)}), "
          f"vs oracle {d_tight_ref:.3e}")
    assert d_tight <= 0.05
    assert d_tight_ref <= max(2 * d_eager_ref, 0.05)


SMALL = ModelConfig(vocab_size=2048, hidden_size=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64,
                    intermediate_size=512, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)


def test_engine_mixed_graphs_equal_eager_steps(hiplib):
    """Prompts of 150-700 tokens under a 256-token step budget arrive in two waves, so chunked prefills run
    beside decoding rows. Greedy streams with the mixed graphs equal those of an engine without graphs
    (which runs the same staged steps unrecorded), and both, like the unpadded eager forward, follow the fp32
    oracle teacher-forced at every position within the shape's logit-error bound (tests/parity.py)."""
    from nanoserve_amd.engine import LLMEngine
    sd = random_state_dict(SMALL, seed=3, dtype=torch.bfloat16)
    model = Qwen2Model(SMALL, {k: v.cuda() for k, v in sd.items()})
    g = torch.Generator().manual_seed(4)
    reqs = [(torch.randint(0, 2048, (int(torch.randint(150, 700, (1,), generator=g)),), generator=g).tolist(), 24)
            for _ in range(10)]

    def run(capture_first=False, **kw):
        eng = LLMEngine(model, [], max_seq_len=1024, max_num_seqs=8, batch_wait_s=0.0, max_num_batched_tokens=256,
                        kv_cache_tokens=16384, **kw)
        if capture_first:
            secs = eng.capture_graphs()
            st0 = eng.stats
            print(f"capture_graphs: {secs:.1f} s, decode buckets {st0['graph_buckets']}, mixed keys "
                  f"{st0['piecewise_buckets']}, mixed graphs {st0['piecewise_graph_bytes'] / 2**20:.1f} MiB device + "
                  f"{st0['piecewise_graph_host_bytes'] / 2**10:.0f} KiB pinned", flush=True)
        rec = LogitsRecorder(eng)
        ids, outs, steps = {}, {}, 0
        for i, (p, n) in enumerate(reqs[:5]):
            ids[eng.add_request(p, n, ignore_eos=True)] = i
        while eng.has_unfinished() or len(ids) < len(reqs):
            if steps == 6:
                for i in range(5, len(reqs)):
                    ids[eng.add_request(reqs[i][0], reqs[i][1], ignore_eos=True)] = i
            rec.ids = ids
            step_out = eng.step()
            rec.commit(step_out)
            for o in step_out:
                outs.setdefault(ids[o.seq_id], []).append(o.token)
            steps += 1
        assert eng.kv.num_free_blocks == eng.kv.pool.num_blocks - eng.executor.reserved_blocks
        return [outs[i] for i in range(len(reqs))], eng.stats, rec.per_request(len(reqs))

    graphed, st, lg_graphed = run()
    print(f"mixed-graph steps {st['piecewise_steps']} of {st['steps']}, buckets {st['piecewise_buckets']}", flush=True)
    assert st["piecewise_graphs"] and st["piecewise_steps"] > 0
    # every graph captured at start-up: the same streams, and no step captured anything
    upfront, stu, _ = run(capture_first=True)
    assert stu["graph_captures_in_run"] == 0 and stu["piecewise_steps"] == st["piecewise_steps"]
    assert set(st["piecewise_buckets"]) <= set(stu["piecewise_buckets"])
    assert stu["piecewise_graph_bytes"] > 0 and stu["piecewise_graph_host_bytes"] > 0
    assert upfront == graphed
    staged, st2, _ = run(cuda_graphs=False)
    assert st2["piecewise_steps"] == 0 and not st2["piecewise_graphs"]
    assert graphed == staged
    unpadded, st3, lg_unpadded = run(piecewise_graphs=False)
    assert st3["piecewise_steps"] == 0
    assert all(len(o) == 24 for o in graphed)
    orc = OracleModel(SMALL, sd, dtype=torch.float32)
    ps = [p for p, _ in reqs]
    for label, outs, lg in (("mixed graphs", graphed, lg_graphed), ("unpadded eager", unpadded, lg_unpadded)):
        check_streams(label, ps, outs, orc, delta_max=DELTA_SMALL, min_identical=len(reqs) - 1, min_agree=0.98,
                      ours_logits=lg)

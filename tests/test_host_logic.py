"""Known answers for the host integer layer on the CPU (no GPU, no model), run as data: each case is a
script of operations with the expected result of every step.

The expected values are the known answers of the reference's own tests (tests/test_paged_kv.py:14-91,
tests/test_prefix_cache.py:29-163, tests/test_scheduler.py:15-192, tests/test_chunked_prefill.py:44-72);
the step-by-step agreement with the reference's engine as a whole is pinned separately by
tests/test_host_traces.py.
"""
import pytest
import torch

from nanoserve_amd.kv_cache import BlockPool, BlockTable, NoFreeBlocks, PagedKVCache
from nanoserve_amd.kv_manager import PagedKVManager
from nanoserve_amd.model import QWEN25_0_5B, QWEN25_1_5B, QWEN25_3B, ModelConfig
from nanoserve_amd.scheduler import Scheduler, SeqStatus, Sequence

TINY = ModelConfig(vocab_size=10, hidden_size=8, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=3,
                   intermediate_size=16, rope_theta=10000.0, rms_norm_eps=1e-6, tie_word_embeddings=True)

# ------------------------------------------------------------------------------------ block pool scripts
# (name, pool kwargs, script). Ops: ("alloc", want id) | ("alloc!",) must raise | ("free", ids) |
# ("free!", ids) must raise | ("nfree", want) | ("table", name, tokens) reserve+commit+register a table |
# ("release", name) | ("lookup", tokens, max_blocks, want: list of (table name, block index) or ids) |
# ("pin", name, n) pin the first n blocks of a table | ("unpin", name, n) | ("parked", want count) |
# ("ref", name, i, want)
POOL_SCRIPTS = [
    ("ascending ids, then exhausted", dict(num_blocks=4), [
        ("alloc", 0), ("alloc", 1), ("alloc", 2), ("alloc", 3), ("nfree", 0), ("alloc!",),
        ("free", [1]), ("nfree", 1), ("alloc", 1)]),
    ("freed ids come back last in, first out", dict(num_blocks=8), [
        ("alloc", 0), ("alloc", 1), ("alloc", 2), ("alloc", 3), ("alloc", 4), ("free", [1, 3]),
        ("alloc", 3), ("alloc", 1), ("alloc", 5)]),
    ("double free", dict(num_blocks=2), [("alloc", 0), ("free", [0]), ("free!", [0])]),
    ("full blocks found by exact prefix", dict(num_blocks=16, block_size=4, prefix_caching=True), [
        ("table", "t", list(range(10))),
        ("lookup", list(range(10)), None, [("t", 0), ("t", 1)]),
        ("lookup", list(range(8)) + [99, 98], None, [("t", 0), ("t", 1)]),
        ("lookup", [0, 1, 2, 3, 9, 9, 9, 9], None, [("t", 0)]),
        ("lookup", [5, 1, 2, 3], None, []),
        ("lookup", list(range(10)), 1, [("t", 0)])]),
    ("equal tokens after a different prefix do not match", dict(num_blocks=16, block_size=4, prefix_caching=True), [
        ("table", "t", [1, 1, 1, 1, 7, 7, 7, 7]),
        ("lookup", [2, 2, 2, 2, 7, 7, 7, 7], None, []),
        ("lookup", [1, 1, 1, 1, 7, 7, 7, 7], None, [("t", 0), ("t", 1)])]),
    ("released cached blocks stay findable and count as free", dict(num_blocks=4, block_size=4, prefix_caching=True), [
        ("table", "t", list(range(8))), ("nfree", 2), ("keep", "t", "u"), ("release", "t"), ("nfree", 4),
        ("parked", 2), ("pin", "u", 2), ("parked", 0), ("nfree", 2), ("unpin", "u", 2), ("parked", 2)]),
    ("allocation evicts the block released longest ago", dict(num_blocks=2, block_size=4, prefix_caching=True), [
        ("table", "a", [1, 1, 1, 1]), ("table", "b", [2, 2, 2, 2]), ("keep", "a", "a0"),
        ("release", "a"), ("release", "b"), ("alloc_is", "a0", 0),
        ("lookup", [1, 1, 1, 1], None, []), ("lookup", [2, 2, 2, 2], None, [("b0", 0)]),
        ("alloc_any",), ("lookup", [2, 2, 2, 2], None, []), ("alloc!",)]),
    ("a prefix computed twice is cached once", dict(num_blocks=8, block_size=4, prefix_caching=True), [
        ("table", "a", list(range(8))), ("table", "b", list(range(8))),
        ("lookup", list(range(8)), None, [("a", 0), ("a", 1)]), ("release", "a"), ("release", "b"),
        ("nfree", 8), ("parked", 2)]),
    ("double free with prefix caching", dict(num_blocks=4, block_size=4, prefix_caching=True), [
        ("alloc", 0), ("free", [0]), ("free!", [0])]),
]


def run_pool_script(kwargs, script):
    pool = BlockPool(**kwargs)
    bs = pool.block_size
    tables, kept = {}, {}
    for op in script:
        kind = op[0]
        if kind == "alloc":
            assert pool.allocate() == op[1], op
        elif kind == "alloc!":
            with pytest.raises(NoFreeBlocks):
                pool.allocate()
        elif kind == "alloc_any":
            pool.allocate()
        elif kind == "alloc_is":
            assert pool.allocate() == kept[op[1]][op[2]]
        elif kind == "free":
            pool.free(op[1])
        elif kind == "free!":
            with pytest.raises(ValueError):
                pool.free(op[1])
        elif kind == "nfree":
            assert pool.num_free == op[1], op
        elif kind == "parked":
            assert pool.num_evictable == op[1], op
        elif kind == "table":
            t = BlockTable(bs)
            t.reserve(len(op[2]), pool)
            t.commit(len(op[2]))
            pool.register(t, op[2])
            tables[op[1]] = t
            kept[op[1] + "0"] = list(t.blocks)
        elif kind == "keep":
            kept[op[2]] = list(tables[op[1]].blocks)
        elif kind == "release":
            tables[op[1]].release(pool)
        elif kind == "lookup":
            want = [kept[n][i] if n in kept else tables[n].blocks[i] for n, i in op[3]]
            assert pool.lookup(op[1], op[2]) == want, op
        elif kind == "pin":
            pool.pin(kept[op[1]][:op[2]])
        elif kind == "unpin":
            pool.free(kept[op[1]][:op[2]])
        else:
            raise AssertionError(f"unknown op {kind}")
    return pool


@pytest.mark.parametrize("name,kwargs,script", POOL_SCRIPTS, ids=[c[0] for c in POOL_SCRIPTS])
def test_block_pool_script(name, kwargs, script):
    run_pool_script(kwargs, script)


def test_shared_prefix_is_refcounted_by_every_holder():
    """Config 5 in miniature: 32 requests pin one 4-block prefix; it returns to the parked set only when the
    last holder lets go."""
    pool = BlockPool(200, 4, prefix_caching=True)
    prefix = list(range(16))
    owner = BlockTable(4)
    owner.reserve(17, pool)
    owner.commit(17)
    pool.register(owner, prefix + [100])
    holders = []
    for r in range(32):
        hits = pool.lookup(prefix + [200 + r], max_blocks=len(prefix) // 4)
        assert hits == owner.blocks[:4]
        pool.pin(hits)
        holders.append(hits)
    assert [pool.refcount(b) for b in owner.blocks[:4]] == [33] * 4
    owner.release(pool)
    for h in holders[:-1]:
        pool.free(h)
    assert pool.num_evictable == 0 and [pool.refcount(b) for b in holders[0]] == [1] * 4
    pool.free(holders[-1])
    assert pool.num_evictable == 4 and pool.evictable() == holders[0][::-1]   # released tail first


# -------------------------------------------------------------------------------- tables, slots, sizing
@pytest.mark.parametrize("bs,n_tokens,seed", [(4, 5, 0), (16, 100, 1), (16, 1, 2), (4, 33, 3)])
def test_slot_formula_on_fragmented_tables(bs, n_tokens, seed):
    """slot(t) = table[t // bs] * bs + t % bs (kv_cache.py:225-228), from any committed offset."""
    pool = BlockPool(64, bs)
    pool.shuffle_free(seed)
    t = BlockTable(bs)
    t.reserve(n_tokens + 7, pool)
    assert len(t.blocks) == -(-(n_tokens + 7) // bs)
    for start in (0, n_tokens // 2, n_tokens):
        t.num_tokens = start
        assert t.slots(7) == [t.blocks[p // bs] * bs + p % bs for p in range(start, start + 7)]


def test_table_growth_truncate_rewind_release():
    pool = BlockPool(10, 4)
    t = BlockTable(4)
    steps = [  # (reserve n, commit n, blocks after)
        (5, 5, 2), (3, 3, 2), (1, 1, 3)]
    for r, c, nb in steps:
        t.reserve(r, pool)
        t.commit(c)
        assert len(t.blocks) == nb
    t.rewind(6)
    assert t.num_tokens == 6 and len(t.blocks) == 3
    with pytest.raises(ValueError):
        t.rewind(7)
    t.truncate(5, pool)
    assert t.num_tokens == 5 and len(t.blocks) == 2 and pool.num_free == 8
    t.release(pool)
    assert pool.num_free == 10 and t.blocks == [] and t.num_tokens == 0


def test_pool_write_and_gather_round_trip_with_fragmented_blocks():
    torch.manual_seed(0)
    pool = PagedKVCache(TINY, num_blocks=12, block_size=4, device="cpu", dtype=torch.float32)
    pool.allocator.shuffle_free(0)
    seqs = {name: (BlockTable(4), torch.randn(n, 2, 3), torch.randn(n, 2, 3)) for name, n in (("A", 7), ("B", 10))}
    for chunk in ((("A", 3), ("B", 10)), (("A", 4),)):
        slots, ks, vs = [], [], []
        for name, n in chunk:
            table, k, v = seqs[name]
            table.reserve(n, pool.allocator)
            slots += table.slots(n)
            ks.append(k[table.num_tokens:table.num_tokens + n])
            vs.append(v[table.num_tokens:table.num_tokens + n])
            table.commit(n)
        for layer in range(TINY.n_layers):
            pool.write(layer, torch.cat(ks), torch.cat(vs), torch.tensor(slots))
    for name, (table, k, v) in seqs.items():
        gk, gv = pool.gather(1, torch.tensor(table.blocks), table.num_tokens)
        assert torch.equal(gk[0].transpose(0, 1), k) and torch.equal(gv[0].transpose(0, 1), v)


@pytest.mark.parametrize("cfg,dtype,want", [(QWEN25_0_5B, torch.bfloat16, 12288), (QWEN25_1_5B, torch.bfloat16, 28672),
                                            (QWEN25_3B, torch.bfloat16, 36864), (TINY, torch.float32, 96)])
def test_kv_bytes_per_token(cfg, dtype, want):
    assert cfg.kv_bytes_per_token(dtype) == want          # 0.5B: tests/test_model.py:24


def test_pool_sizing_from_a_token_budget():
    pool = PagedKVCache.from_token_budget(TINY, num_tokens=33, block_size=16, device="cpu", dtype=torch.float32)
    assert pool.num_blocks == 3 and pool.reserved_bytes == 3 * 16 * 96
    assert PagedKVCache.tokens_for_bytes(TINY, pool.reserved_bytes, torch.float32) == 48


# ------------------------------------------------------------------------------------------- scheduling
def make_seq(i, prompt_len=4, max_new=8, t=0.0):
    return Sequence(i, list(range(prompt_len)), max_new, arrival_time=t)


def step_and_commit(s, out_token=1):
    """Schedule a step, commit every scheduled chunk and give finished prefills an output token; returns
    ([(seq_id, chunk)], admitted ids, ids that got a token)."""
    plan = s.schedule(now=0.0)
    got = []
    for x, n in zip(plan.scheduled, plan.chunks):
        if x.block_table is not None:
            x.block_table.commit(n)
        x.num_cached += n
        if x.num_cached == x.num_tokens:
            x.tokens.append(out_token)
            got.append(x.seq_id)
    return [(x.seq_id, n) for x, n in zip(plan.scheduled, plan.chunks)], [x.seq_id for x in plan.admitted], got


def scheduler(budget=100, max_seqs=8, kv_tokens=None, block_size=4, chunked=False, policy="continuous", wait=0.02):
    kv = None
    if kv_tokens is not None:
        kv = PagedKVManager(TINY, budget_tokens=kv_tokens, block_size=block_size, device="cpu", dtype=torch.float32)
    return Scheduler(policy, max_num_seqs=max_seqs, max_num_batched_tokens=budget, batch_wait_s=wait, kv=kv,
                     chunked_prefill=chunked)


# (name, scheduler kwargs, requests [(prompt_len, max_new)], expected per step [(scheduled, admitted)])
SCHEDULES = [
    ("continuous admits up to max_num_seqs", dict(max_seqs=2), [(4, 8)] * 3,
     [([(0, 4), (1, 4)], [0, 1]), ([(0, 1), (1, 1)], [])]),
    ("the token budget limits prefill admission", dict(budget=10), [(6, 8), (6, 8)],
     [([(0, 6)], [0]), ([(0, 1), (1, 6)], [1])]),
    ("first come first served never skips the head", dict(budget=10), [(6, 8), (9, 8), (2, 8)],
     [([(0, 6)], [0]), ([(0, 1), (1, 9)], [1]), ([(0, 1), (1, 1), (2, 2)], [2])]),
    ("a long prompt is prefilled in budget-sized chunks", dict(budget=10, kv_tokens=256, chunked=True), [(25, 4)],
     [([(0, 10)], [0]), ([(0, 10)], []), ([(0, 5)], []), ([(0, 1)], [])]),
    ("admission waits for free blocks", dict(kv_tokens=16), [(10, 2), (6, 2)],
     [([(0, 10)], [0]), ([(0, 1)], []), ([(0, 1)], [])]),
]


@pytest.mark.parametrize("name,kw,reqs,want", SCHEDULES, ids=[c[0] for c in SCHEDULES])
def test_schedule_table(name, kw, reqs, want):
    s = scheduler(**kw)
    for i, (p, n) in enumerate(reqs):
        s.add(make_seq(i, p, n))
    for k, (sched, adm) in enumerate(want):
        got, got_adm, _ = step_and_commit(s)
        assert (got, got_adm) == (sched, adm), f"step {k}"


def test_decodes_get_the_budget_first():
    """tests/test_chunked_prefill.py: a decode costs 1, the chunk takes the other 9 of a 10-token budget."""
    s = scheduler(budget=10, kv_tokens=256, chunked=True)
    s.add(make_seq(0, 4, 4))
    step_and_commit(s)
    s.add(make_seq(1, 25, 4))
    got, _, _ = step_and_commit(s)
    assert dict(got) == {0: 1, 1: 9}


def test_continuous_fills_a_freed_seat_on_the_very_next_step():
    s = scheduler(max_seqs=2)
    seqs = [make_seq(i) for i in range(3)]
    for x in seqs:
        s.add(x)
    step_and_commit(s)
    s.finish(seqs[0])
    got, adm, _ = step_and_commit(s)
    assert got == [(1, 1), (2, 4)] and adm == [2] and seqs[0].status is SeqStatus.FINISHED


def test_static_policy_admits_between_batches_only():
    s = scheduler(max_seqs=2, policy="static", wait=0.0)
    seqs = [make_seq(i) for i in range(3)]
    for x in seqs:
        s.add(x)
    assert step_and_commit(s)[1] == [0, 1]
    s.finish(seqs[0])
    assert step_and_commit(s)[:2] == ([(1, 1)], [])
    s.finish(seqs[1])
    assert step_and_commit(s)[1] == [2]
    late = scheduler(max_seqs=3, policy="static", wait=0.02)
    late.add(make_seq(0, t=1.0))
    late.add(make_seq(1, t=1.005))
    assert late.schedule(now=1.01).scheduled == []
    assert [x.seq_id for x in late.schedule(now=1.03).admitted] == [0, 1]


def test_preemption_evicts_the_newest_and_it_recomputes_everything():
    s = scheduler(kv_tokens=16)
    a, b = make_seq(0, 8), make_seq(1, 8)
    s.add(a)
    s.add(b)
    step_and_commit(s)
    assert s.kv.num_free_blocks == 0
    got, _, _ = step_and_commit(s)
    assert got == [(0, 1)] and s.num_preemptions == 1
    assert b.status is SeqStatus.WAITING and s.waiting[0] is b
    assert b.num_cached == 0 and b.block_table is None and b.output_ids == [1]
    assert b.step_tokens() == (list(range(8)) + [1], range(0, 9)) and b.step_cost == 9
    assert len(a.block_table.blocks) == 3


def test_decode_takes_a_new_block_only_at_a_block_boundary():
    s = scheduler(kv_tokens=32)
    a = make_seq(0, 7)
    s.add(a)
    for want in (2, 2, 3):
        step_and_commit(s)
        assert len(a.block_table.blocks) == want


@pytest.mark.parametrize("kw,prompt,max_new", [(dict(budget=10), 11, 4), (dict(kv_tokens=16), 10, 10)])
def test_requests_that_can_never_run_are_rejected_on_add(kw, prompt, max_new):
    with pytest.raises(ValueError):
        scheduler(**kw).add(make_seq(0, prompt, max_new))


def test_sequence_step_inputs():
    x = make_seq(0, 3)
    assert x.is_prefill and x.step_tokens() == ([0, 1, 2], range(0, 3))
    x.num_cached = 3
    x.tokens.append(99)
    assert not x.is_prefill and x.step_tokens() == ([99], range(3, 4))
    assert x.prompt_ids == [0, 1, 2] and x.output_ids == [99] and x.num_outputs == 1


def test_finishing_returns_every_block():
    s = scheduler(kv_tokens=32)
    a = make_seq(0, 9)
    s.add(a)
    step_and_commit(s)
    s.finish(a)
    assert s.kv.num_free_blocks == 8 and a.block_table is None and not s.has_unfinished()


# ---------------------------------------------------------------------------------------- step batches
def test_step_batch_of_a_mixed_step():
    kv = PagedKVManager(TINY, budget_tokens=256, block_size=4, device="cpu", dtype=torch.float32)
    s = Scheduler("continuous", max_num_seqs=8, max_num_batched_tokens=100, kv=kv)
    a, b = make_seq(0, 6), make_seq(1, 3)
    s.add(a)
    s.add(b)
    plan = s.schedule(0.0)
    sb = kv.batch(plan)
    assert sb.token_ids == [0, 1, 2, 3, 4, 5, 0, 1, 2] and sb.positions == [0, 1, 2, 3, 4, 5, 0, 1, 2]
    assert [x.ctx_len for x in sb.seqs] == [0, 0] and sb.n_prefill == 2 and not sb.dec_idx
    assert sb.seqs[0].block_table == a.block_table.blocks
    for x, n in zip(plan.scheduled, plan.chunks):
        kv.commit(x, n)
        x.num_cached += n
        x.tokens.append(9)
    plan = s.schedule(0.0)
    sb = kv.batch(plan)
    assert sb.pure_decode and sb.dec_idx == [0, 1] and sb.dec_lens == [7, 4]
    assert sb.slots == [a.block_table.blocks[1] * 4 + 2, b.block_table.blocks[0] * 4 + 3]
    meta = kv.decode_meta(sb)
    assert meta.all_rows and meta.context_lens.tolist() == [7, 4] and meta.block_tables.dtype == torch.int32
    assert meta.block_tables.tolist() == [a.block_table.blocks, b.block_table.blocks + [0]]
    assert kv.decode_meta(sb, width=5).block_tables.shape == (2, 5)


def test_prefix_hits_leave_one_token_to_compute():
    kv = PagedKVManager(TINY, budget_tokens=256, block_size=4, device="cpu", dtype=torch.float32, prefix_caching=True)
    a = make_seq(0, 12)
    kv.admit(a)
    kv.commit(a, 12)
    a.num_cached = 12
    b = make_seq(1, 12)
    kv.admit(b)
    assert b.num_cached == 8 and b.block_table.blocks[:2] == a.block_table.blocks[:2]   # (12 - 1) // 4 = 2
    assert kv.prefix_hit_tokens == 8 and kv.prefix_query_tokens == 24
    assert [kv.refcount(x) for x in a.block_table.blocks] == [2, 2, 1]

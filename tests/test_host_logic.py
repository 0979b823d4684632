"""Integer host logic of the decode loop on the CPU (no GPU, no model): block allocator, block tables,
pool sizing, prefix-caching allocator, scheduler policies, paged admission / preemption, chunked prefill.

The known answers are the reference's own (tests/test_paged_kv.py:14-91, tests/test_prefix_cache.py:29-90,
tests/test_scheduler.py:15-192, tests/test_chunked_prefill.py:44-72), restated against this package's API.
"""
import random

import pytest
import torch

from nanoserve_amd.kv_cache import BlockAllocator, BlockTable, NoFreeBlocks, PagedKVCache, PrefixCachingAllocator
from nanoserve_amd.kv_manager import PagedKVManager
from nanoserve_amd.model import ModelConfig
from nanoserve_amd.scheduler import Scheduler, SeqStatus, Sequence

TINY = ModelConfig(vocab_size=10, hidden_size=8, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=3,
                   intermediate_size=16, rope_theta=10000.0, rms_norm_eps=1e-6, tie_word_embeddings=True)
TINY1 = ModelConfig(vocab_size=10, hidden_size=8, n_layers=1, n_heads=2, n_kv_heads=1, head_dim=2,
                    intermediate_size=8, rope_theta=10000.0, rms_norm_eps=1e-6, tie_word_embeddings=True)


# ---------------------------------------------------------------------------------- allocator, tables, pool
def test_allocator_hands_out_every_block_once_then_raises():
    a = BlockAllocator(4)
    got = [a.allocate() for _ in range(4)]
    assert got == [0, 1, 2, 3] and a.num_free == 0        # ascending ids: tables are bit-exact with the reference
    with pytest.raises(NoFreeBlocks):
        a.allocate()
    a.free([got[1]])
    assert a.num_free == 1 and a.allocate() == got[1]


def test_allocator_reuses_freed_blocks_last_in_first_out():
    a = BlockAllocator(8)
    blocks = [a.allocate() for _ in range(5)]
    a.free([blocks[1], blocks[3]])
    assert a.allocate() == 3 and a.allocate() == 1 and a.allocate() == 5


def test_allocator_rejects_double_free():
    a = BlockAllocator(2)
    b = a.allocate()
    a.free([b])
    with pytest.raises(ValueError):
        a.free([b])


def test_block_table_grows_one_block_per_block_size_tokens():
    a = BlockAllocator(10)
    t = BlockTable(block_size=4)
    assert t.blocks_needed(5) == 2
    t.reserve(5, a)
    assert len(t.blocks) == 2
    assert t.slots(5) == [t.blocks[0] * 4 + i for i in range(4)] + [t.blocks[1] * 4]
    t.commit(5)
    assert t.blocks_needed(3) == 0
    t.reserve(3, a)
    t.commit(3)
    assert t.blocks_needed(1) == 1
    t.reserve(1, a)
    assert t.slots(1) == [t.blocks[2] * 4]
    t.commit(1)
    used = a.num_free
    t.release(a)
    assert a.num_free == used + 3 and t.blocks == [] and t.num_tokens == 0


def test_truncate_frees_blocks_past_the_new_length():
    a = BlockAllocator(10)
    t = BlockTable(block_size=4)
    t.reserve(10, a)
    t.commit(10)
    t.truncate(5, a)
    assert t.num_tokens == 5 and len(t.blocks) == 2 and a.num_free == 8


def test_slot_formula_on_fragmented_tables():
    """slot(t) = table[t // bs] * bs + t % bs for a shuffled free list (kv_cache.py:225-228)."""
    a = BlockAllocator(64)
    random.Random(0).shuffle(a._free)
    t = BlockTable(16)
    t.reserve(100, a)
    s = t.slots(100)
    assert s == [t.blocks[p // 16] * 16 + p % 16 for p in range(100)]
    t.commit(37)
    assert t.slots(5) == [t.blocks[p // 16] * 16 + p % 16 for p in range(37, 42)]


def test_pool_write_and_gather_round_trip_with_fragmented_blocks():
    torch.manual_seed(0)
    pool = PagedKVCache(TINY, num_blocks=12, block_size=4, device="cpu", dtype=torch.float32)
    random.Random(0).shuffle(pool.allocator._free)
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
        assert gk.shape == (1, 2, table.num_tokens, 3)
        assert torch.equal(gk[0].transpose(0, 1), k) and torch.equal(gv[0].transpose(0, 1), v)


def test_pool_sizing_from_a_token_budget():
    pool = PagedKVCache.from_token_budget(TINY, num_tokens=33, block_size=16, device="cpu", dtype=torch.float32)
    assert pool.num_blocks == 3
    assert pool.reserved_bytes == 3 * 16 * TINY.kv_bytes_per_token(torch.float32)
    assert PagedKVCache.tokens_for_bytes(TINY, pool.reserved_bytes, torch.float32) == 48


def test_kv_bytes_per_token_of_the_benchmark_shapes():
    from nanoserve_amd.model import QWEN25_0_5B, QWEN25_1_5B, QWEN25_3B
    assert QWEN25_0_5B.kv_bytes_per_token(torch.bfloat16) == 12288        # tests/test_model.py:24
    assert QWEN25_1_5B.kv_bytes_per_token(torch.bfloat16) == 28672
    assert QWEN25_3B.kv_bytes_per_token(torch.bfloat16) == 36864


# ------------------------------------------------------------------------------------------ prefix cache
BS = 4


def table_with(alloc, tokens):
    t = BlockTable(BS)
    t.reserve(len(tokens), alloc)
    t.commit(len(tokens))
    alloc.register(t, tokens)
    return t


def test_full_blocks_are_cached_and_found_by_exact_prefix():
    alloc = PrefixCachingAllocator(BlockAllocator(16), BS)
    toks = list(range(10))
    t = table_with(alloc, toks)
    assert alloc.lookup(toks) == t.blocks[:2]
    assert alloc.lookup(toks[:8] + [99, 98]) == t.blocks[:2]
    assert alloc.lookup([0, 1, 2, 3, 9, 9, 9, 9]) == t.blocks[:1]
    assert alloc.lookup([5, 1, 2, 3]) == []
    assert alloc.lookup(toks, max_blocks=1) == t.blocks[:1]


def test_same_tokens_after_a_different_prefix_do_not_match():
    alloc = PrefixCachingAllocator(BlockAllocator(16), BS)
    table_with(alloc, [1, 1, 1, 1, 7, 7, 7, 7])
    assert alloc.lookup([2, 2, 2, 2, 7, 7, 7, 7]) == []
    assert len(alloc.lookup([1, 1, 1, 1, 7, 7, 7, 7])) == 2


def test_freed_cached_blocks_are_evictable_and_reusable():
    alloc = PrefixCachingAllocator(BlockAllocator(4), BS)
    t = table_with(alloc, list(range(8)))
    assert alloc.num_free == 2
    t.release(alloc)
    assert alloc.num_free == 4 and alloc.num_evictable == 2
    hits = alloc.lookup(list(range(8)))
    alloc.pin(hits)
    assert alloc.num_evictable == 0 and alloc.num_free == 2
    alloc.free(hits)
    assert alloc.num_evictable == 2


def test_allocation_evicts_least_recently_freed_cached_block():
    alloc = PrefixCachingAllocator(BlockAllocator(2), BS)
    a = table_with(alloc, [1, 1, 1, 1])
    b = table_with(alloc, [2, 2, 2, 2])
    a_block = a.blocks[0]
    a.release(alloc)
    b.release(alloc)
    assert alloc.allocate() == a_block
    assert alloc.lookup([1, 1, 1, 1]) == [] and len(alloc.lookup([2, 2, 2, 2])) == 1
    alloc.allocate()
    assert alloc.lookup([2, 2, 2, 2]) == []
    with pytest.raises(NoFreeBlocks):
        alloc.allocate()


def test_duplicate_prefix_computed_twice_is_registered_once():
    alloc = PrefixCachingAllocator(BlockAllocator(8), BS)
    a = table_with(alloc, list(range(8)))
    b = table_with(alloc, list(range(8)))
    assert alloc.lookup(list(range(8))) == a.blocks
    a.release(alloc)
    b.release(alloc)
    assert alloc.num_free == 8 and alloc.num_evictable == 2


def test_double_free_is_detected():
    alloc = PrefixCachingAllocator(BlockAllocator(4), BS)
    blk = alloc.allocate()
    alloc.free([blk])
    with pytest.raises(ValueError):
        alloc.free([blk])


def test_shared_prefix_is_refcounted_across_many_requests():
    """Config-5 shape in miniature: one prefix pinned by 32 requests; blocks return to the LRU list only
    when the last holder frees them."""
    alloc = PrefixCachingAllocator(BlockAllocator(200), BS)
    prefix = list(range(16))                       # 4 full blocks
    owner = table_with(alloc, prefix + [100])
    holders = []
    for r in range(32):
        hits = alloc.lookup(prefix + [200 + r], max_blocks=(len(prefix)) // BS)
        assert hits == owner.blocks[:4]
        alloc.pin(hits)
        holders.append(hits)
    assert all(alloc.ref[b] == 33 for b in owner.blocks[:4])
    owner.release(alloc)
    for h in holders[:-1]:
        alloc.free(h)
    assert alloc.num_evictable == 0 and all(alloc.ref[b] == 1 for b in owner.blocks[:4])
    alloc.free(holders[-1])
    assert alloc.num_evictable == 4


# -------------------------------------------------------------------------------------------- scheduler
def seq(i, prompt_len=4, max_new=8, t=0.0):
    return Sequence(seq_id=i, prompt_ids=list(range(prompt_len)), max_new_tokens=max_new, arrival_time=t)


def ids(seqs):
    return [s.seq_id for s in seqs]


def test_continuous_admits_up_to_max_num_seqs():
    s = Scheduler("continuous", max_num_seqs=2, max_num_batched_tokens=100)
    for i in range(3):
        s.add(seq(i))
    out = s.schedule(now=0.0)
    assert ids(out.scheduled) == [0, 1] and ids(out.admitted) == [0, 1]
    assert [x.status for x in out.scheduled] == [SeqStatus.RUNNING] * 2
    assert ids(s.waiting) == [2]


def test_continuous_fills_a_freed_seat_on_the_very_next_step():
    s = Scheduler("continuous", max_num_seqs=2, max_num_batched_tokens=100)
    a, b, c = seq(0), seq(1), seq(2)
    for x in (a, b, c):
        s.add(x)
    s.schedule(now=0.0)
    a.output_ids.append(7); a.num_cached = 4
    b.output_ids.append(7); b.num_cached = 4
    s.finish(a)
    out = s.schedule(now=0.0)
    assert ids(out.scheduled) == [1, 2] and ids(out.admitted) == [2]
    assert a.status == SeqStatus.FINISHED


def test_token_budget_limits_prefill_admission():
    s = Scheduler("continuous", max_num_seqs=8, max_num_batched_tokens=10)
    s.add(seq(0, prompt_len=6))
    s.add(seq(1, prompt_len=6))
    out = s.schedule(now=0.0)
    assert ids(out.admitted) == [0]
    out.scheduled[0].output_ids.append(1); out.scheduled[0].num_cached = 6
    out = s.schedule(now=0.0)
    assert ids(out.admitted) == [1] and ids(out.scheduled) == [0, 1]


def test_first_come_first_served_never_skips_the_head_of_the_queue():
    s = Scheduler("continuous", max_num_seqs=8, max_num_batched_tokens=10)
    s.add(seq(0, prompt_len=6))
    s.add(seq(1, prompt_len=9))
    s.add(seq(2, prompt_len=2))
    assert ids(s.schedule(now=0.0).admitted) == [0]


def test_prompt_longer_than_the_token_budget_is_rejected_on_add():
    s = Scheduler("continuous", max_num_seqs=8, max_num_batched_tokens=10)
    with pytest.raises(ValueError):
        s.add(seq(0, prompt_len=11))


def test_static_never_admits_while_a_batch_is_running():
    s = Scheduler("static", max_num_seqs=2, max_num_batched_tokens=100, batch_wait_s=0.0)
    a, b, c = seq(0), seq(1), seq(2)
    for x in (a, b, c):
        s.add(x)
    assert ids(s.schedule(now=0.0).admitted) == [0, 1]
    a.output_ids.append(1); a.num_cached = 4
    b.output_ids.append(1); b.num_cached = 4
    s.finish(a)
    out = s.schedule(now=1.0)
    assert ids(out.scheduled) == [1] and out.admitted == []
    s.finish(b)
    assert ids(s.schedule(now=2.0).admitted) == [2]


def test_static_waits_for_a_full_batch_or_the_timeout():
    s = Scheduler("static", max_num_seqs=3, max_num_batched_tokens=100, batch_wait_s=0.02)
    s.add(seq(0, t=1.0))
    s.add(seq(1, t=1.005))
    assert s.schedule(now=1.01).scheduled == []
    assert ids(s.schedule(now=1.03).admitted) == [0, 1]


def test_step_inputs_prefill_then_decode():
    x = seq(0, prompt_len=3)
    assert x.is_prefill and x.step_tokens() == ([0, 1, 2], [0, 1, 2])
    x.num_cached = 3
    x.output_ids.append(99)
    assert not x.is_prefill and x.step_tokens() == ([99], [3])
    x.num_cached = 4
    x.output_ids.append(98)
    assert x.step_tokens() == ([98], [4])


def test_preempted_request_recomputes_prompt_plus_outputs():
    x = seq(0, prompt_len=3)
    x.output_ids += [7, 8]
    x.num_cached = 0
    assert x.is_prefill and x.step_tokens() == ([0, 1, 2, 7, 8], [0, 1, 2, 3, 4])
    assert x.step_cost == 5


def paged_scheduler(num_tokens, block_size=4, **kw):
    kv = PagedKVManager(TINY1, budget_tokens=num_tokens, block_size=block_size, device="cpu", dtype=torch.float32)
    return Scheduler("continuous", max_num_seqs=8, max_num_batched_tokens=100, kv=kv, **kw), kv


def run_step(s, now=0.0):
    out = s.schedule(now=now)
    for x in out.scheduled:
        n = len(x.step_tokens()[0])
        x.block_table.commit(n)
        x.num_cached += n
        x.output_ids.append(1)
    return out


def test_admission_waits_for_free_blocks():
    s, kv = paged_scheduler(16)
    s.add(seq(0, prompt_len=10, max_new=2))
    s.add(seq(1, prompt_len=6, max_new=2))
    out = run_step(s)
    assert ids(out.admitted) == [0] and kv.num_free_blocks == 1


def test_decode_takes_a_new_block_only_at_a_block_boundary():
    s, kv = paged_scheduler(32)
    a = seq(0, prompt_len=7)
    s.add(a)
    run_step(s)
    assert len(a.block_table.blocks) == 2
    run_step(s)
    assert len(a.block_table.blocks) == 2
    run_step(s)
    assert len(a.block_table.blocks) == 3


def test_preempts_the_most_recent_request_when_blocks_run_out():
    s, kv = paged_scheduler(16)
    a, b = seq(0, prompt_len=8), seq(1, prompt_len=8)
    s.add(a)
    s.add(b)
    run_step(s)
    assert kv.num_free_blocks == 0
    out = run_step(s)
    assert ids(out.scheduled) == [0] and s.num_preemptions == 1
    assert b.status == SeqStatus.WAITING and s.waiting[0] is b
    assert b.num_cached == 0 and b.block_table is None and b.output_ids == [1]
    assert len(a.block_table.blocks) == 3


def test_request_that_can_never_fit_is_rejected():
    s, kv = paged_scheduler(16)
    with pytest.raises(ValueError):
        s.add(seq(0, prompt_len=10, max_new=10))


def test_finishing_returns_all_blocks():
    s, kv = paged_scheduler(32)
    a = seq(0, prompt_len=9)
    s.add(a)
    run_step(s)
    s.finish(a)
    assert kv.num_free_blocks == 8 and a.block_table is None


def test_has_unfinished():
    s = Scheduler("continuous", max_num_seqs=1, max_num_batched_tokens=100)
    assert not s.has_unfinished()
    x = seq(0)
    s.add(x)
    assert s.has_unfinished()
    s.schedule(now=0.0)
    s.finish(x)
    assert not s.has_unfinished()


# --------------------------------------------------------------------------------------- chunked prefill
def sched(budget, pool_tokens=256):
    kv = PagedKVManager(TINY1, budget_tokens=pool_tokens, block_size=4, device="cpu", dtype=torch.float32)
    return Scheduler("continuous", max_num_seqs=8, max_num_batched_tokens=budget, kv=kv, chunked_prefill=True)


def fake_step(s):
    out = s.schedule(now=0.0)
    sampled = []
    for x, n in zip(out.scheduled, out.chunks):
        x.block_table.commit(n)
        x.num_cached += n
        if x.num_cached == x.num_tokens:
            x.output_ids.append(7)
            sampled.append(x.seq_id)
    return out, sampled


def test_long_prompt_is_prefilled_in_budget_sized_chunks():
    s = sched(budget=10)
    a = Sequence(seq_id=0, prompt_ids=list(range(25)), max_new_tokens=4)
    s.add(a)
    chunks = []
    for _ in range(3):
        out, sampled = fake_step(s)
        chunks.append(out.chunks[0])
        assert sampled == ([0] if len(chunks) == 3 else [])
    assert chunks == [10, 10, 5]
    assert a.step_tokens(1) == ([7], [25])


def test_decodes_get_the_budget_first():
    s = sched(budget=10)
    a = Sequence(seq_id=0, prompt_ids=list(range(4)), max_new_tokens=4)
    s.add(a)
    fake_step(s)
    b = Sequence(seq_id=1, prompt_ids=list(range(25)), max_new_tokens=4)
    s.add(b)
    out, _ = fake_step(s)
    assert dict(zip([x.seq_id for x in out.scheduled], out.chunks)) == {0: 1, 1: 9}


def test_without_chunking_long_prompts_are_still_rejected():
    kv = PagedKVManager(TINY1, budget_tokens=256, block_size=4, device="cpu", dtype=torch.float32)
    s = Scheduler("continuous", max_num_seqs=8, max_num_batched_tokens=10, kv=kv, chunked_prefill=False)
    with pytest.raises(ValueError):
        s.add(Sequence(seq_id=0, prompt_ids=list(range(25)), max_new_tokens=4))


# ----------------------------------------------------------------------------------- KV manager metadata
def test_decode_meta_and_slots_of_a_mixed_step():
    kv = PagedKVManager(TINY1, budget_tokens=256, block_size=4, device="cpu", dtype=torch.float32)
    a = Sequence(seq_id=0, prompt_ids=list(range(6)), max_new_tokens=4)
    b = Sequence(seq_id=1, prompt_ids=list(range(3)), max_new_tokens=4)
    for x in (a, b):
        kv.admit(x)
    kv.begin_step()
    sa, sb = kv.seq_input(a, 6), kv.seq_input(b, 3)
    for x, n in ((a, 6), (b, 3)):
        kv.commit(x, n)
        x.num_cached = n
        x.output_ids.append(9)
    assert not sa.use_kernel and sa.ctx_len == 0 and sa.block_table.tolist() == a.block_table.blocks
    kv.try_append(a)
    kv.try_append(b)
    kv.begin_step()
    ia, ib = kv.seq_input(a, 1), kv.seq_input(b, 1)
    assert ia.use_kernel and ib.use_kernel
    meta = kv.decode_meta()
    assert meta.token_idx.tolist() == [0, 1] and meta.all_rows
    assert meta.context_lens.tolist() == [7, 4]
    assert meta.block_tables.dtype == torch.int32
    assert meta.block_tables.tolist() == [a.block_table.blocks, b.block_table.blocks + [0]]
    slots, tables, lens = kv.graph_inputs()
    assert slots == [a.block_table.blocks[1] * 4 + 2, b.block_table.blocks[0] * 4 + 3] and lens == [7, 4]


def test_prefix_hits_leave_one_token_to_compute():
    kv = PagedKVManager(TINY1, budget_tokens=256, block_size=4, device="cpu", dtype=torch.float32,
                        prefix_caching=True)
    a = Sequence(seq_id=0, prompt_ids=list(range(12)), max_new_tokens=4)
    kv.admit(a)
    kv.commit(a, 12)
    a.num_cached = 12
    b = Sequence(seq_id=1, prompt_ids=list(range(12)), max_new_tokens=4)
    kv.admit(b)
    assert b.num_cached == 8 and b.block_table.blocks[:2] == a.block_table.blocks[:2]   # (12 - 1) // 4 = 2
    assert kv.prefix_hit_tokens == 8 and kv.prefix_query_tokens == 24

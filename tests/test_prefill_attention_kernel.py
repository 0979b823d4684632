"""HIP paged chunked-prefill attention kernel vs the CPU oracle (causal-offset mask + GQA + SDPA).

The contract is nanoserve/model.py:283-318: new token j of a sequence with ctx_len cached tokens sees keys
0 .. ctx_len + j (the explicit mask of :297-299 for a continuation, causal SDPA for a fresh prefill), with
the keys read from the sequence's pages as PagedKVCache.gather does (kv_cache.py:281-288). The oracle is
oracle/ops.py causal_offset_attention, itself pinned against an fp64 brute force in test_oracle_ops.py.
Tolerance: bf16 max|diff| <= 1e-2 against the fp32 oracle on the same bf16 inputs (the decode kernel's
bar, tests/test_paged_attention_kernel.py:47-64 of the reference). Inputs are drawn on the CPU with seeded
generators. Covered: fresh prefills and continuations across page and tile boundaries, head layouts of
the 0.5B / 1.5B / 3B models, several sequences in one launch among rows that belong to none (left
untouched), fragmented tables, NaN poison in unwritten slots and in pages past a sequence's end, and the
BASELINE config-4 chunk (1536 new tokens on a 512-token context, 1.5B heads).
"""
import pytest
import torch

from oracle.ops import causal_offset_attention
from tests.conftest import cpu_gen

pytestmark = pytest.mark.gpu

BS = 16


def make_seqs(specs, n_heads, n_kv, hd, seed=0, extra_blocks=4, width=None, gap=0):
    """specs = [(ctx_len, n_new)]. Returns q [N, H, D] (sequences back to back, `gap` unrelated rows before
    each), pools, tables, seq list [(q_start, T, ctx)] and the per-sequence contiguous k, v for the oracle."""
    g = cpu_gen(seed)
    pages = [-(-(c + t) // BS) for c, t in specs]
    num_blocks = sum(pages) + extra_blocks
    kpool = torch.randn(num_blocks, BS, n_kv, hd, generator=g).to(torch.bfloat16)
    vpool = torch.randn(num_blocks, BS, n_kv, hd, generator=g).to(torch.bfloat16)
    perm = torch.randperm(num_blocks, generator=g)
    W = width or max(pages)
    tables = torch.zeros(len(specs), W, dtype=torch.int32)
    seqs, ks, vs = [], [], []
    used, row = 0, 0
    for i, ((c, t), np_) in enumerate(zip(specs, pages)):
        tables[i, :np_] = perm[used:used + np_].int()
        used += np_
        blocks = tables[i, :np_].long()
        ks.append(kpool[blocks].reshape(-1, n_kv, hd)[:c + t])
        vs.append(vpool[blocks].reshape(-1, n_kv, hd)[:c + t])
        row += gap
        seqs.append((row, t, c))
        row += t
    q = torch.randn(row, n_heads, hd, generator=g).to(torch.bfloat16)
    return q, kpool, vpool, tables, seqs, ks, vs


def run(q, kpool, vpool, tables, seqs, scale, out=None):
    from nanoserve_amd.kernels.paged_attention import paged_attention_prefill, prefill_seq_info
    info = prefill_seq_info([s[0] for s in seqs], [s[1] for s in seqs], [s[2] for s in seqs], "cuda")
    o = paged_attention_prefill(q.cuda(), kpool.cuda(), vpool.cuda(), tables.cuda(), info,
                                max(s[1] for s in seqs), max(s[1] + s[2] for s in seqs), scale,
                                out=None if out is None else out.cuda())
    return o.cpu()


def check(out, q, seqs, ks, vs, scale, tol=1e-2):
    for (q0, t, c), k, v in zip(seqs, ks, vs):
        ref = causal_offset_attention(q[q0:q0 + t].float(), k.float(), v.float(), c, scale)
        got = out[q0:q0 + t].float()
        assert torch.isfinite(got).all()
        err = (got - ref).abs().max().item()
        assert err <= tol, f"ctx={c} T={t}: max|diff| {err}"


@pytest.mark.parametrize("n_heads,n_kv,hd", [(14, 2, 64), (12, 2, 128), (16, 2, 128)])
@pytest.mark.parametrize("T", [1, 15, 16, 17, 64, 65, 100, 257])
def test_fresh_prefill_matches_causal_sdpa(hiplib, n_heads, n_kv, hd, T):
    q, kp, vp, tables, seqs, ks, vs = make_seqs([(0, T)], n_heads, n_kv, hd, seed=T)
    out = run(q, kp, vp, tables, seqs, hd ** -0.5)
    check(out, q, seqs, ks, vs, hd ** -0.5)


@pytest.mark.parametrize("n_heads,n_kv,hd", [(14, 2, 64), (12, 2, 128)])
@pytest.mark.parametrize("ctx,T", [(1, 1), (5, 33), (16, 16), (17, 200), (100, 64), (512, 129), (700, 3)])
def test_continuation_chunk_matches_offset_mask(hiplib, n_heads, n_kv, hd, ctx, T):
    q, kp, vp, tables, seqs, ks, vs = make_seqs([(ctx, T)], n_heads, n_kv, hd, seed=ctx + 7 * T)
    out = run(q, kp, vp, tables, seqs, hd ** -0.5)
    check(out, q, seqs, ks, vs, hd ** -0.5)


def test_several_sequences_in_one_launch_leave_other_rows_untouched(hiplib):
    """Three sequences of different shapes between unrelated rows (e.g. a step's decode rows): each is
    exact against its own oracle, and the unrelated rows of `out` keep their sentinel."""
    specs = [(0, 70), (300, 5), (33, 130)]
    q, kp, vp, tables, seqs, ks, vs = make_seqs(specs, 12, 2, 128, seed=3, gap=3, width=40)
    sentinel = torch.full_like(q, 7.0)
    out = run(q, kp, vp, tables, seqs, 0.09, out=sentinel)
    check(out, q, seqs, ks, vs, 0.09)
    mine = torch.zeros(q.shape[0], dtype=torch.bool)
    for q0, t, _ in seqs:
        mine[q0:q0 + t] = True
    assert (out[~mine] == 7.0).all()


def test_unwritten_slots_and_pages_past_the_end_are_never_used(hiplib):
    """The unused tail of each sequence's last page is NaN, and every table entry past the sequence's pages
    points at a NaN block: a kernel that let either into the result would return NaN."""
    specs = [(40, 23), (0, 77), (500, 1)]
    q, kp, vp, tables, seqs, ks, vs = make_seqs(specs, 16, 2, 128, seed=11, extra_blocks=3, width=64)
    used = set(tables.flatten().tolist())
    poison = next(b for b in range(kp.shape[0]) if b not in used)
    kp[poison] = float("nan")
    vp[poison] = float("nan")
    for i, (c, t) in enumerate(specs):
        n = c + t
        nb = -(-n // BS)
        tables[i, nb:] = poison
        last = tables[i, nb - 1].item()
        kp[last, n - (nb - 1) * BS:] = float("nan")
        vp[last, n - (nb - 1) * BS:] = float("nan")
    out = run(q, kp, vp, tables, seqs, 128 ** -0.5)
    check(out, q, seqs, ks, vs, 128 ** -0.5)


def test_result_does_not_depend_on_block_placement(hiplib):
    """The same tokens under two different page permutations give identical bits."""
    specs = [(200, 90)]
    q, kp, vp, tables, seqs, ks, vs = make_seqs(specs, 12, 2, 128, seed=21, extra_blocks=30)
    out1 = run(q, kp, vp, tables, seqs, 0.1)
    g = cpu_gen(5)
    n_pages = -(-290 // BS)
    new_ids = torch.randperm(kp.shape[0], generator=g)[:n_pages]
    kp2, vp2 = torch.zeros_like(kp), torch.zeros_like(vp)
    kp2[new_ids] = kp[tables[0, :n_pages].long()]
    vp2[new_ids] = vp[tables[0, :n_pages].long()]
    tables2 = tables.clone()
    tables2[0, :n_pages] = new_ids.int()
    out2 = run(q, kp2, vp2, tables2, seqs, 0.1)
    assert torch.equal(out1, out2)


def test_config4_chunk(hiplib):
    """BASELINE config 4's prefill: one sequence, 1536 new tokens on 512 cached ones, 12/2 heads, hd 128."""
    q, kp, vp, tables, seqs, ks, vs = make_seqs([(512, 1536)], 12, 2, 128, seed=4)
    out = run(q, kp, vp, tables, seqs, 128 ** -0.5)
    check(out, q, seqs, ks, vs, 128 ** -0.5)


def test_rejects_unsupported_arguments(hiplib):
    from nanoserve_amd.kernels.paged_attention import paged_attention_prefill, prefill_seq_info
    q, kp, vp, tables, seqs, _, _ = make_seqs([(0, 20)], 12, 2, 128)
    info = prefill_seq_info([0], [20], [0], "cuda")
    with pytest.raises(RuntimeError, match="bf16 only"):
        paged_attention_prefill(q.float().cuda(), kp.float().cuda(), vp.float().cuda(), tables.cuda(), info, 20, 20, 0.1)
    q96 = torch.zeros(20, 12, 96, dtype=torch.bfloat16, device="cuda")
    kp96 = torch.zeros(kp.shape[0], BS, 2, 96, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="head_dim"):
        paged_attention_prefill(q96, kp96, kp96, tables.cuda(), info, 20, 20, 0.1)


def test_long_partition_refreshes_its_block_window(hiplib):
    """max_kv understated (here: n_new) gives one partition per tile; its 25 stages outrun the kernel's
    16-stage window of block ids, which is then refreshed mid-loop. Results must not change."""
    from nanoserve_amd.kernels.paged_attention import paged_attention_prefill, prefill_seq_info
    q, kp, vp, tables, seqs, ks, vs = make_seqs([(1500, 100)], 12, 2, 128, seed=31)
    info = prefill_seq_info([0], [100], [1500], "cuda")
    out = paged_attention_prefill(q.cuda(), kp.cuda(), vp.cuda(), tables.cuda(), info, 100, 100, 128 ** -0.5).cpu()
    check(out, q, seqs, ks, vs, 128 ** -0.5)


def test_one_workspace_serves_every_shape(hiplib):
    """Calls of different shapes (few tiles, then many sequences and tiles, then few again) share the
    wrapper's workspace: the counters sit in a fixed region no call's partials overlap, so every call
    matches the oracle and a repeat of itself."""
    for it, specs in enumerate([[(900, 40)], [(512, 200)] * 12 + [(3000, 64)], [(1200, 17), (0, 300)],
                                [(2500, 129)] * 3]):
        q, kp, vp, tables, seqs, ks, vs = make_seqs(specs, 12, 2, 128, seed=60 + it)
        print(f"prefill shared workspace call {it}: {len(specs)} sequences", flush=True)
        out = run(q, kp, vp, tables, seqs, 128 ** -0.5)
        check(out, q, seqs, ks, vs, 128 ** -0.5)
        assert torch.equal(out, run(q, kp, vp, tables, seqs, 128 ** -0.5))


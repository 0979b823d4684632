"""ns_paged_attn_mixed (a mixed step's attention in one launch) against the two launches it replaces.

nanoserve/model.py:277-318 attends a step's decode rows (one query per sequence, nanoserve/kernels/
paged_attention.py:85-105) and its prefill chunks (causal-offset mask) separately; here both kinds of
workgroups share one grid. The contract: the result equals ns_paged_attn_prefill over the chunk rows plus
ns_paged_attn_decode_rows over the decode rows, bitwise, rows belonging to neither keep their contents, and
the chunk rows also match the fp32 oracle (causal_offset_attention) within the bf16 tolerance of the prefill
tests. Cases: the 1.5B head layout (several KV heads, hd 128: each KV head a workgroup row), the 0.5B layout
(hd 64: whole 256-byte token rows), multi-partition chunks and decode rows, no decode rows, no chunks, and a
decode table too wide for the whole-row kernel (then the two are launched one after the other).
"""
import pytest
import torch

from oracle.ops import causal_offset_attention
from tests.conftest import cpu_gen

pytestmark = pytest.mark.gpu

BS = 16


def build(n_heads, n_kv, hd, chunks, dec_ctx, seed, dec_width=None):
    """chunks = [(ctx, T)] prefill chunks, dec_ctx = decode rows' context lengths. Rows of q: each chunk's T
    tokens, then the decode rows, scattered with a few unrelated rows between them."""
    g = cpu_gen(seed)
    pf_pages = [-(-(c + t) // BS) for c, t in chunks]
    dc_pages = [-(-c // BS) for c in dec_ctx]
    nb = sum(pf_pages) + sum(dc_pages) + 4
    kp = torch.randn(nb, BS, n_kv, hd, generator=g).to(torch.bfloat16)
    vp = torch.randn(nb, BS, n_kv, hd, generator=g).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=g).int()
    used = 0
    W = max(pf_pages) if pf_pages else 1
    pf_tab = torch.zeros(len(chunks), W, dtype=torch.int32)
    for i, n in enumerate(pf_pages):
        pf_tab[i, :n] = perm[used:used + n]
        used += n
    DW = dec_width or (max(dc_pages) if dc_pages else 1)
    dc_tab = torch.zeros(len(dec_ctx), DW, dtype=torch.int32)
    for i, n in enumerate(dc_pages):
        dc_tab[i, :n] = perm[used:used + n]
        used += n
    info, row = [], 2
    for c, t in chunks:
        info.append([row, t, c, 0])
        row += t + 1
    rows = []
    for _ in dec_ctx:
        rows.append(row)
        row += 2
    N = row + 3
    q = torch.randn(N, n_heads, hd, generator=g).to(torch.bfloat16)
    return q, kp, vp, pf_tab, torch.tensor(info, dtype=torch.int32).reshape(-1, 4), dc_tab, \
        torch.tensor(dec_ctx, dtype=torch.int32), torch.tensor(rows, dtype=torch.int64)


def both_ways(n_heads, n_kv, hd, chunks, dec_ctx, seed, dec_width=None):
    from nanoserve_amd.kernels.paged_attention import (paged_attention_decode_rows, paged_attention_mixed,
                                                       paged_attention_prefill)
    q, kp, vp, pf_tab, info, dc_tab, lens, rows = build(n_heads, n_kv, hd, chunks, dec_ctx, seed, dec_width)
    q, kp, vp = q.cuda(), kp.cuda(), vp.cuda()
    pf_tab, info, dc_tab, lens, rows = pf_tab.cuda(), info.cuda(), dc_tab.cuda(), lens.cuda(), rows.cuda()
    max_new = max((t for _, t in chunks), default=0)
    max_kv = max((c + t for c, t in chunks), default=0)
    scale = hd ** -0.5
    sentinel = torch.full_like(q, 7.0)
    ref = sentinel.clone()
    if dec_ctx:
        paged_attention_decode_rows(q, kp, vp, dc_tab, lens, rows, scale, ref)
    if chunks:
        paged_attention_prefill(q, kp, vp, pf_tab, info, max_new, max_kv, scale, out=ref)
    got = sentinel.clone()
    print(f"mixed launch: heads {n_heads}/{n_kv} hd {hd} chunks {chunks} decode rows {len(dec_ctx)}", flush=True)
    paged_attention_mixed(q, kp, vp, pf_tab, info, max_new, max_kv, dc_tab, lens, rows, scale, got)
    torch.cuda.synchronize()
    return q.cpu(), kp.cpu(), vp.cpu(), pf_tab.cpu(), info.cpu(), ref.cpu(), got.cpu(), sentinel.cpu(), scale


@pytest.mark.parametrize("n_heads,n_kv,hd", [(12, 2, 128), (14, 2, 64), (16, 2, 128)])
@pytest.mark.parametrize("chunks,dec_ctx", [
    ([(512, 300)], [300, 1200, 2000, 17, 700]),      # multi-partition chunk tiles and decode rows
    ([(0, 40), (100, 129)], [1, 16, 33]),
    ([(1500, 64)], [4000, 90]),
])
def test_mixed_launch_equals_the_two_launches(hiplib, n_heads, n_kv, hd, chunks, dec_ctx):
    q, kp, vp, pf_tab, info, ref, got, sentinel, scale = both_ways(n_heads, n_kv, hd, chunks, dec_ctx, seed=hd + len(chunks))
    assert torch.equal(got, ref)
    # the chunk rows against the oracle, too
    for s, (c, t) in enumerate(chunks):
        q0 = int(info[s, 0])
        n = -(-(c + t) // BS)
        blocks = pf_tab[s, :n].long()
        k = kp[blocks].reshape(-1, n_kv, hd)[:c + t].float()
        v = vp[blocks].reshape(-1, n_kv, hd)[:c + t].float()
        o = causal_offset_attention(q[q0:q0 + t].float(), k, v, c, scale)
        assert (got[q0:q0 + t].float() - o).abs().max().item() <= 1e-2
    # rows that are neither chunk nor decode rows keep the sentinel (the two-launch reference never writes them)
    assert (ref == 7.0).all(-1).all(-1).sum() == q.shape[0] - sum(t for _, t in chunks) - len(dec_ctx)


@pytest.mark.parametrize("chunks,dec_ctx,dec_width", [
    ([(200, 90)], [], None),          # no decode rows: the prefill alone
    ([], [300, 40, 1000], None),      # no chunks: the decode rows alone
    ([(64, 100)], [50, 900], 1100),   # a decode table of 1100 pages: the per-head kernel, two launches
])
def test_mixed_launch_degenerate_cases(hiplib, chunks, dec_ctx, dec_width):
    _, _, _, _, _, ref, got, sentinel, _ = both_ways(12, 2, 128, chunks, dec_ctx, seed=5, dec_width=dec_width)
    assert torch.equal(got, ref)
    untouched = (ref == 7.0).all(-1).all(-1)
    assert torch.equal(got[untouched], sentinel[untouched])


def test_repeated_mixed_launches_leave_the_workspaces_clean(hiplib):
    """Counters of both merges are back at zero after each call: the same call twice, and a different shape in
    between, give identical results."""
    a = both_ways(12, 2, 128, [(512, 300)], [1200, 2000], seed=9)
    both_ways(16, 2, 128, [(100, 500), (1000, 64)], [300] * 7, seed=10)
    b = both_ways(12, 2, 128, [(512, 300)], [1200, 2000], seed=9)
    assert torch.equal(a[6], b[6]) and torch.equal(a[6], a[5])

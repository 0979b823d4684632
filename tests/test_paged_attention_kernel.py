"""HIP paged-attention decode kernel vs the CPU oracle (gather + SDPA, oracle/ops.py).

Procedure and tolerances follow the reference's tests/test_paged_attention_kernel.py:21-73: head layouts of
Qwen2.5-0.5B / 1.5B / 3B, context lengths {1, 15, 16, 17, 100, 333, 700}, fragmented random-permutation
block tables; fp32 max|diff| <= 1e-5; bf16 max|diff| <= 1e-2 against the fp32 oracle on the same bf16
inputs; ctx=1 returns that token's value for every head of the group. Inputs are drawn on the CPU with a
seeded generator so the oracle and the GPU see identical values. Added: the BASELINE config-2 shape (B=32,
ctx U[512, 4096], 64k-block pool), split-K state carried across calls (counters back at zero, merge words
of earlier calls never taken), NaN poison in padding table entries and past-ctx tokens, and hipGraph replay
against eager calls.
"""
import math

import pytest
import torch

from oracle.ops import paged_attention_reference
from tests.conftest import cpu_gen

pytestmark = pytest.mark.gpu

CONFIGS = [(14, 2, 64), (12, 2, 128), (16, 2, 128)]
CTX_LENS = [1, 15, 16, 17, 100, 333, 700]


def make_case(n_heads, n_kv, hd, ctx_lens, dtype, block_size=16, seed=0, extra_blocks=5, width=None):
    g = cpu_gen(seed)
    num_blocks = sum(-(-L // block_size) for L in ctx_lens) + extra_blocks
    k = torch.randn(num_blocks, block_size, n_kv, hd, generator=g).to(dtype)
    v = torch.randn(num_blocks, block_size, n_kv, hd, generator=g).to(dtype)
    q = torch.randn(len(ctx_lens), n_heads, hd, generator=g).to(dtype)
    perm = torch.randperm(num_blocks, generator=g)
    max_blocks = width or max(-(-L // block_size) for L in ctx_lens)
    tables = torch.zeros(len(ctx_lens), max_blocks, dtype=torch.int32)
    used = 0
    for i, L in enumerate(ctx_lens):
        nb = -(-L // block_size)
        tables[i, :nb] = perm[used:used + nb].int()
        used += nb
    lens = torch.tensor(ctx_lens, dtype=torch.int32)
    return q, k, v, tables, lens


def run(q, k, v, tables, lens, scale):
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    out = paged_attention_decode(q.cuda(), k.cuda(), v.cuda(), tables.cuda(), lens.cuda(), scale)
    return out.cpu()


@pytest.mark.parametrize("n_heads,n_kv,hd", CONFIGS)
def test_fp32_matches_reference(hiplib, n_heads, n_kv, hd):
    q, k, v, tables, lens = make_case(n_heads, n_kv, hd, CTX_LENS, torch.float32)
    scale = hd ** -0.5
    out = run(q, k, v, tables, lens, scale)
    ref = paged_attention_reference(q, k, v, tables, lens, scale)
    assert (out - ref).abs().max().item() <= 1e-5


@pytest.mark.parametrize("n_heads,n_kv,hd", CONFIGS)
def test_bf16_matches_reference(hiplib, n_heads, n_kv, hd):
    q, k, v, tables, lens = make_case(n_heads, n_kv, hd, CTX_LENS, torch.bfloat16)
    scale = hd ** -0.5
    out = run(q, k, v, tables, lens, scale).float()
    ref = paged_attention_reference(q.float(), k.float(), v.float(), tables, lens, scale)
    err = (out - ref).abs().max().item()
    print(f"bf16 ({n_heads},{n_kv},{hd}) max|diff| vs fp32 oracle = {err:.2e}")
    assert err <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_single_request_single_token(hiplib, dtype):
    q, k, v, tables, lens = make_case(14, 2, 64, [1], dtype)
    out = run(q, k, v, tables, lens, 0.125)
    blk = tables[0, 0].long()
    expected = v[blk, 0].repeat_interleave(7, dim=0)     # one key => weight 1 => that key's value
    assert torch.allclose(out[0].float(), expected.float(), atol=1e-6)


@pytest.mark.parametrize("n_heads,n_kv,hd", [(14, 2, 64), (12, 2, 128)])
def test_config2_shape_split_k(hiplib, n_heads, n_kv, hd):
    """BASELINE config 2 (B=32, ctx U[512, 4096], 16-token pages in a 64k-block pool, table width 256),
    scaled to hd 128 too; every row spans several partitions, so the in-kernel merge is exercised."""
    g = cpu_gen(2)
    ctx = torch.randint(512, 4097, (32,), generator=g).tolist()
    q, k, v, tables, lens = make_case(n_heads, n_kv, hd, ctx, torch.bfloat16, seed=3, extra_blocks=64,
                                      width=256)
    scale = hd ** -0.5
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    dq, dk, dv, dt, dl = q.cuda(), k.cuda(), v.cuda(), tables.cuda(), lens.cuda()
    out1 = paged_attention_decode(dq, dk, dv, dt, dl, scale).cpu()
    out2 = paged_attention_decode(dq, dk, dv, dt, dl, scale).cpu()     # counters must have reset to 0
    ref = paged_attention_reference(q.float(), k.float(), v.float(), tables, lens, scale)
    err = (out1.float() - ref).abs().max().item()
    print(f"config-2 shape ({n_heads},{n_kv},{hd}) max|diff| = {err:.2e}")
    assert err <= 1e-2
    assert torch.equal(out1, out2)


@pytest.mark.parametrize("n_heads,n_kv,hd", [(12, 2, 128), (14, 2, 64)])
def test_result_does_not_depend_on_the_table_width(hiplib, n_heads, n_kv, hd):
    """BASELINE config 3's rows (contexts 1025 .. 1152) in tables 73 pages wide (the graph runner's width
    for max_seq_len 1168) and 80 and 256 pages wide (other callers pad to other widths): a row's
    partitions are fixed 32-page runs of its own pages, so all three give bitwise the same output. Contexts
    sit on and next to the partition boundaries (512 / 1024 tokens), inside the last page and at the full
    width, and the output is checked against the oracle."""
    ctx = [1, 16, 17, 511, 512, 513, 1023, 1024, 1025, 1056, 1100, 1151, 1152, 1160, 1168]
    ctx = ctx + [1025 + 9 * i for i in range(16)]
    q, k, v, tables, lens = make_case(n_heads, n_kv, hd, ctx, torch.bfloat16, seed=31, extra_blocks=16, width=73)
    scale = hd ** -0.5
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    dq, dk, dv, dl = q.cuda(), k.cuda(), v.cuda(), lens.cuda()
    outs = []
    for W in (73, 80, 256):
        t = torch.zeros(len(ctx), W, dtype=torch.int32)
        t[:, :min(W, 73)] = tables[:, :min(W, 73)]
        outs.append(paged_attention_decode(dq, dk, dv, t.cuda(), dl, scale).cpu())
    ref = paged_attention_reference(q.float(), k.float(), v.float(), tables, lens, scale)
    err = (outs[0].float() - ref).abs().max().item()
    print(f"config-3 rows ({n_heads},{n_kv},{hd}) max|diff| = {err:.2e}")
    assert err <= 1e-2
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


def test_one_workspace_serves_every_shape(hiplib):
    """A split-K workspace shared by calls of different shapes on one stream (a few rows, then many rows,
    then the per-head kernel, then a few rows again): the arrival counters live in a fixed region that no
    call's partials overlap, so every call equals the same call on a fresh workspace."""
    from nanoserve_amd import _lib
    L = _lib.lib()
    g = cpu_gen(23)
    shared = torch.zeros(64 << 20, dtype=torch.uint8, device="cuda")
    for it, (B, nh, nkv, hd, W, mx) in enumerate([(3, 14, 2, 64, 256, 4096), (200, 14, 2, 64, 256, 4096),
                                                  (20, 12, 2, 128, 1100, 17000), (5, 12, 2, 128, 73, 1168),
                                                  (128, 12, 2, 128, 73, 1168)]):
        ctx = torch.randint(1, mx + 1, (B,), generator=g).tolist()
        q, k, v, tables, lens = make_case(nh, nkv, hd, ctx, torch.bfloat16, seed=40 + it, extra_blocks=4, width=W)
        dq, dk, dv, dt, dl = q.cuda(), k.cuda(), v.cuda(), tables.cuda(), lens.cuda()
        outs = []
        for ws in (shared, torch.zeros_like(shared)):
            out = torch.full_like(dq, float("nan"))
            _lib.check(L.ns_paged_attn_decode(
                dq.data_ptr(), dq.stride(0), dq.stride(1), dk.data_ptr(), dv.data_ptr(), dk.stride(0), dk.stride(1),
                dk.stride(2), dt.data_ptr(), dt.stride(0), dl.data_ptr(), out.data_ptr(), out.stride(0),
                out.stride(1), B, nh, nkv, hd, 16, W, dk.shape[0], hd ** -0.5, 1, ws.data_ptr(), ws.numel(),
                _lib.stream_of(dq)), "decode")
            outs.append(out.cpu())
        print(f"shared workspace call {it}: B={B} width {W}", flush=True)
        assert torch.equal(outs[0], outs[1]), f"call {it}: shared workspace differs from a fresh one"
        if it in (0, 3):
            ref = paged_attention_reference(q.float(), k.float(), v.float(), tables, lens, hd ** -0.5)
            assert (outs[0].float() - ref).abs().max().item() <= 1e-2


def test_merge_words_of_earlier_calls_are_never_taken(hiplib):
    """Several calls of one shape share the split-K workspace while each row's partition count changes
    (1 .. 8 partitions of 32 pages, table width 256): a merger must fold only this call's partials, never
    words an earlier call left in the same slots. Every call is checked against the oracle and against a
    second call with the same inputs."""
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    B, W, nh, nkv, hd = 8, 256, 14, 2, 64
    g = cpu_gen(21)
    q, k, v, _, _ = make_case(nh, nkv, hd, [4096] * B, torch.bfloat16, seed=21, extra_blocks=8, width=W)
    dk, dv = k.cuda(), v.cuda()
    schedule = [[4096, 600, 1, 2000, 513, 4000, 100, 3000],     # partitions 8 2 1 4 2 8 1 6
                [300, 4096, 2048, 1, 512, 4096, 700, 1000],     #            1 8 4 1 1 8 2 2
                [4096, 513, 2049, 3000, 4096, 1, 4096, 4096]]   #            8 2 5 6 8 1 8 8
    for it, ctx in enumerate(schedule + [torch.randint(1, W * 16 + 1, (B,), generator=g).tolist()]):
        qq = torch.randn(B, nh, hd, generator=g).to(torch.bfloat16)
        perm = torch.randperm(k.shape[0], generator=g)[:B * W].view(B, W).int()
        lens = torch.tensor(ctx, dtype=torch.int32)
        out1 = paged_attention_decode(qq.cuda(), dk, dv, perm.cuda(), lens.cuda(), hd ** -0.5).cpu()
        out2 = paged_attention_decode(qq.cuda(), dk, dv, perm.cuda(), lens.cuda(), hd ** -0.5).cpu()
        ref = paged_attention_reference(qq.float(), k.float(), v.float(), perm, lens, hd ** -0.5)
        err = (out1.float() - ref).abs().max().item()
        print(f"call {it}: ctx {ctx} max|diff| {err:.2e}")
        assert err <= 1e-2
        assert torch.equal(out1, out2)


@pytest.mark.parametrize("n_heads,n_kv,hd", [(12, 2, 128), (14, 2, 64)])
def test_per_head_kernel_for_tables_wider_than_the_row_merge(hiplib, n_heads, n_kv, hd):
    """A table of 1100 pages (more partitions than the whole-row kernel merges) takes the per-head kernel;
    contexts up to 1100 pages."""
    g = cpu_gen(22)
    ctx = [1, 700, 17600, 9000, 333]
    q, k, v, tables, lens = make_case(n_heads, n_kv, hd, ctx, torch.bfloat16, seed=22, extra_blocks=4, width=1100)
    out = run(q, k, v, tables, lens, hd ** -0.5)
    ref = paged_attention_reference(q.float(), k.float(), v.float(), tables, lens, hd ** -0.5)
    assert (out.float() - ref).abs().max().item() <= 1e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_padding_entries_and_past_ctx_tokens_are_never_used(hiplib, dtype):
    """Padding table entries point at a NaN-filled block and the unused tail of each last page is NaN:
    a kernel that read either would return NaN."""
    ctx = [17, 100, 333, 700, 5]
    q, k, v, tables, lens = make_case(12, 2, 128, ctx, dtype, extra_blocks=3, width=64)
    poison = k.shape[0] - 1
    assert poison not in tables[tables != 0].tolist()
    kp, vp = k.clone(), v.clone()
    kp[poison] = float("nan")
    vp[poison] = float("nan")
    for i, L in enumerate(ctx):
        nb = -(-L // 16)
        tables[i, nb:] = poison
        last = tables[i, nb - 1].item()
        kp[last, L - (nb - 1) * 16:] = float("nan")
        vp[last, L - (nb - 1) * 16:] = float("nan")
    out = run(q, kp, vp, tables, lens, 128 ** -0.5)
    assert torch.isfinite(out.float()).all()
    ref = paged_attention_reference(q.float(), k.float(), v.float(), tables, lens, 128 ** -0.5)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert (out.float() - ref).abs().max().item() <= tol


def test_graph_replay_matches_eager(hiplib):
    """Captured once, replayed with new context lengths and tables written into the static inputs."""
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    B, W = 8, 64
    q, k, v, tables, lens = make_case(12, 2, 128, [1000] * B, torch.bfloat16, seed=5, extra_blocks=80, width=W)
    dq, dk, dv = q.cuda(), k.cuda(), v.cuda()
    st, sl = tables.cuda(), lens.cuda()
    paged_attention_decode(dq, dk, dv, st, sl, 0.1)          # eager warm-up allocates the workspace
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = paged_attention_decode(dq, dk, dv, st, sl, 0.1)
    g = cpu_gen(9)
    for _ in range(3):
        new_lens = torch.randint(1, W * 16 + 1, (B,), generator=g, dtype=torch.int32)
        perm = torch.randperm(k.shape[0], generator=g)[:B * W].view(B, W).int()
        st.copy_(perm)
        sl.copy_(new_lens)
        graph.replay()
        got = out.cpu()
        torch.cuda.synchronize()
        ref = paged_attention_decode(dq, dk, dv, st, sl, 0.1).cpu()
        assert torch.equal(got, ref)
        oracle = paged_attention_reference(q.float(), k.float(), v.float(), perm, new_lens, 0.1)
        assert (got.float() - oracle).abs().max().item() <= 1e-2


@pytest.mark.parametrize("dtype,n_heads,n_kv,hd,width", [(torch.bfloat16, 12, 2, 128, None),
                                                          (torch.bfloat16, 14, 2, 64, None),
                                                          (torch.bfloat16, 12, 2, 128, 1100),
                                                          (torch.float32, 12, 2, 128, None)])
def test_rows_entry_point_equals_gather_decode_scatter(hiplib, dtype, n_heads, n_kv, hd, width):
    """ns_paged_attn_decode_rows (a mixed step's decode rows, nanoserve/model.py:274-281): entries read their
    queries from rows `rows` of a larger q and write the same rows of out; the result equals decoding the
    gathered rows, bitwise, and every other row of out keeps what it held (whole-row, per-head and fp32
    kernels)."""
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode_rows
    ctx = [1, 700, 2000, 17, 333, 64]
    q, k, v, tables, lens = make_case(n_heads, n_kv, hd, ctx, dtype, seed=31, width=width)
    g = cpu_gen(32)
    N = 40
    rows = torch.randperm(N, generator=g)[:len(ctx)]
    qa = torch.randn(N, n_heads, hd, generator=g).to(dtype)
    qa[rows] = q
    sentinel = torch.full((N, n_heads, hd), 7.0, dtype=dtype)
    out = sentinel.clone().cuda()
    paged_attention_decode_rows(qa.cuda(), k.cuda(), v.cuda(), tables.cuda(), lens.cuda(), rows.cuda(), hd ** -0.5,
                                out)
    got = out.cpu()
    ref = run(q, k, v, tables, lens, hd ** -0.5)
    assert torch.equal(got[rows], ref)
    others = torch.ones(N, dtype=torch.bool)
    others[rows] = False
    assert torch.equal(got[others], sentinel[others])


def test_rejects_unsupported_shapes(hiplib):
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    q, k, v, tables, lens = make_case(14, 2, 64, [20], torch.bfloat16)
    k8 = k.view(-1, 8, 2, 64)   # block size 8: the kernels need 16
    with pytest.raises(RuntimeError, match="block_size"):
        paged_attention_decode(q.cuda(), k8.cuda(), k8.cuda(), tables.cuda(), lens.cuda(), 0.1)


@pytest.mark.parametrize("n_heads,n_kv,hd,ctx_lens", [
    (14, 2, 64, None),                      # BASELINE config 2 (whole-row: both KV heads in one 256-byte row)
    (12, 2, 128, None),                     # the 1.5B decode step's shape (a workgroup row per KV head)
    (12, 2, 128, CTX_LENS),                 # short and one-page contexts
    (16, 2, 128, CTX_LENS)])                # group 8 with a row per KV head: beyond its registers -> error
def test_valu_products_variant(hiplib, n_heads, n_kv, hd, ctx_lens):
    """The A/B kernel with the QK^T and P.V products on the vector ALUs (ns_paged_attn_decode_valu): the same
    partitions and merge as the MFMA kernel, so it meets the same fp32-oracle bound and stays within bf16
    rounding of the MFMA kernel's output; shapes outside its register budget are refused."""
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    if ctx_lens is None:
        g = cpu_gen(8)
        ctx_lens = torch.randint(512, 4097, (32,), generator=g).tolist()
    q, k, v, tables, lens = make_case(n_heads, n_kv, hd, ctx_lens, torch.bfloat16, seed=9, extra_blocks=16)
    scale = hd ** -0.5
    dq, dk, dv, dt, dl = q.cuda(), k.cuda(), v.cuda(), tables.cuda(), lens.cuda()
    if n_heads // n_kv > (6 if hd == 128 and n_kv > 1 else 8):
        with pytest.raises(RuntimeError, match="GQA group"):
            paged_attention_decode(dq, dk, dv, dt, dl, scale, products="valu")
        return
    valu = paged_attention_decode(dq, dk, dv, dt, dl, scale, products="valu").cpu().float()
    valu2 = paged_attention_decode(dq, dk, dv, dt, dl, scale, products="valu").cpu().float()
    mfma = paged_attention_decode(dq, dk, dv, dt, dl, scale).cpu().float()
    ref = paged_attention_reference(q.float(), k.float(), v.float(), tables, lens, scale)
    e_ref, e_mfma = (valu - ref).abs().max().item(), (valu - mfma).abs().max().item()
    print(f"valu ({n_heads},{n_kv},{hd}) vs oracle {e_ref:.2e}, vs mfma {e_mfma:.2e}")
    assert e_ref <= 1e-2 and e_mfma <= 1e-2
    assert torch.equal(valu, valu2)


@pytest.mark.parametrize("n_heads,n_kv,hd", [(12, 2, 128), (16, 2, 128), (14, 2, 64)])
def test_paired_rows_equal_unpaired(hiplib, n_heads, n_kv, hd):
    """Speculative-verify rows: k + 1 rows per sequence share its block table with contexts ctx + 1 .. ctx + k + 1.
    With the pairing (pair_rows) two such rows run in one workgroup row of the whole-row kernel; every output
    equals the unpaired kernel's bitwise, including contexts on and next to page (16) and partition (512)
    boundaries, odd group sizes (a row left alone) and rows of other sequences between them. At 14 / 2 heads
    with hd 64 (one workgroup holds all 14 heads) the pairing does not fit and is ignored."""
    from nanoserve_amd.kernels.paged_attention import pair_rows, paged_attention_decode
    g = cpu_gen(41)
    bases = [15, 16, 511, 510, 1023, 700, 31, 2000]
    ks = [4, 2, 4, 1, 3, 0, 4, 2]
    nb = sum(-(-(b + k + 1) // 16) for b, k in zip(bases, ks)) + 8
    k = torch.randn(nb, 16, n_kv, hd, generator=g).to(torch.bfloat16)
    v = torch.randn(nb, 16, n_kv, hd, generator=g).to(torch.bfloat16)
    perm = torch.randperm(nb, generator=g)
    width = max(-(-(b + kk + 1) // 16) for b, kk in zip(bases, ks))
    tables_l, lens, used = [], [], 0
    for b, kk in zip(bases, ks):
        n = -(-(b + kk + 1) // 16)
        t = perm[used:used + n].tolist() + [0] * (width - n)
        used += n
        for j in range(kk + 1):
            tables_l.append(t)              # one list object per sequence, as the verify step stages them
            lens.append(b + j + 1)
    B = len(lens)
    q = torch.randn(B, n_heads, hd, generator=g).to(torch.bfloat16).cuda()
    tables = torch.tensor(tables_l, dtype=torch.int32).cuda()
    ctx = torch.tensor(lens, dtype=torch.int32).cuda()
    pairs_h = [9] * B
    pair_rows(tables_l, pairs_h)
    assert pairs_h.count(1) == sum((kk + 1) // 2 for kk in ks) and pairs_h.count(-1) == pairs_h.count(1)
    pairs = torch.tensor(pairs_h, dtype=torch.int32).cuda()
    kd, vd, scale = k.cuda(), v.cuda(), hd ** -0.5
    plain = paged_attention_decode(q, kd, vd, tables, ctx, scale)
    paired = paged_attention_decode(q, kd, vd, tables, ctx, scale, pairs=pairs)
    paired2 = paged_attention_decode(q, kd, vd, tables, ctx, scale, pairs=pairs)
    assert torch.equal(plain, paired) and torch.equal(paired, paired2)
    ref = paged_attention_reference(q.cpu().float(), k.float(), v.float(), tables.cpu(), ctx.cpu(), scale)
    assert (paired.cpu().float() - ref).abs().max().item() <= 1e-2

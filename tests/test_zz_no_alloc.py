"""ns_paged_attn_decode_noalloc (split-K workspace in the library's fixed device array) against
ns_paged_attn_decode with a caller workspace, both called through the C ABI: bitwise equal outputs on
consecutive calls whose second input is smaller (the array keeps the previous call's contents), on the
per-head kernel's wide tables, and a shape beyond the array's size rejected before any launch."""
import ctypes

import pytest
import torch

from nanoserve_amd import _lib


def make_case(B, n_heads, n_kv, hd, max_ctx, width, num_blocks, seed):
    g = torch.Generator().manual_seed(seed)
    ctx = torch.randint(1, max_ctx + 1, (B,), generator=g)
    perm = torch.randperm(num_blocks, generator=g)
    tables = torch.zeros(B, width, dtype=torch.int32)
    used = 0
    for b in range(B):
        n = -(-int(ctx[b]) // 16)
        tables[b, :n] = perm[used:used + n].int()
        used += n
    q = torch.randn(B, n_heads, hd, generator=g).to(torch.bfloat16)
    return q.cuda(), tables.cuda(), ctx.int().cuda()


def call(q, k, v, tables, ctx, workspace=None):
    """One launch through the C ABI; workspace None -> the allocation-free entry point."""
    L = _lib.load_library()
    B, nh, hd = q.shape
    NB, bs, nkv, _ = k.shape
    out = torch.full_like(q, float("nan"))
    args = (q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1),
            k.stride(2), tables.data_ptr(), tables.stride(0), ctx.data_ptr(), out.data_ptr(), out.stride(0),
            out.stride(1), B, nh, nkv, hd, bs, tables.shape[1], NB, hd ** -0.5, 1)
    stream = torch.cuda.current_stream().cuda_stream
    if workspace is None:
        st = L.ns_paged_attn_decode_noalloc(*args, stream)
    else:
        st = L.ns_paged_attn_decode(*args, workspace.data_ptr(), workspace.numel(), stream)
    _lib.check(st, "decode")
    return out


@pytest.mark.gpu
def test_noalloc_decode_equals_the_workspace_entry_point(hiplib):
    L = _lib.load_library()
    g = torch.Generator().manual_seed(0)
    cases = [  # (B, n_heads, n_kv, hd, max_ctx, width, pool blocks): config 2, then smaller, then wide tables
        (32, 14, 2, 64, 4096, 256, 65536),
        (5, 14, 2, 64, 900, 64, 65536),
        (4, 12, 2, 128, 17000, 1100, 16384),
        (3, 12, 2, 128, 300, 20, 16384),
    ]
    pools = {}
    for i, (B, nh, nkv, hd, mc, W, NB) in enumerate(cases):
        print(f"noalloc case {i}: B={B} {nh}/{nkv}/{hd} width {W}", flush=True)
        key = (nkv, hd, NB)
        if key not in pools:
            pools[key] = (torch.randn(NB, 16, nkv, hd, generator=g).to(torch.bfloat16).cuda(),
                          torch.randn(NB, 16, nkv, hd, generator=g).to(torch.bfloat16).cuda())
        k, v = pools[key]
        q, tables, ctx = make_case(B, nh, nkv, hd, mc, W, NB, seed=10 + i)
        need = L.ns_decode_workspace_bytes(B, nkv, hd, W, 1)
        assert need <= 16 << 20
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device="cuda")
        ref = call(q, k, v, tables, ctx, ws)
        for rep in range(2):
            got = call(q, k, v, tables, ctx)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"case {i} call {rep}: noalloc output differs"
            assert not torch.isnan(got).any()


def test_noalloc_rejects_a_shape_beyond_its_scratch():
    """Checked on the host before any GPU work (runs without a GPU)."""
    L = _lib.load_library()
    B, W = 4096, 1024
    assert L.ns_decode_workspace_bytes(B, 2, 128, W, 1) > 16 << 20
    st = L.ns_paged_attn_decode_noalloc(None, 0, 0, None, None, 0, 0, 0, None, 0, None, None, 0, 0,
                                        B, 12, 2, 128, 16, W, 1 << 16, 0.088, 1, None)
    assert st == 1
    assert b"scratch" in L.ns_last_error()

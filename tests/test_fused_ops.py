"""HIP fused token-wise kernels vs the CPU oracle's unfused ops (oracle/ops.py).

Gates follow the reference's tests/test_fused_ops.py:29-96: fp32 within 1e-5; bf16 at least 99% bitwise
identical and the rest within 1 bf16 ulp; the residual add is exact; RoPE writes rotated K and plain V at
exactly the given slots and nothing else. Inputs are drawn on the CPU (seeded) and copied to the GPU, so the
oracle (torch on the CPU) and the kernels see identical values.
"""
import pytest
import torch

from oracle import ops
from tests.conftest import cpu_gen

pytestmark = pytest.mark.gpu

DT = [torch.float32, torch.bfloat16]


def check(out, ref, dtype, ulps=1):
    out = out.cpu()
    assert out.shape == ref.shape and out.dtype == ref.dtype
    if dtype == torch.float32:
        torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
        return
    same = (out == ref).float().mean().item()
    assert same >= 0.99, f"only {same:.4f} bitwise identical"
    torch.testing.assert_close(out.float(), ref.float(), rtol=ulps * 2 ** -7, atol=1e-6)   # <= `ulps` bf16 ulps


# RMSNorm rounds twice: y = round(x * inv), out = round(w * y). A different fp32 summation order can move inv
# by an fp32 ulp and flip y by one bf16 ulp, which w (|w| ~ 1.3 at most here) carries into out: at most
# 2^-7 |w y| before the final rounding, so 2 bf16 ulps of out. The reference's 1-ulp gate holds at its
# 37-row shapes; at 1552 x 1536 rows a flip of y lands on a large |w| now and then.
def norm_ulps(rows):
    return 1 if rows <= 64 else 2


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,n", [(37, 896), (37, 1536), (37, 2048), (1552, 1536)])
def test_rms_norm(hiplib, dtype, rows, n):
    from nanoserve_amd.kernels.fused import rms_norm
    g = cpu_gen(0)
    x = (torch.randn(rows, n, generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(n, generator=g)).to(dtype)
    check(rms_norm(x.cuda(), w.cuda(), 1e-6), ops.rms_norm(x, w, 1e-6), dtype, norm_ulps(rows))


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,n", [(37, 896), (1552, 1536)])
def test_rms_norm_with_residual_add(hiplib, dtype, rows, n):
    from nanoserve_amd.kernels.fused import rms_norm
    g = cpu_gen(1)
    x, a = (torch.randn(1, rows, n, generator=g).to(dtype) for _ in range(2))
    w = (1 + 0.1 * torch.randn(n, generator=g)).to(dtype)
    out, res = rms_norm(a.cuda(), w.cuda(), 1e-6, residual=x.cuda())
    ref_out, ref_res = ops.rms_norm_residual(a, w, 1e-6, x)
    assert torch.equal(res.cpu(), ref_res)                     # the add is exact: same rounding as PyTorch
    check(out, ref_out, dtype, norm_ulps(rows))


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("rows,n", [(37, 4864), (37, 8960), (37, 11008), (37, 100), (1552, 8960)])
def test_silu_mul(hiplib, dtype, rows, n):
    from nanoserve_amd.kernels.fused import silu_mul
    g = cpu_gen(2)
    x = (torch.randn(1, rows, 2 * n, generator=g) * 2).to(dtype)
    check(silu_mul(x.cuda()), ops.silu_mul(x), dtype)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("N,nh,nkv,hd", [(37, 14, 2, 64), (37, 12, 2, 128), (37, 16, 2, 128), (1552, 12, 2, 128)])
def test_rope_qkv_and_cache_write(hiplib, dtype, N, nh, nkv, hd):
    from nanoserve_amd.kernels.fused import rope_qkv
    g = cpu_gen(3)
    NB = max(8, -(-2 * N // 16))
    qkv = torch.randn(N, (nh + 2 * nkv) * hd, generator=g).to(dtype)
    positions = torch.randint(0, 2000, (N,), generator=g)
    cos, sin = ops.rope_tables(positions, hd, 1_000_000.0, dtype)
    slots = torch.randperm(NB * 16, generator=g)[:N]
    k_cache = torch.zeros(NB, 16, nkv, hd, dtype=dtype, device="cuda")
    v_cache = torch.zeros_like(k_cache)
    q, k, v = rope_qkv(qkv.cuda(), cos.cuda(), sin.cuda(), nh, nkv, hd, k_cache, v_cache, slots.cuda())

    rk, rv = torch.zeros(NB, 16, nkv, hd, dtype=dtype), torch.zeros(NB, 16, nkv, hd, dtype=dtype)
    q0, k0, v0 = ops.rope_qkv(qkv, cos, sin, nh, nkv, hd, rk, rv, slots)
    check(q, q0, dtype)
    check(k, k0, dtype)
    assert torch.equal(v.cpu(), v0)
    k, v = k.cpu(), v.cpu()
    flat_k, flat_v = k_cache.cpu().view(-1, nkv, hd), v_cache.cpu().view(-1, nkv, hd)
    assert torch.equal(flat_k[slots], k) and torch.equal(flat_v[slots], v)
    untouched = torch.ones(NB * 16, dtype=torch.bool)
    untouched[slots] = False
    assert not flat_k[untouched].any() and not flat_v[untouched].any()


def test_rope_without_cache(hiplib):
    from nanoserve_amd.kernels.fused import rope_qkv
    g = cpu_gen(4)
    qkv = torch.randn(5, (12 + 4) * 128, generator=g).to(torch.bfloat16)
    cos, sin = ops.rope_tables(torch.arange(5), 128, 1e6, torch.bfloat16)
    q, k, v = rope_qkv(qkv.cuda(), cos.cuda(), sin.cuda(), 12, 2, 128)
    q0, k0, v0 = ops.rope_qkv(qkv, cos, sin, 12, 2, 128)
    check(q, q0, torch.bfloat16)
    check(k, k0, torch.bfloat16)
    assert torch.equal(v.cpu(), v0)


@pytest.mark.parametrize("dtype", DT)
@pytest.mark.parametrize("H,hd,N", [(1536, 128, 32), (896, 64, 5), (2048, 128, 64), (256, 64, 200)])
def test_embed_rope(hiplib, dtype, H, hd, N):
    """x = embedding rows exactly; cos/sin equal the oracle's RoPE tables (HF order: fp32 positions *
    inv_freq, cat, cos/sin, cast) to the check's gate; the row statistics are the 16-column sums of x^2
    (fp64 closed form), and the norm they feed equals the oracle's rms_norm of x."""
    from nanoserve_amd.kernels.fused import embed_rope
    from nanoserve_amd.kernels.linear import NormedRows
    g = cpu_gen(11)
    V = 1000
    embed = (torch.randn(V, H, generator=g) * 0.5).to(dtype)
    ids = torch.randint(0, V, (N,), generator=g)
    pos = torch.randint(0, 40000, (N,), generator=g)
    inv = 1.0 / (1e6 ** (torch.arange(0, hd, 2, dtype=torch.float) / hd))
    stats = dtype == torch.bfloat16 and N <= 64
    x, cos, sin, sq = embed_rope(ids.cuda(), pos.cuda(), embed.cuda(), inv.cuda(), hd, row_stats=stats)
    assert torch.equal(x.cpu(), embed[ids])
    c_ref, s_ref = ops.rope_tables(pos, hd, 1e6, dtype)
    check(cos, c_ref, dtype)
    check(sin, s_ref, dtype)
    if stats:
        ref = (embed[ids].double() ** 2).view(N, H // 16, 16).sum(-1).T
        torch.testing.assert_close(sq[:, :N].cpu().double(), ref, rtol=1e-5, atol=1e-6)
        w = (1 + 0.1 * torch.randn(H, generator=g)).to(dtype)
        h = NormedRows(x, sq, w.cuda(), 1e-6).tensor()
        check(h, ops.rms_norm(embed[ids], w, 1e-6), dtype)
    else:
        assert sq is None


def test_embed_rope_out_of_range_id_gives_a_zero_row(hiplib):
    from nanoserve_amd.kernels.fused import embed_rope
    embed = torch.randn(10, 64).to(torch.bfloat16).cuda()
    ids = torch.tensor([3, 10, -1, 9]).cuda()
    x, _, _, _ = embed_rope(ids, torch.arange(4).cuda(), embed, torch.ones(32).cuda(), 64)
    assert torch.equal(x[0], embed[3]) and torch.equal(x[3], embed[9])
    assert not x[1].any() and not x[2].any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_gather_rows(hiplib, dtype):
    """ns_gather_rows (the LM head's row selection, nanoserve/model.py:353-356): bitwise equal to x[idx] for
    repeated, unordered indices, from a strided view; an index outside [0, n) gives a zero row; no rows is a no-op."""
    from nanoserve_amd import _lib
    from nanoserve_amd.kernels.fused import gather_rows
    g = cpu_gen(71)
    base = torch.randn(40, 1600, generator=g).to(dtype).cuda()
    x = base[:, :1536]                                   # rows 1600 elements apart
    idx = torch.tensor([39, 0, 7, 7, 21, 38], dtype=torch.int64, device="cuda")
    assert torch.equal(gather_rows(x, idx).cpu(), x[idx].cpu())
    out = torch.full((3, 1536), 5.0, dtype=dtype, device="cuda")
    bad = torch.tensor([2, 40, -1], dtype=torch.int64, device="cuda")
    L = _lib.lib()
    rb = 1536 * x.element_size()
    assert L.ns_gather_rows(x.data_ptr(), x.stride(0) * x.element_size(), 40, bad.data_ptr(), 3, rb, out.data_ptr(), rb,
                            _lib.stream_of(x)) == 0, L.ns_last_error()
    assert torch.equal(out[0].cpu(), x[2].cpu()) and not out[1:].cpu().any()
    assert L.ns_gather_rows(x.data_ptr(), x.stride(0) * x.element_size(), 40, bad.data_ptr(), 0, rb, out.data_ptr(), rb,
                            _lib.stream_of(x)) == 0
    assert L.ns_gather_rows(x.data_ptr(), 8, 40, bad.data_ptr(), 3, rb, out.data_ptr(), rb, _lib.stream_of(x)) != 0

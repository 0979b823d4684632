"""Skinny HIP GEMMs (csrc/gemm.hip) vs the CPU oracle.

The oracle of a projection is the exact product of the same bf16 values accumulated in fp32 on the CPU and
rounded once to bf16 (what F.linear computes, nanoserve/model.py:231,256-257,362); the fused epilogues are
checked against the oracle's unfused ops applied to that rounded product (oracle/ops.py). Gate: at least
99% bitwise identical (the reference's `check`, tests/test_fused_ops.py:29-36) and every element within
1 bf16 ulp plus the error a different fp32 summation order may legitimately carry: Higham's deterministic
dot-product bound gamma_K * sum|x||w| (per element, for both sides), propagated through each epilogue's
Lipschitz constant. Near-cancelling sums at K = 8960 can exceed 1 ulp relative; no systematic error can
pass. Also: KV writes exact at the slots, determinism, and graph replay == eager.
"""
import pytest
import torch

from oracle import ops
from tests.conftest import cpu_gen

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def ulp(t):
    """bf16 spacing at |t| (2^-7 relative; the smallest normal spacing near 0)."""
    return torch.clamp(t.float().abs(), min=2.0 ** -126) * 2.0 ** -7


def bf16_check(out, ref, what, bound=None):
    """>= 99% bitwise identical, and every element within 1 bf16 ulp of the oracle plus `bound`, the
    per-element error the fp32 accumulation may legitimately carry (0 if not given)."""
    out = out.cpu()
    assert out.shape == ref.shape and out.dtype == ref.dtype == BF, what
    same = (out == ref).float().mean().item()
    assert same >= 0.99, f"{what}: only {same:.4f} bitwise identical"
    err = (out.float() - ref.float()).abs()
    allowed = ulp(ref) + (0 if bound is None else bound)
    bad = err > allowed
    assert not bad.any(), f"{what}: {int(bad.sum())} elements beyond the bound, worst {float((err - allowed).max()):.3e}"


def dot_bound(x, w):
    """Deterministic bound on |fl32(x . w) - x . w| for any summation order (Higham, gamma_K), twice over:
    both the kernel and the oracle carry it."""
    K = x.shape[1]
    u = 2.0 ** -24
    gamma = K * u / (1 - K * u)
    return 2 * gamma * (x.double().abs() @ w.double().abs().T).float()


def operands(M, N, K, seed=0, scale=1.0):
    g = cpu_gen(seed)
    x = (torch.randn(M, K, generator=g) * scale).to(BF)
    w = (torch.randn(N, K, generator=g) * 0.05).to(BF)
    return x, w


def ref_linear(x, w, b=None):
    y = x.float() @ w.float().T
    if b is not None:
        y = y + b.float()
    return y.to(BF)


@pytest.mark.parametrize("M", [1, 7, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("N,K", [(2048, 1536), (1536, 8960), (17920, 1536), (1000, 896)])
def test_linear(hiplib, M, N, K):
    from nanoserve_amd.kernels.linear import linear
    x, w = operands(M, N, K, seed=M + N)
    b = (torch.randn(N, generator=cpu_gen(1)) * 0.1).to(BF)
    bd = dot_bound(x, w)
    bf16_check(linear(x.cuda(), w.cuda(), b.cuda()), ref_linear(x, w, b), f"linear M={M} N={N} K={K}", bd)
    bf16_check(linear(x.cuda(), w.cuda()), ref_linear(x, w), f"linear (no bias) M={M} N={N} K={K}", bd)


def test_lm_head_shape(hiplib):
    from nanoserve_amd.kernels.linear import linear
    x, w = operands(32, 151936, 1536, seed=3)
    bf16_check(linear(x.cuda(), w.cuda()), ref_linear(x, w), "lm head 32x151936x1536", dot_bound(x, w))


@pytest.mark.parametrize("M", [1, 16, 32])
@pytest.mark.parametrize("K", [896, 1280, 1536, 2048])
def test_wide_projection_persistent_kernel(hiplib, M, K):
    """Wide projections without bias (at least four 64-row tiles per CU, M <= 32, K <= 2048: the LM head) run
    on persistent workgroups that keep their activation fragments in registers across tiles. N = 65573 (a
    partial last tile), K with a partial and a padding chunk; a normalised input equals its materialised
    norm bitwise here too."""
    from nanoserve_amd.kernels.linear import linear, linear_residual_rms_norm
    N = 65536 + 37
    x, w = operands(M, N, K, seed=M + K)
    wd = w.cuda()
    bf16_check(linear(x.cuda(), wd), ref_linear(x, w), f"wide M={M} N={N} K={K}", dot_bound(x, w))
    if M == 32:
        x0, w0 = operands(M, K, 512, seed=40)
        res = torch.randn(M, K, generator=cpu_gen(41)).to(BF).cuda()
        nw = (1 + 0.1 * torch.randn(K, generator=cpu_gen(42))).to(BF).cuda()
        hn, _ = linear_residual_rms_norm(x0.cuda(), w0.cuda(), res, nw, 1e-6)
        assert torch.equal(linear(hn, wd), linear(hn.tensor(), wd))


@pytest.mark.parametrize("M", [1, 24, 32, 64])
@pytest.mark.parametrize("I,K", [(8960, 1536), (4864, 896), (11008, 2048)])
def test_linear_silu_mul(hiplib, M, I, K):
    from nanoserve_amd.kernels.linear import linear_silu_mul
    x, w = operands(M, 2 * I, K, seed=4, scale=2.0)
    gu = ref_linear(x, w)
    # an input moved by e (accumulation error + 1 ulp of rounding) moves silu(g)*u by at most
    # (|u| * max|silu'| + |silu(g)|) * e, with |silu'| <= 1.1
    e = dot_bound(x, w) + ulp(gu)
    g_, u_ = gu[:, :I].float(), gu[:, I:].float()
    bound = (1.1 * u_.abs() + torch.nn.functional.silu(g_).abs() + 1.1 * e[:, I:]) * torch.maximum(e[:, :I], e[:, I:])
    bf16_check(linear_silu_mul(x.cuda(), w.cuda()), ops.silu_mul(gu), f"silu_mul M={M} I={I}", 2 * bound)


@pytest.mark.parametrize("M", [1, 20, 32, 64, 65, 96, 120, 128, 129])
@pytest.mark.parametrize("N,K,norm", [(1536, 1536, True), (1536, 8960, True), (896, 4864, False), (2048, 11008, True)])
def test_linear_residual_rms_norm(hiplib, M, N, K, norm):
    """Up to 64 rows the skinny / tile-16 kernels, up to 128 (verify batches) their 16- or 64-row token blocks
    with the residual and row statistics in the epilogue, above that the plain GEMM and the RMSNorm kernel."""
    from nanoserve_amd.kernels.linear import linear_residual_rms_norm
    x, w = operands(M, N, K, seed=5)
    g = cpu_gen(6)
    res = torch.randn(M, N, generator=g).to(BF)
    nw = (1 + 0.1 * torch.randn(N, generator=g)).to(BF)
    h, r = linear_residual_rms_norm(x.cuda(), w.cuda(), res.cuda(), nw.cuda() if norm else None, 1e-6)
    y = ref_linear(x, w)
    ref_r = res + y
    e = dot_bound(x, w) + ulp(y)                     # error of the rounded projection
    bf16_check(r, ref_r, "residual sum", e)
    if norm:
        rf = ref_r.float()
        inv = torch.rsqrt(rf.pow(2).mean(-1, keepdim=True) + 1e-6)
        # h = w * r * inv: each r moved by <= e + ulp(r); inv moves by <= inv * (max relative change)
        er = e + ulp(ref_r)
        rel = (er.abs() / rf.abs().clamp(min=1e-6)).max(dim=-1, keepdim=True).values.clamp(max=1.0)
        bound = nw.float().abs() * inv * (er + rf.abs() * rel) * 2
        hh = h.tensor() if hasattr(h, "tensor") else h   # a NormedRows up to 128 rows, a tensor above
        bf16_check(hh, ops.rms_norm(ref_r, nw, 1e-6), "rms_norm of the sum", bound)
    else:
        assert h is None


@pytest.mark.parametrize("M", [1, 20, 32, 64, 65, 96, 120, 192, 193, 1552])
@pytest.mark.parametrize("nh,nkv,hd,K", [(12, 2, 128, 1536), (14, 2, 64, 896), (16, 2, 128, 2048)])
def test_linear_rope_qkv_and_cache_write(hiplib, M, nh, nkv, hd, K):
    """M <= 64: the skinny kernels; 65..192 rows: the tile-16 kernel in 16-token blocks (verify batches);
    193 and 1552 (the config-4 mixed step): the tiled kernel with the RoPE epilogue."""
    from nanoserve_amd import _lib
    from nanoserve_amd.kernels.linear import linear_rope_qkv
    assert _lib.lib().ns_gemm_rope_qkv_fits(M, K, nh, nkv, hd, 0) == 1
    assert _lib.lib().ns_gemm_rope_qkv_fits(M, K, nh, nkv, hd, 1) == (1 if M <= 128 else 0)
    N = (nh + 2 * nkv) * hd
    x, w = operands(M, N, K, seed=7)
    g = cpu_gen(8)
    b = (torch.randn(N, generator=g) * 0.1).to(BF)
    cos, sin = ops.rope_tables(torch.randint(0, 4000, (M,), generator=g), hd, 1e6, BF)
    nb = max(16, 2 * (M // 16 + 1))   # cache blocks of 16 slots, twice the rows
    slots = torch.randperm(nb * 16, generator=g)[:M]
    kc = torch.zeros(nb, 16, nkv, hd, dtype=BF, device="cuda")
    vc = torch.zeros_like(kc)
    q, k, v = linear_rope_qkv(x.cuda(), w.cuda(), b.cuda(), cos.cuda(), sin.cuda(), nh, nkv, hd, kc, vc, slots.cuda())
    rk, rv = torch.zeros(nb, 16, nkv, hd, dtype=BF), torch.zeros(nb, 16, nkv, hd, dtype=BF)
    qkv = ref_linear(x, w, b)
    q0, k0, v0 = ops.rope_qkv(qkv, cos, sin, nh, nkv, hd, rk, rv, slots)
    # rotation mixes two inputs with |cos|, |sin| <= 1: an input error e becomes <= 2e (+ roundings)
    e = dot_bound(x, w) + ulp(qkv)
    eh = torch.maximum(e.view(M, -1, hd), e.view(M, -1, hd).roll(hd // 2, dims=-1))   # each output mixes d, d +- hd/2
    bound = 3 * eh
    bf16_check(q, q0, "q", bound[:, :nh] + 2 * ulp(q0))
    bf16_check(k, k0, "k", bound[:, nh:nh + nkv] + 2 * ulp(k0))
    bf16_check(v, v0, "v", e.view(M, -1, hd)[:, nh + nkv:])
    flat_k, flat_v = kc.cpu().view(-1, nkv, hd), vc.cpu().view(-1, nkv, hd)
    assert torch.equal(flat_k[slots], k.cpu()) and torch.equal(flat_v[slots], v.cpu())
    untouched = torch.ones(nb * 16, dtype=torch.bool)
    untouched[slots] = False
    assert not flat_k[untouched].any() and not flat_v[untouched].any()


def test_deterministic_and_graph_replay(hiplib):
    from nanoserve_amd.kernels.linear import linear, linear_residual_rms_norm, linear_silu_mul
    x, w = operands(32, 1536, 8960, seed=9)
    x2, wgu = operands(32, 2 * 8960, 1536, seed=10)
    res = torch.randn(32, 1536, generator=cpu_gen(11)).to(BF).cuda()
    nw = torch.ones(1536, dtype=BF, device="cuda")
    dx, dw, dx2, dwgu = x.cuda(), w.cuda(), x2.cuda(), wgu.cuda()

    def step():
        a = linear(dx, dw)
        b = linear_silu_mul(dx2, dwgu)
        h, r = linear_residual_rms_norm(dx, dw, res, nw, 1e-6)
        return a, b, h.tensor(), r

    eager1 = [t.clone() for t in step()]
    eager2 = [t.clone() for t in step()]
    for a, b in zip(eager1, eager2):
        assert torch.equal(a, b)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = step()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for a, b in zip(outs, eager1):
            assert torch.equal(a, b)
        step()   # eager work between replays


@pytest.mark.parametrize("M", [1, 32, 64])
@pytest.mark.parametrize("K", [1536, 896])
def test_norm_on_load_equals_the_materialised_norm(hiplib, M, K):
    """A projection of a NormedRows (r + its row statistics, normalised fragment by fragment as the GEMM
    loads it) equals the same projection of NormedRows.tensor() bitwise, for every consumer kind, and row
    selection (the LM head's) keeps that."""
    from nanoserve_amd.kernels.linear import linear, linear_residual_rms_norm, linear_rope_qkv, linear_silu_mul
    x0, w0 = operands(M, K, 512, seed=12)
    res = torch.randn(M, K, generator=cpu_gen(13)).to(BF).cuda()
    nw = (1 + 0.1 * torch.randn(K, generator=cpu_gen(14))).to(BF).cuda()
    hn, r = linear_residual_rms_norm(x0.cuda(), w0.cuda(), res, nw, 1e-6)
    h = hn.tensor()
    assert torch.equal(h, hn.tensor())
    # the materialised norm agrees with the oracle's rms_norm of the same r (different summation order)
    ref = ops.rms_norm(r.cpu(), nw.cpu(), 1e-6)
    same, ulps = ops.bf16_ulp_close(h.cpu(), ref)
    assert same >= 0.99 and ulps <= 1.0, (same, ulps)

    _, w = operands(M, 1000, K, seed=15)
    b = (torch.randn(1000, generator=cpu_gen(16)) * 0.1).to(BF).cuda()
    assert torch.equal(linear(hn, w.cuda(), b), linear(h, w.cuda(), b))
    _, wgu = operands(M, 2 * 1024, K, seed=17)
    assert torch.equal(linear_silu_mul(hn, wgu.cuda()), linear_silu_mul(h, wgu.cuda()))
    nh, nkv, hd = 12, 2, 128
    _, wq = operands(M, (nh + 2 * nkv) * hd, K, seed=18)
    cos, sin = ops.rope_tables(torch.arange(M) + 7, hd, 1e6, BF)
    qa = linear_rope_qkv(hn, wq.cuda(), None, cos.cuda(), sin.cuda(), nh, nkv, hd)
    qb = linear_rope_qkv(h, wq.cuda(), None, cos.cuda(), sin.cuda(), nh, nkv, hd)
    for a_, b_ in zip(qa, qb):
        assert torch.equal(a_, b_)
    idx = torch.arange(M - 1, -1, -2, device="cuda")
    assert torch.equal(linear(hn.rows(idx), w.cuda()), linear(h[idx].contiguous(), w.cuda()))

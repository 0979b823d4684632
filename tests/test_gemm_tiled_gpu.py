"""HIP GEMMs above 64 rows (csrc/gemm.hip: prefill chunks, mixed steps, speculative verify batches) vs the
CPU oracle, with the gate of the skinny-kernel tests: >= 99% bitwise identical to the fp32-accumulated,
once-rounded product and every element within 1 bf16 ulp plus Higham's deterministic bound gamma_K * sum|x||w|
(for both sides), propagated through the SiLU epilogue. The product replaces F.linear at
nanoserve/model.py:231,256-257 on the large-token path. At 1552 rows the check covers every 128-row tile
(its first, middle and last rows and the partial last tile) and every column. Routes: up to 192 rows the
K <= 2048 projections run the tile-16 kernel in 16-token blocks and the 8960-long ones the skinny kernel in
64-row token blocks; otherwise the tiled kernel (1552 x 17920 on 256 x 256 tiles; long K (>= 128 steps)
on 256 x 128 or 128 x 128 tiles K-sliced to one workgroup per CU; the rest on 128 x 128).
Also: K-sliced products are deterministic and share the skinny kernels' workspace."""
import pytest
import torch

from oracle import ops
from tests.conftest import cpu_gen
from tests.test_gemm_kernels import BF, bf16_check, dot_bound, operands, ref_linear, ulp

pytestmark = pytest.mark.gpu


def check_rows(M):
    """Rows to check: all of them up to 160, else the edges and middle of every 128-row tile."""
    if M <= 160:
        return torch.arange(M)
    rows = sorted({r for t0 in range(0, M, 128) for r in (t0, t0 + 1, t0 + 63, t0 + 64, t0 + 126, t0 + 127)
                   if r < M} | {M - 1, M - 2})
    return torch.tensor(rows)


@pytest.mark.parametrize("M", [65, 96, 120, 300, 1552])
@pytest.mark.parametrize("N,K,bias", [(2048, 1536, True), (1536, 8960, False), (1536, 1536, False), (1003, 896, True),
                                      (17920, 1536, True)])
def test_tiled_linear(hiplib, M, N, K, bias):
    from nanoserve_amd.kernels.linear import linear
    x, w = operands(M, N, K, seed=M + N)
    b = (torch.randn(N, generator=cpu_gen(1)) * 0.1).to(BF) if bias else None
    y = linear(x.cuda(), w.cuda(), b.cuda() if bias else None).cpu()
    rows = check_rows(M)
    xs = x[rows]
    bf16_check(y[rows], ref_linear(xs, w, b), f"tiled linear M={M} N={N} K={K} bias={bias}", dot_bound(xs, w))


@pytest.mark.parametrize("M,N,K,bias", [(2048, 1536, 8960, False), (1300, 1003, 4864, True), (512, 1536, 8960, False)])
def test_long_k_plans(hiplib, M, N, K, bias):
    """Long-K shapes on each one-round plan: 256 x 128 tiles in 2 K slices (2048 rows), 256 x 128 tiles in 4
    slices with a partial last tile in both dimensions and a bias (1300 x 1003), 128 x 128 tiles in 5 slices
    (512 rows)."""
    from nanoserve_amd.kernels.linear import linear
    x, w = operands(M, N, K, seed=M + 3 * N)
    b = (torch.randn(N, generator=cpu_gen(2)) * 0.1).to(BF) if bias else None
    y = linear(x.cuda(), w.cuda(), b.cuda() if bias else None).cpu()
    rows = torch.tensor(sorted({r for t0 in range(0, M, 128) for r in (t0, t0 + 127) if r < M} | {M - 1}))
    xs = x[rows]
    bf16_check(y[rows], ref_linear(xs, w, b), f"long-K linear M={M} N={N} K={K} bias={bias}", dot_bound(xs, w))


@pytest.mark.parametrize("M", [65, 96, 120, 1552])
@pytest.mark.parametrize("I,K", [(8960, 1536), (4864, 896), (100, 256)])
def test_tiled_linear_silu_mul(hiplib, M, I, K):
    from nanoserve_amd.kernels.linear import linear_silu_mul
    x, w = operands(M, 2 * I, K, seed=4, scale=2.0)
    out = linear_silu_mul(x.cuda(), w.cuda()).cpu()
    rows = check_rows(M)
    xs = x[rows]
    gu = ref_linear(xs, w)
    e = dot_bound(xs, w) + ulp(gu)
    g_, u_ = gu[:, :I].float(), gu[:, I:].float()
    bound = (1.1 * u_.abs() + torch.nn.functional.silu(g_).abs() + 1.1 * e[:, I:]) * torch.maximum(e[:, :I], e[:, I:])
    bf16_check(out[rows], ops.silu_mul(gu), f"tiled silu_mul M={M} I={I} K={K}", 2 * bound)


def test_tiled_split_k_is_deterministic_and_shares_the_workspace(hiplib):
    """M = 96 on the 1536 x 8960 down projection (64-row token blocks of the skinny kernel, K sliced); two
    calls agree bitwise, also with skinny calls (which use the same workspace counters) in between."""
    from nanoserve_amd.kernels.linear import linear
    x, w = operands(96, 1536, 8960, seed=9)
    xd, wd = x.cuda(), w.cuda()
    a = linear(xd, wd)
    linear(xd[:32].contiguous(), wd)
    b = linear(xd, wd)
    linear(xd[:7].contiguous(), wd)
    c = linear(xd, wd)
    assert torch.equal(a, b) and torch.equal(a, c)
    bf16_check(a.cpu(), ref_linear(x, w), "split-K tiled 96x1536x8960", dot_bound(x, w))


def test_normalised_input_above_64_rows_through_the_c_abi(hiplib):
    """ns_gemm takes a normalised input (r + row statistics) up to NS_NORM_ROWS = 128 rows when the tile-16
    kernel takes the shape (its 16-row token blocks normalise on load), bitwise equal to the product of the
    materialised norm; above 128 rows it refuses (the Python layer materialises the input there)."""
    from nanoserve_amd import _lib
    from nanoserve_amd.kernels.linear import NORM_ROWS, NormedRows
    L = _lib.lib()
    for M in (96, 129):
        x, w = operands(M, 256, 256, seed=3)
        xd, wd = x.cuda(), w.cuda()
        y = torch.empty(M, 256, dtype=BF, device="cuda")
        sq = torch.zeros(16, NORM_ROWS, device="cuda")
        rows = min(M, NORM_ROWS)
        sq[:, :rows] = xd[:rows].float().pow(2).view(rows, 16, 16).sum(-1).t()
        nw = (1 + 0.1 * torch.randn(256, generator=cpu_gen(4))).to(BF).cuda()
        rc = L.ns_gemm(xd.data_ptr(), wd.data_ptr(), None, y.data_ptr(), M, 256, 256, 1, sq.data_ptr(),
                       nw.data_ptr(), 1e-6, None, 0, _lib.stream_of(xd))
        if M > NORM_ROWS:
            assert rc != 0 and b"normalised" in L.ns_last_error()
            continue
        assert rc == 0, L.ns_last_error()
        h = NormedRows(xd, sq, nw, 1e-6).tensor()
        y2 = torch.empty_like(y)
        assert L.ns_gemm(h.data_ptr(), wd.data_ptr(), None, y2.data_ptr(), M, 256, 256, 1, None, None, 0.0, None, 0,
                         _lib.stream_of(xd)) == 0
        assert torch.equal(y, y2)


@pytest.mark.parametrize("M,N,K", [(96, 1536, 1536), (120, 1536, 8960), (128, 896, 4864)])
def test_residual_row_statistics_above_64_rows_through_the_c_abi(hiplib, M, N, K):
    """ns_gemm_residual_norm_stats on verify-sized batches (65-128 rows): the tile-16 kernel's 16-row token
    blocks (K <= 2048) or the skinny kernel's 64-row blocks (longer K) with the residual sum and the
    per-16-column row sums of squares in the epilogue; r against the fp64 product, the statistics exactly
    the row sums of r^2 (every row, both token blocks' halves), and the norm applied from them against the
    oracle's rms_norm of r."""
    from nanoserve_amd import _lib
    from nanoserve_amd.kernels.linear import NORM_ROWS, NormedRows
    L = _lib.lib()
    x, w = operands(M, N, K, seed=21)
    res = torch.randn(M, N, generator=cpu_gen(22)).to(BF)
    xd, wd, rd = x.cuda(), w.cuda(), res.cuda()
    r = torch.empty(M, N, dtype=BF, device="cuda")
    sq = torch.full((N // 16, NORM_ROWS), float("nan"), device="cuda")
    ws = torch.zeros(max(L.ns_gemm_workspace_bytes(M, N, K), 256), dtype=torch.uint8, device="cuda")
    rc = L.ns_gemm_residual_norm_stats(xd.data_ptr(), wd.data_ptr(), rd.data_ptr(), r.data_ptr(), sq.data_ptr(), M, N, K,
                                       1, ws.data_ptr(), ws.numel(), _lib.stream_of(xd))
    assert rc == 0, L.ns_last_error()
    y = ref_linear(x, w)
    bf16_check(r.cpu(), res + y, f"residual sum {M}x{N}x{K}", dot_bound(x, w) + ulp(y))
    want = r.float().pow(2).view(M, N // 16, 16).sum(-1).t()
    assert torch.allclose(sq[:, :M], want, rtol=1e-5, atol=1e-6)
    nw = (1 + 0.1 * torch.randn(N, generator=cpu_gen(23))).to(BF).cuda()
    h = NormedRows(r, sq, nw, 1e-6).tensor().cpu()
    same, ulps = ops.bf16_ulp_close(h, ops.rms_norm(r.cpu(), nw.cpu(), 1e-6))
    assert same >= 0.99 and ulps <= 1.0, (same, ulps)


@pytest.mark.parametrize("M,nh,nkv,hd,K,bias,cache", [
    (193, 12, 2, 128, 1536, True, True),     # 4-wave 128 x 128 tiles, a partial last row tile
    (1552, 12, 2, 128, 1536, True, True),    # 8-wave 128 x 128 tiles: the config-4 mixed step's QKV
    (1552, 14, 2, 64, 896, True, False),     # two 64-wide heads per tile, no cache
    (300, 16, 2, 128, 2048, False, True),
    (512, 16, 2, 128, 4096, True, True),     # long K: K slices merged before the epilogue
    (8192, 12, 2, 128, 1536, True, True),    # 256 x 256 tiles (two heads each)
])
def test_tiled_rope_epilogue_equals_gemm_then_rope(hiplib, M, nh, nkv, hd, K, bias, cache):
    """Above 192 rows ns_gemm_rope_qkv rotates in the tiled kernel's epilogue: q, k, v and the cache pages
    are bit-identical to the tiled STORE product followed by the RoPE kernel (the unfused route, each
    checked against the oracle elsewhere), on the same plan."""
    from nanoserve_amd.kernels.fused import rope_qkv
    from nanoserve_amd.kernels.linear import linear, linear_rope_qkv
    N = (nh + 2 * nkv) * hd
    x, w = operands(M, N, K, seed=M + hd)
    g = cpu_gen(M)
    b = (torch.randn(N, generator=g) * 0.1).to(BF).cuda() if bias else None
    cos, sin = ops.rope_tables(torch.randint(0, 32768, (M,), generator=g), hd, 1e6, BF)
    cos, sin = cos.cuda(), sin.cuda()
    nb = 2 * (M // 16 + 1)
    slots = torch.randperm(nb * 16, generator=g)[:M].cuda() if cache else None
    caches = []
    for _ in range(2):
        kc = torch.zeros(nb, 16, nkv, hd, dtype=BF, device="cuda") if cache else None
        caches.append((kc, torch.zeros_like(kc) if cache else None))
    dx, dw = x.cuda(), w.cuda()
    fused = linear_rope_qkv(dx, dw, b, cos, sin, nh, nkv, hd, *caches[0], slots)
    plain = rope_qkv(linear(dx, dw, b), cos, sin, nh, nkv, hd, *caches[1], slots)
    for name, a, r in zip("qkv", fused, plain):
        assert torch.equal(a, r), f"{name}: {(a.float() - r.float()).abs().max().item()}"
    if cache:
        assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])


@pytest.mark.parametrize("M,N,K", [(193, 1536, 1536), (1552, 1536, 1536), (1552, 1536, 8960), (1665, 2048, 4864),
                                   (8192, 1536, 1536)])
def test_tiled_residual_epilogue_equals_product_then_norm(hiplib, M, N, K):
    """Above 192 rows linear_residual_rms_norm adds the residual in the tiled kernel's epilogue and runs the
    RMSNorm kernel on the sum alone: the sum and the normalised rows are bit-identical to the plain product
    followed by the residual RMSNorm kernel (8960-long K: K-sliced plans merge before the epilogue)."""
    from nanoserve_amd.kernels.fused import rms_norm
    from nanoserve_amd.kernels.linear import linear, linear_residual_rms_norm
    x, w = operands(M, N, K, seed=M + K)
    g = cpu_gen(M + 1)
    res = torch.randn(M, N, generator=g).to(BF).cuda()
    nw = (1 + 0.1 * torch.randn(N, generator=g)).to(BF).cuda()
    dx, dw = x.cuda(), w.cuda()
    h, r = linear_residual_rms_norm(dx, dw, res, nw, 1e-6)
    h0, r0 = rms_norm(linear(dx, dw), nw, 1e-6, residual=res)
    assert torch.equal(r, r0), f"sum: {(r.float() - r0.float()).abs().max().item()}"
    assert torch.equal(h, h0), f"norm: {(h.float() - h0.float()).abs().max().item()}"
    none, r1 = linear_residual_rms_norm(dx, dw, res, None, 1e-6)
    assert none is None and torch.equal(r1, r0)

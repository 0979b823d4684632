"""HIP GEMMs above 64 rows (csrc/gemm.hip: prefill chunks, mixed steps, speculative verify batches) vs the
CPU oracle, with the gate of the skinny-kernel tests: >= 99% bitwise identical to the fp32-accumulated,
once-rounded product and every element within 1 bf16 ulp plus Higham's deterministic bound gamma_K * sum|x||w|
(for both sides), propagated through the SiLU epilogue. The product replaces F.linear at
nanoserve/model.py:231,256-257 on the large-token path. At 1552 rows the check covers every 128-row tile
(its first, middle and last rows and the partial last tile) and every column. Routes: up to 192 rows the
K <= 2048 projections run the tile-16 kernel in 16-token blocks and the 8960-long ones the skinny kernel in
64-row token blocks; otherwise the tiled kernel (1552 x 17920 on 256 x 256 tiles, the rest on 128 x 128,
K-sliced where K is long and the tiles are few).
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


@pytest.mark.parametrize("M", [65, 96, 120, 1552])
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


def test_tiled_rejects_normalised_input_through_the_c_abi(hiplib):
    """The C entry point refuses a normalised input above 64 rows (the Python layer materialises it)."""
    from nanoserve_amd import _lib
    x, w = operands(65, 256, 256, seed=3)
    xd, wd = x.cuda(), w.cuda()
    y = torch.empty(65, 256, dtype=BF, device="cuda")
    sq = torch.zeros(16, 64, device="cuda")
    nw = torch.ones(256, dtype=BF, device="cuda")
    rc = _lib.lib().ns_gemm(xd.data_ptr(), wd.data_ptr(), None, y.data_ptr(), 65, 256, 256, 1, sq.data_ptr(),
                            nw.data_ptr(), 1e-6, None, 0, _lib.stream_of(xd))
    assert rc != 0 and b"normalised" in _lib.lib().ns_last_error()

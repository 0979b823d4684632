"""Fragment-packed decode GEMMs (csrc/packed_gemm.hip) vs the CPU oracle.

The packed layout is restated here in numpy and compared byte for byte with what ns_pack_weight writes, for
every tile row order. Each packed projection is held to the gate of the row-major skinny kernels
(tests/test_gemm_kernels.py): >= 99% bitwise identical to the oracle's product rounded once, and every
element within 1 bf16 ulp plus Higham's bound for a different fp32 summation order, propagated through the
epilogue. Also: KV writes exact at the slots, the fused greedy argmax equals torch.argmax of the stored
logits, a normalised input equals its materialised norm bitwise, results are deterministic and a graph
replay equals the eager call. Shapes: the 1.5B decode projections at M = 1 .. 64 (QKV and O token-split
at M = 17 .. 32, down on ten K slices, gate/up and the LM head unsliced), the 0.5B and 3B ones, and odd
sizes; the K-sliced plans are exercised here even though the model routes them to the row-major kernels.
"""
import numpy as np
import pytest
import torch

from oracle import ops
from tests.conftest import cpu_gen
from tests.test_gemm_kernels import BF, bf16_check, dot_bound, operands, ref_linear, ulp

pytestmark = pytest.mark.gpu


def packed_layout(w: np.ndarray, order: int, hd: int = 0) -> np.ndarray:
    """The layout of csrc/packed_gemm.hip restated: tile t, step s, lane l holds 8 values
    W[row(t, l % 16)][32 s + 8 (l // 16) ...]; uint16 [tiles, steps, 64, 8]."""
    N, K = w.shape
    if order == 1:      # gate/up: 8 gate rows then the matching 8 up rows
        half = N // 2
        tiles = -(-half // 8)
        rows = [[min(8 * t + r, half - 1) if r < 8 else half + min(8 * t + r - 8, half - 1) for r in range(16)]
                for t in range(tiles)]
    elif order == 2:    # RoPE: 8 dims of a head and the 8 dims half a head further
        tph = hd // 16
        rows = [[(t // tph) * hd + 8 * (t % tph) + (r if r < 8 else hd // 2 + r - 8) for r in range(16)]
                for t in range(N // 16)]
    else:
        rows = [[min(16 * t + r, N - 1) for r in range(16)] for t in range(-(-N // 16))]
    rows = np.array(rows)                                     # [tiles, 16]
    steps = K // 32
    out = np.empty((len(rows), steps, 64, 8), dtype=np.uint16)
    for lane in range(64):
        kcols = 8 * (lane // 16) + np.arange(8)
        for s in range(steps):
            out[:, s, lane, :] = w[rows[:, lane % 16]][:, 32 * s + kcols]
    return out


@pytest.mark.parametrize("N,K,order,hd", [(100, 64, 0, 0), (2 * 56, 96, 1, 0), (2 * 60, 64, 1, 0), (8 * 128, 64, 2, 128),
                                          (6 * 64, 32, 2, 64)])
def test_pack_layout(hiplib, N, K, order, hd):
    from nanoserve_amd.kernels.linear import PackedWeight
    _, w = operands(1, N, K, seed=N + K)
    pw = PackedWeight(w.cuda(), order, hd)
    got = pw.p.cpu().numpy().view(np.uint16)
    want = packed_layout(w.view(torch.int16).numpy().view(np.uint16), order, hd).reshape(-1)
    assert got.shape == want.shape and np.array_equal(got, want)


def packed(w, order=0, hd=0):
    from nanoserve_amd.kernels.linear import PackedWeight
    return PackedWeight(w.cuda(), order, hd)


@pytest.fixture(autouse=True)
def every_packed_plan():
    """Run the packed kernels on every plan here, the K-sliced ones included (the model's routing sends
    sliced plans to the row-major kernels)."""
    from nanoserve_amd.kernels.linear import packed_sliced_plans
    with packed_sliced_plans():
        yield


@pytest.mark.parametrize("M", [1, 7, 16, 17, 32, 33, 64])
@pytest.mark.parametrize("N,K", [(2048, 1536), (1536, 8960), (17920, 1536), (1000, 896), (1536, 1536)])
def test_packed_linear(hiplib, M, N, K):
    from nanoserve_amd.kernels.linear import linear
    x, w = operands(M, N, K, seed=M + N)
    b = (torch.randn(N, generator=cpu_gen(1)) * 0.1).to(BF)
    pw, bd = packed(w), dot_bound(x, w)
    bf16_check(linear(x.cuda(), pw, b.cuda()), ref_linear(x, w, b), f"packed linear M={M} N={N} K={K}", bd)
    bf16_check(linear(x.cuda(), pw), ref_linear(x, w), f"packed linear (no bias) M={M} N={N} K={K}", bd)


@pytest.mark.parametrize("M", [1, 24, 32, 64])
@pytest.mark.parametrize("I,K", [(8960, 1536), (4864, 896), (11008, 2048), (100, 64)])
def test_packed_silu_mul(hiplib, M, I, K):
    from nanoserve_amd.kernels.linear import linear_silu_mul
    x, w = operands(M, 2 * I, K, seed=4, scale=2.0)
    gu = ref_linear(x, w)
    e = dot_bound(x, w) + ulp(gu)
    g_, u_ = gu[:, :I].float(), gu[:, I:].float()
    bound = (1.1 * u_.abs() + torch.nn.functional.silu(g_).abs() + 1.1 * e[:, I:]) * torch.maximum(e[:, :I], e[:, I:])
    bf16_check(linear_silu_mul(x.cuda(), packed(w, 1)), ops.silu_mul(gu), f"packed silu_mul M={M} I={I}", 2 * bound)


@pytest.mark.parametrize("M", [1, 20, 32, 64])
@pytest.mark.parametrize("N,K,norm", [(1536, 1536, True), (1536, 8960, True), (896, 4864, False), (2048, 11008, True),
                                      (1000, 512, True)])
def test_packed_residual_rms_norm(hiplib, M, N, K, norm):
    from nanoserve_amd.kernels.linear import linear_residual_rms_norm
    x, w = operands(M, N, K, seed=5)
    g = cpu_gen(6)
    res = torch.randn(M, N, generator=g).to(BF)
    nw = (1 + 0.1 * torch.randn(N, generator=g)).to(BF)
    h, r = linear_residual_rms_norm(x.cuda(), packed(w), res.cuda(), nw.cuda() if norm else None, 1e-6)
    y = ref_linear(x, w)
    ref_r = res + y
    e = dot_bound(x, w) + ulp(y)
    bf16_check(r, ref_r, "residual sum", e)
    if not norm:
        assert h is None
        return
    # the row statistics are the sums of the stored r^2 over each 16 columns (halves of 8, in order)
    rf = torch.nn.functional.pad(r.cpu().float(), (0, -N % 16)).view(M, -1, 2, 8)
    want = (rf.pow(2).sum(-1)[..., 0] + rf.pow(2).sum(-1)[..., 1]).T          # [N/16, M]
    got = h.sumsq.cpu()[:, :M]
    assert torch.allclose(got, want, rtol=1e-6, atol=0)
    ref_h = ops.rms_norm(r.cpu(), nw, 1e-6)
    same, ulps = ops.bf16_ulp_close(h.tensor().cpu(), ref_h)
    assert same >= 0.99 and ulps <= 1.0, (same, ulps)


@pytest.mark.parametrize("M", [1, 20, 32, 33, 64])
@pytest.mark.parametrize("nh,nkv,hd,K", [(12, 2, 128, 1536), (14, 2, 64, 896), (16, 2, 128, 2048), (4, 2, 64, 256)])
def test_packed_rope_qkv_and_cache_write(hiplib, M, nh, nkv, hd, K):
    from nanoserve_amd.kernels.linear import linear_rope_qkv
    N = (nh + 2 * nkv) * hd
    x, w = operands(M, N, K, seed=7)
    g = cpu_gen(8)
    b = (torch.randn(N, generator=g) * 0.1).to(BF)
    cos, sin = ops.rope_tables(torch.randint(0, 4000, (M,), generator=g), hd, 1e6, BF)
    slots = torch.randperm(16 * 16, generator=g)[:M]
    kc = torch.zeros(16, 16, nkv, hd, dtype=BF, device="cuda")
    vc = torch.zeros_like(kc)
    q, k, v = linear_rope_qkv(x.cuda(), packed(w, 2, hd), b.cuda(), cos.cuda(), sin.cuda(), nh, nkv, hd, kc, vc,
                              slots.cuda())
    rk, rv = torch.zeros(16, 16, nkv, hd, dtype=BF), torch.zeros(16, 16, nkv, hd, dtype=BF)
    qkv = ref_linear(x, w, b)
    q0, k0, v0 = ops.rope_qkv(qkv, cos, sin, nh, nkv, hd, rk, rv, slots)
    e = dot_bound(x, w) + ulp(qkv)
    eh = torch.maximum(e.view(M, -1, hd), e.view(M, -1, hd).roll(hd // 2, dims=-1))
    bound = 3 * eh
    bf16_check(q, q0, "q", bound[:, :nh] + 2 * ulp(q0))
    bf16_check(k, k0, "k", bound[:, nh:nh + nkv] + 2 * ulp(k0))
    bf16_check(v, v0, "v", e.view(M, -1, hd)[:, nh + nkv:])
    flat_k, flat_v = kc.cpu().view(-1, nkv, hd), vc.cpu().view(-1, nkv, hd)
    assert torch.equal(flat_k[slots], k.cpu()) and torch.equal(flat_v[slots], v.cpu())
    untouched = torch.ones(16 * 16, dtype=torch.bool)
    untouched[slots] = False
    assert not flat_k[untouched].any() and not flat_v[untouched].any()


@pytest.mark.parametrize("M,N,K", [(32, 151936, 1536), (1, 151936, 1536), (64, 20000, 896), (17, 151936, 2048)])
def test_packed_lm_head_argmax(hiplib, M, N, K):
    """The LM head with the greedy choice fused: logits within the GEMM gate, tokens == torch.argmax of the
    stored logits (first maximal index), on the normalised input the decode step hands it, and equal to the
    materialised norm's result bitwise."""
    from nanoserve_amd.kernels.linear import linear, linear_argmax, linear_residual_rms_norm
    x0, w0 = operands(M, K, 512, seed=20)
    res = torch.randn(M, K, generator=cpu_gen(21)).to(BF).cuda()
    nw = (1 + 0.1 * torch.randn(K, generator=cpu_gen(22))).to(BF).cuda()
    hn, _ = linear_residual_rms_norm(x0.cuda(), w0.cuda(), res, nw, 1e-6)
    h = hn.tensor()
    _, w = operands(M, N, K, seed=23)
    pw = packed(w)
    tok = torch.empty(M, dtype=torch.int64, device="cuda")
    y = linear_argmax(hn, pw, tok)
    hc = h.cpu()
    bf16_check(y, ref_linear(hc, w), f"packed lm head M={M} N={N} K={K}", dot_bound(hc, w))
    assert torch.equal(tok, y.float().argmax(-1))
    assert torch.equal(y, linear(h, pw))
    tok2 = torch.empty_like(tok)
    assert torch.equal(linear_argmax(h, pw, tok2), y) and torch.equal(tok2, tok)


def test_packed_argmax_ties_take_the_first_index(hiplib):
    """Rows whose maximum appears in several tiles (and workgroups): the first index, like torch.argmax."""
    from nanoserve_amd.kernels.linear import linear_argmax
    M, N, K = 4, 151936, 1536
    x = torch.zeros(M, K, dtype=BF)
    w = torch.zeros(N, K, dtype=BF)
    for m, cols in enumerate([[5, 100000], [151935, 7], [64000, 64001, 3], [150000]]):
        x[m, m] = 1.0
        w[cols, m] = 2.0      # row m's logits: 2 at its columns, 0 elsewhere
    tok = torch.empty(M, dtype=torch.int64, device="cuda")
    y = linear_argmax(x.cuda(), packed(w), tok)
    assert tok.tolist() == y.float().argmax(-1).tolist() == [5, 7, 3, 150000]


def test_packed_deterministic_and_graph_replay(hiplib):
    from nanoserve_amd.kernels.linear import linear, linear_residual_rms_norm, linear_silu_mul
    x, w = operands(32, 1536, 8960, seed=9)
    x2, wgu = operands(32, 2 * 8960, 1536, seed=10)
    res = torch.randn(32, 1536, generator=cpu_gen(11)).to(BF).cuda()
    nw = torch.ones(1536, dtype=BF, device="cuda")
    dx, dx2 = x.cuda(), x2.cuda()
    pw, pgu = packed(w), packed(wgu, 1)

    def step():
        a = linear(dx, pw)
        b = linear_silu_mul(dx2, pgu)
        h, r = linear_residual_rms_norm(dx, pw, res, nw, 1e-6)
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
        step()


@pytest.mark.parametrize("M", [1, 32, 64])
def test_packed_norm_on_load_equals_the_materialised_norm(hiplib, M):
    from nanoserve_amd.kernels.linear import linear, linear_residual_rms_norm, linear_rope_qkv, linear_silu_mul
    K = 1536
    x0, w0 = operands(M, K, 512, seed=12)
    res = torch.randn(M, K, generator=cpu_gen(13)).to(BF).cuda()
    nw = (1 + 0.1 * torch.randn(K, generator=cpu_gen(14))).to(BF).cuda()
    hn, _ = linear_residual_rms_norm(x0.cuda(), w0.cuda(), res, nw, 1e-6)
    h = hn.tensor()
    _, w = operands(M, 1000, K, seed=15)
    b = (torch.randn(1000, generator=cpu_gen(16)) * 0.1).to(BF).cuda()
    pw = packed(w)
    assert torch.equal(linear(hn, pw, b), linear(h, pw, b))
    _, wgu = operands(M, 2 * 1024, K, seed=17)
    pgu = packed(wgu, 1)
    assert torch.equal(linear_silu_mul(hn, pgu), linear_silu_mul(h, pgu))
    nh, nkv, hd = 12, 2, 128
    _, wq = operands(M, (nh + 2 * nkv) * hd, K, seed=18)
    pq = packed(wq, 2, hd)
    cos, sin = ops.rope_tables(torch.arange(M) + 7, hd, 1e6, BF)
    qa = linear_rope_qkv(hn, pq, None, cos.cuda(), sin.cuda(), nh, nkv, hd)
    qb = linear_rope_qkv(h, pq, None, cos.cuda(), sin.cuda(), nh, nkv, hd)
    for a_, b_ in zip(qa, qb):
        assert torch.equal(a_, b_)
    idx = torch.arange(M - 1, -1, -2, device="cuda")
    assert torch.equal(linear(hn.rows(idx), pw), linear(h[idx].contiguous(), pw))

"""The LM head with the greedy argmax fused (csrc/gemm.hip persist_gemm_kernel<..., AM = true>, ns_gemm_argmax):
F.linear(x, lm_head) (nanoserve/model.py:362) followed by logits.argmax(-1) (nanoserve/engine.py:239) in one
launch. The logits must equal the unfused LM head's bitwise and the tokens must equal ns_argmax_rows on them,
with torch.argmax's tie rules: the first maximal index (also when the tied rows sit in different tiles and
workgroups) and NaN above every number. Every launch leaves its keys and counter at zero, so
repeated calls (and a smaller batch after a larger one) start clean."""
import pytest
import torch

from nanoserve_amd import _lib

pytestmark = pytest.mark.gpu
BF = torch.bfloat16


def fused(x, w, tokens):
    from nanoserve_amd.kernels.linear import linear_argmax
    M = (x.r if hasattr(x, "r") else x).shape[0]
    assert _lib.lib().ns_gemm_argmax_fused(M, w.shape[0], w.shape[1]) == 1
    return linear_argmax(x, w, tokens)


def unfused(x, w):
    from nanoserve_amd.kernels.linear import linear
    from nanoserve_amd.kernels.sampling import argmax_rows
    y = linear(x, w)
    return y, argmax_rows(y)


def weights(N, K, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return (torch.randn(N, K, generator=g, device="cuda") * 0.05).to(BF)


@pytest.mark.parametrize("M", [1, 7, 16, 17, 32])
@pytest.mark.parametrize("N,K", [(151936, 1536), (65600, 896)])
def test_fused_equals_lm_head_then_argmax(hiplib, M, N, K):
    w = weights(N, K, seed=M)
    x = torch.randn(M, K, generator=torch.Generator(device="cuda").manual_seed(100 + M), device="cuda").to(BF)
    tok = torch.full((M,), -1, dtype=torch.int64, device="cuda")
    y = fused(x, w, tok)
    y_ref, tok_ref = unfused(x, w)
    assert torch.equal(y, y_ref)
    assert torch.equal(tok, tok_ref)
    assert torch.equal(tok.cpu(), y.float().argmax(-1).cpu())


def test_fused_with_normalised_input_and_pinned_tokens(hiplib):
    from nanoserve_amd.kernels.linear import NormedRows
    M, N, K = 32, 151936, 1536
    w = weights(N, K, seed=5)
    g = torch.Generator(device="cuda").manual_seed(6)
    r = torch.randn(M, K, generator=g, device="cuda").to(BF)
    sq = torch.zeros(K // 16, 64, device="cuda")
    sq[:, :M] = (r.float() ** 2).view(M, -1, 16).sum(-1).T
    nw = (1 + 0.1 * torch.randn(K, generator=g, device="cuda")).to(BF)
    x = NormedRows(r, sq, nw, 1e-6)
    tok = torch.full((M,), -1, dtype=torch.int64, pin_memory=True)
    y = fused(x, w, tok)
    torch.cuda.synchronize()
    y_ref, tok_ref = unfused(x, w)
    assert torch.equal(y, y_ref)
    assert torch.equal(tok, tok_ref.cpu())


def test_ties_zeros_and_nan_follow_torch_argmax(hiplib):
    M, N, K = 8, 151936, 1536
    w = weights(N, K, seed=7).abs()                     # positive weights and inputs: positive logits
    x = torch.randn(M, K, generator=torch.Generator(device="cuda").manual_seed(8), device="cuda").abs().to(BF)
    # one scaled weight row at four places in different tiles and workgroups -> equal maxima; the first wins
    w[1234] = w[5000] = w[40000] = w[140000] = 4 * w[1234]
    x[2] = 0          # an all-zero row: every logit +0 (the accumulators start at +0), index 0 wins
    x[3, 17] = float("nan")   # every logit NaN: index 0
    tok = torch.full((M,), -1, dtype=torch.int64, device="cuda")
    y = fused(x, w, tok)
    y_ref, tok_ref = unfused(x, w)
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))   # NaN-safe bitwise comparison
    assert torch.equal(tok, tok_ref)
    assert tok[0].item() == 1234 and tok[1].item() == 1234 and tok[2].item() == 0 and tok[3].item() == 0
    # a NaN in weight row 77777: that logit is NaN in every row (0 * NaN too) and ranks above every number
    w[77777, 5] = float("nan")
    y = fused(x, w, tok)
    y_ref, tok_ref = unfused(x, w)
    assert torch.equal(tok, tok_ref)
    t = tok.tolist()
    assert t[3] == 0 and all(v == 77777 for i, v in enumerate(t) if i != 3)


def test_repeated_calls_start_clean(hiplib):
    """Keys and counter are reset by every launch: a large batch, then a smaller one with lower maxima, then the
    large one again, each equal to the unfused result."""
    N, K = 151936, 1536
    w = weights(N, K, seed=9)
    g = torch.Generator(device="cuda").manual_seed(10)
    big = torch.randn(32, K, generator=g, device="cuda").to(BF) * 4
    small = torch.randn(5, K, generator=g, device="cuda").to(BF) * 0.25
    for x in (big, small, big, small):
        tok = torch.empty(x.shape[0], dtype=torch.int64, device="cuda")
        fused(x, w, tok)
        assert torch.equal(tok, unfused(x, w)[1])


def test_fused_entry_point_refuses_other_shapes(hiplib):
    lib = _lib.lib()
    assert lib.ns_gemm_argmax_fused(33, 151936, 1536) == 0      # more rows than the persistent kernel takes
    assert lib.ns_gemm_argmax_fused(32, 4096, 1536) == 0        # too few tiles to stay persistent
    assert lib.ns_gemm_argmax_fused(32, 151936, 4096) == 0      # K > 2048
    x = torch.zeros(33, 1536, dtype=BF, device="cuda")
    w = torch.zeros(151936, 1536, dtype=BF, device="cuda")
    y = torch.empty(33, 151936, dtype=BF, device="cuda")
    tok = torch.empty(33, dtype=torch.int64, device="cuda")
    ws = torch.zeros(1 << 18, dtype=torch.uint8, device="cuda")
    rc = lib.ns_gemm_argmax(x.data_ptr(), w.data_ptr(), y.data_ptr(), 33, 151936, 1536, 1, None, None, 0.0,
                            tok.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(x))
    assert rc == 1 and b"ns_gemm_argmax_fused" in lib.ns_last_error()

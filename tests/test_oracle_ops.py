"""Pins the CPU oracle's op-level functions (oracle/ops.py) to checks that do not retype them: an fp64
brute force with explicit slot arithmetic, closed forms evaluated in fp64, HF transformers' own modules,
known answers from the reference's tests, and invariants. Each pin is shown to be sensitive by planting a
plausible mistake in a copy of the oracle function and checking that the same comparison then fails.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import ops


def paged_case(n_heads, n_kv, hd, ctx, nb_extra=3, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    nblocks = sum(-(-c // 16) for c in ctx) + nb_extra
    k = torch.randn(nblocks, 16, n_kv, hd, generator=g).to(dtype)
    v = torch.randn(nblocks, 16, n_kv, hd, generator=g).to(dtype)
    q = torch.randn(len(ctx), n_heads, hd, generator=g).to(dtype)
    perm = torch.randperm(nblocks, generator=g)
    width = max(-(-c // 16) for c in ctx) + 2
    tables = torch.full((len(ctx), width), nblocks - 1, dtype=torch.int32)  # padding names a real block
    used = 0
    for i, c in enumerate(ctx):
        n = -(-c // 16)
        tables[i, :n] = perm[used:used + n].int()
        used += n
    return q, k, v, tables, torch.tensor(ctx, dtype=torch.int32)


CASES = [(14, 2, 64, [1, 16, 17, 40]), (12, 2, 128, [5, 33, 64]), (16, 2, 128, [2, 31]), (4, 4, 64, [19, 3])]


@pytest.mark.parametrize("n_heads,n_kv,hd,ctx", CASES)
def test_paged_reference_equals_fp64_brute_force(n_heads, n_kv, hd, ctx):
    q, k, v, t, c = paged_case(n_heads, n_kv, hd, ctx)
    ref = ops.paged_attention_reference(q, k, v, t, c, hd ** -0.5).double().numpy()
    bf = ops.paged_attention_fp64(q, k, v, t, c, hd ** -0.5)
    assert np.abs(ref - bf).max() < 1e-5


def test_single_token_context_returns_that_value_row():
    """tests/test_paged_attention_kernel.py:67-73 of the reference: ctx = 1 -> every head of the group
    gets V of the one slot."""
    q, k, v, t, c = paged_case(14, 2, 64, [1, 1])
    out = ops.paged_attention_reference(q, k, v, t, c, 0.125)
    for b in range(2):
        blk = int(t[b, 0])
        for h in range(14):
            assert torch.allclose(out[b, h], v[blk, 0, h // 7], atol=1e-6)


def test_paged_reference_is_independent_of_block_placement():
    q, k, v, t, c = paged_case(12, 2, 128, [50, 17])
    out = ops.paged_attention_reference(q, k, v, t, c, 0.1)
    perm = torch.randperm(k.shape[0], generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(len(perm))
    k2, v2 = k[perm], v[perm]                # block j of the new pool = old block perm[j]
    t2 = inv[t.long()].int()
    assert torch.equal(ops.paged_attention_reference(q, k2, v2, t2, c, 0.1), out)


def test_brute_force_catches_planted_mistakes():
    """The fp64 comparison above fails for plausible mistakes in the gather + SDPA oracle."""
    q, k, v, t, c = paged_case(14, 2, 64, [23, 40])
    bf = ops.paged_attention_fp64(q, k, v, t, c, 0.125)

    def gqa_interleaved(q, k_pool, v_pool, block_tables, context_lens, scale):   # head h -> kv h % nkv
        out = []
        for b in range(q.shape[0]):
            L = int(context_lens[b])
            blocks = block_tables[b, :-(-L // 16)].long()
            kk = k_pool[blocks].reshape(-1, 2, 64)[:L]
            vv = v_pool[blocks].reshape(-1, 2, 64)[:L]
            rows = []
            for h in range(q.shape[1]):
                p = torch.softmax(kk[:, h % 2] @ q[b, h] * scale, 0)
                rows.append(p @ vv[:, h % 2])
            out.append(torch.stack(rows))
        return torch.stack(out)

    def no_scale(*a):
        return ops.paged_attention_reference(*a[:-1], 1.0)

    def reads_whole_last_block(q, k_pool, v_pool, block_tables, context_lens, scale):
        full = torch.tensor([-(-int(x) // 16) * 16 for x in context_lens], dtype=torch.int32)
        return ops.paged_attention_reference(q, k_pool, v_pool, block_tables, full, scale)

    for wrong in (gqa_interleaved, no_scale, reads_whole_last_block):
        got = wrong(q, k, v, t, c, 0.125).double().numpy()
        assert np.abs(got - bf).max() > 1e-3, wrong.__name__


def test_causal_offset_attention_equals_fp64_brute_force():
    g = torch.Generator().manual_seed(3)
    T, ctx, H, KVH, D = 5, 11, 6, 2, 32
    q = torch.randn(T, H, D, generator=g)
    k = torch.randn(ctx + T, KVH, D, generator=g)
    v = torch.randn(ctx + T, KVH, D, generator=g)
    for c0 in (ctx, 0):
        kk, vv = (k, v) if c0 else (k[ctx:], v[ctx:])
        out = ops.causal_offset_attention(q, kk, vv, c0, D ** -0.5).double().numpy()
        qn, kn, vn = q.double().numpy(), kk.double().numpy(), vv.double().numpy()
        for j in range(T):
            for h in range(H):
                s = kn[:c0 + j + 1, h // (H // KVH)] @ qn[j, h] * D ** -0.5
                p = np.exp(s - s.max())
                want = (p[:, None] * vn[:c0 + j + 1, h // (H // KVH)]).sum(0) / p.sum()
                assert np.abs(out[j, h] - want).max() < 1e-5


def _bf16_round(x64: torch.Tensor) -> torch.Tensor:
    """Round fp64 values to bf16 with ties to even, via fp32 only where fp32 holds them exactly."""
    return x64.to(torch.float32).to(torch.bfloat16)


def test_silu_mul_equals_hf_activation_and_closed_form():
    from transformers.activations import ACT2FN
    g = torch.Generator().manual_seed(4)
    x = (torch.randn(16, 2 * 300, generator=g) * 3).to(torch.bfloat16)
    gate, up = x[:, :300], x[:, 300:]
    out = ops.silu_mul(x)
    assert torch.equal(out, ACT2FN["silu"](gate) * up)
    # closed form in fp64: round(round(g / (1 + e^-g)) * u)
    g64 = gate.double()
    s = _bf16_round(g64 / (1 + torch.exp(-g64)))
    want = _bf16_round(s.double() * up.double())
    same, ulps = ops.bf16_ulp_close(out, want)
    assert same >= 0.99 and ulps <= 1.0
    # planted mistake: no rounding after silu
    wrong = _bf16_round(g64 / (1 + torch.exp(-g64)) * up.double())
    assert (wrong != out).float().mean().item() > 0.02


def test_rope_qkv_bf16_equals_hf_rotary_and_writes_only_the_slots():
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    g = torch.Generator().manual_seed(5)
    N, nh, nkv, hd = 6, 12, 2, 128
    qkv = torch.randn(N, (nh + 2 * nkv) * hd, generator=g).to(torch.bfloat16)
    cos, sin = ops.rope_tables(torch.arange(40, 40 + N), hd, 1e6, torch.bfloat16)
    kc = torch.randn(4, 16, nkv, hd, generator=g).to(torch.bfloat16)
    vc = torch.randn(4, 16, nkv, hd, generator=g).to(torch.bfloat16)
    kc0, vc0 = kc.clone(), vc.clone()
    slots = torch.tensor([3, 17, 18, 40, 63, 0])
    q, k, v = ops.rope_qkv(qkv, cos, sin, nh, nkv, hd, kc, vc, slots)
    qh = qkv[:, :nh * hd].reshape(N, nh, hd).transpose(0, 1)[None]
    kh = qkv[:, nh * hd:(nh + nkv) * hd].reshape(N, nkv, hd).transpose(0, 1)[None]
    q_hf, k_hf = apply_rotary_pos_emb(qh, kh, cos[None], sin[None])
    assert torch.equal(q, q_hf[0].transpose(0, 1)) and torch.equal(k, k_hf[0].transpose(0, 1))
    assert torch.equal(v, qkv[:, (nh + nkv) * hd:].reshape(N, nkv, hd))
    flat_k, flat_v = kc.view(-1, nkv, hd), vc.view(-1, nkv, hd)
    assert torch.equal(flat_k[slots], k) and torch.equal(flat_v[slots], v)
    untouched = torch.ones(64, dtype=torch.bool)
    untouched[slots] = False
    assert torch.equal(flat_k[untouched], kc0.view(-1, nkv, hd)[untouched])
    assert torch.equal(flat_v[untouched], vc0.view(-1, nkv, hd)[untouched])


def test_rms_norm_residual_add_is_the_exactly_rounded_sum():
    g = torch.Generator().manual_seed(6)
    x = torch.randn(5, 896, generator=g).to(torch.bfloat16)
    r = torch.randn(5, 896, generator=g).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(896, generator=g)).to(torch.bfloat16)
    out, res = ops.rms_norm_residual(x, w, 1e-6, r)
    assert torch.equal(res, _bf16_round(x.double() + r.double()))
    # the normalised output in fp64 closed form, rounded where the HF order rounds
    rd = res.double()
    normed = _bf16_round(rd * torch.rsqrt((rd * rd).mean(-1, keepdim=True) + 1e-6))
    want = _bf16_round(w.double() * normed.double())
    same, ulps = ops.bf16_ulp_close(out, want)
    assert same >= 0.99 and ulps <= 1.0


def test_rms_norm_fp32_closed_form_and_planted_mistake():
    g = torch.Generator().manual_seed(7)
    x = torch.randn(3, 1536, generator=g) * 2
    w = 1 + 0.1 * torch.randn(1536, generator=g)
    out = ops.rms_norm(x, w, 1e-6).double()
    xd = x.double()
    want = w.double() * xd / torch.sqrt((xd * xd).mean(-1, keepdim=True) + 1e-6)
    assert (out - want).abs().max().item() < 1e-5
    wrong = w.double() * xd / torch.sqrt((xd * xd).sum(-1, keepdim=True) / 1535 + 1e-6)   # n - 1
    assert (wrong - want).abs().max().item() > 1e-4


def test_kv_bytes_per_token_known_answer():
    """tests/test_model.py:24 of the reference: 0.5B shape -> 12,288 bytes per token in bf16."""
    assert ops.kv_bytes_per_token(24, 2, 64, 2) == 12288
    assert ops.cdiv(17, 16) == 2 and ops.cdiv(16, 16) == 1 and ops.cdiv(0, 16) == 0

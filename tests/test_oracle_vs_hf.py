"""Pins the CPU oracle against an independent implementation: HF transformers' Qwen2 (built locally from a
Qwen2Config with the same random weights; no download). The reference gates its own forward the same way
(tests/test_model.py:36-64, tests/test_engine.py:45-50): RoPE tables bitwise equal to Qwen2RotaryEmbedding,
RMSNorm equal to Qwen2RMSNorm, fp32 logits within 1e-3, greedy tokens identical to HF generate.
Plus the decode-step invariant: prefill + token-by-token decode == one full forward (tests/test_kv_cache.py).
"""
import pytest
import torch

from nanoserve_amd.model import ModelConfig, random_state_dict
from oracle import ops
from oracle.model import OracleModel

TINY = ModelConfig(vocab_size=300, hidden_size=64, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=16,
                   intermediate_size=96, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)


def hf_model(cfg: ModelConfig, sd):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    hc = Qwen2Config(vocab_size=cfg.vocab_size, hidden_size=cfg.hidden_size, num_hidden_layers=cfg.n_layers,
                     num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv_heads,
                     intermediate_size=cfg.intermediate_size, rope_theta=cfg.rope_theta,
                     rms_norm_eps=cfg.rms_norm_eps, tie_word_embeddings=cfg.tie_word_embeddings,
                     max_position_embeddings=4096, attn_implementation="eager")
    m = Qwen2ForCausalLM(hc).eval()
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and all(k == "lm_head.weight" for k in missing)
    return m


@pytest.fixture(scope="module")
def tiny():
    sd = random_state_dict(TINY, seed=0, dtype=torch.float32)
    return sd, OracleModel(TINY, sd), hf_model(TINY, sd)


def test_rope_tables_equal_hf_bitwise():
    from transformers import Qwen2Config
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RotaryEmbedding
    for hd, dt in ((64, torch.float32), (128, torch.bfloat16)):
        hc = Qwen2Config(hidden_size=hd * 4, num_attention_heads=4, rope_theta=1e6, max_position_embeddings=8192)
        rot = Qwen2RotaryEmbedding(hc)
        pos = torch.randint(0, 4000, (1, 37))
        c_hf, s_hf = rot(torch.zeros(1, dtype=dt), pos)
        c, s = ops.rope_tables(pos[0], hd, 1e6, dt)
        assert torch.equal(c, c_hf[0]) and torch.equal(s, s_hf[0])


def test_rms_norm_equals_hf():
    from transformers.models.qwen2.modeling_qwen2 import Qwen2RMSNorm
    g = torch.Generator().manual_seed(0)
    for dt in (torch.float32, torch.bfloat16):
        x = (torch.randn(9, 896, generator=g) * 3).to(dt)
        n = Qwen2RMSNorm(896, eps=1e-6)
        with torch.no_grad():
            n.weight.copy_(1 + 0.1 * torch.randn(896, generator=g))
        n = n.to(dt)
        assert torch.equal(ops.rms_norm(x, n.weight.data, 1e-6), n(x))


def test_apply_rope_equals_hf():
    from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb
    g = torch.Generator().manual_seed(1)
    q, k = torch.randn(1, 4, 7, 64, generator=g), torch.randn(1, 2, 7, 64, generator=g)
    cos, sin = ops.rope_tables(torch.arange(3, 10), 64, 1e6, torch.float32)
    qh, kh = apply_rotary_pos_emb(q, k, cos[None], sin[None])
    assert torch.equal(ops.apply_rope(q[0].transpose(0, 1), cos, sin), qh[0].transpose(0, 1))
    assert torch.equal(ops.apply_rope(k[0].transpose(0, 1), cos, sin), kh[0].transpose(0, 1))


def test_fp32_logits_match_hf(tiny):
    _, orc, hf = tiny
    ids = torch.randint(0, TINY.vocab_size, (1, 23), generator=torch.Generator().manual_seed(2))
    with torch.no_grad():
        ref = hf(ids).logits[0]
    ours = orc.step([(orc.new_cache(64), ids[0].tolist())], all_logits=True)
    assert (ours - ref).abs().max().item() < 1e-4


def test_greedy_tokens_match_hf_generate(tiny):
    _, orc, hf = tiny
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, TINY.vocab_size, (n,), generator=g).tolist() for n in (5, 17, 33)]
    ours = orc.generate_greedy(prompts, 12)
    for p, toks in zip(prompts, ours):
        with torch.no_grad():
            out = hf.generate(torch.tensor([p]), max_new_tokens=12, do_sample=False, eos_token_id=None,
                              pad_token_id=0)
        assert out[0, len(p):].tolist() == toks


def test_prefill_then_decode_equals_full_forward(tiny):
    _, orc, _ = tiny
    ids = torch.randint(0, TINY.vocab_size, (30,), generator=torch.Generator().manual_seed(4)).tolist()
    full = orc.step([(orc.new_cache(64), ids)], all_logits=True)
    c = orc.new_cache(64)
    orc.step([(c, ids[:20])])
    steps = [orc.step([(c, [t])])[0] for t in ids[20:]]
    assert (torch.stack(steps) - full[20:]).abs().max().item() < 1e-5


def test_chunked_continuation_equals_token_by_token(tiny):
    """Several new tokens on a cached context (causal-offset mask) == one token at a time
    (tests/test_paged_engine.py:79-105)."""
    _, orc, _ = tiny
    ids = torch.randint(0, TINY.vocab_size, (24,), generator=torch.Generator().manual_seed(5)).tolist()
    c1, c2 = orc.new_cache(64), orc.new_cache(64)
    orc.step([(c1, ids[:16])])
    orc.step([(c2, ids[:16])])
    together = orc.step([(c1, ids[16:])], all_logits=True)
    one_by_one = torch.stack([orc.step([(c2, [t])])[0] for t in ids[16:]])
    assert torch.equal(together.argmax(-1), one_by_one.argmax(-1))
    assert (together - one_by_one).abs().max().item() < 1e-4


def test_batched_step_equals_alone(tiny):
    _, orc, _ = tiny
    g = torch.Generator().manual_seed(6)
    prompts = [torch.randint(0, TINY.vocab_size, (n,), generator=g).tolist() for n in (9, 14)]
    caches = [orc.new_cache(64) for _ in prompts]
    together = orc.step([(c, p) for c, p in zip(caches, prompts)])
    alone = torch.stack([orc.step([(orc.new_cache(64), p)])[0] for p in prompts])
    assert (together - alone).abs().max().item() < 1e-4

"""Greedy speculative decoding on the HIP path (nanoserve/speculative.py semantics), with the reference's
own gates (tests/test_speculative.py:1-12):
  * self-speculation (draft == target), fp32, graphed: acceptance >= 95 % and output identical to plain
    greedy decoding of the target;
  * a different draft model, fp32: output identical to plain greedy decoding of the target, which itself
    follows the CPU oracle;
  * bf16: the fp32 oracle on the same weights, teacher-forced at every position, a disagreement allowed
    only within twice the shape's logit-error bound (tests/parity.py);
  * batched requests give the same tokens as one request at a time.
Random-init models (vocab 2048) stand in for the hub checkpoints, which are not available offline.
"""
import pytest
import torch

from nanoserve_amd.model import ModelConfig, Qwen2Model, random_state_dict
from oracle.model import OracleModel
from tests.parity import DELTA_SMALL128, check_streams

pytestmark = pytest.mark.gpu

TARGET = ModelConfig(vocab_size=2048, hidden_size=256, n_layers=3, n_heads=4, n_kv_heads=2, head_dim=64,
                     intermediate_size=512, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
DRAFT = ModelConfig(vocab_size=2048, hidden_size=128, n_layers=2, n_heads=2, n_kv_heads=1, head_dim=64,
                    intermediate_size=256, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
TARGET128 = ModelConfig(vocab_size=2048, hidden_size=768, n_layers=2, n_heads=6, n_kv_heads=2, head_dim=128,
                        intermediate_size=1024, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
MAX_NEW = 24


def prompts(n, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 2048, (int(torch.randint(20, 90, (1,), generator=g)),), generator=g).tolist()
            for _ in range(n)]


def model(cfg, seed, dtype):
    return Qwen2Model(cfg, random_state_dict(cfg, seed=seed, dtype=dtype, device="cuda"))


def spec(target, draft, ps, k=4, max_num_seqs=1, **kw):
    from nanoserve_amd.speculative import SpeculativeEngine
    eng = SpeculativeEngine(target, draft, [], num_speculative_tokens=k, max_seq_len=256, max_num_seqs=max_num_seqs,
                            **kw)
    ids = {eng.add_request(p, MAX_NEW, ignore_eos=True): i for i, p in enumerate(ps)}
    outs = {i: [] for i in range(len(ps))}
    while eng.has_unfinished():
        for o in eng.step():
            outs[ids[o.seq_id]].append(o.token)
    for lane in eng.lanes:
        assert lane.pool.allocator.num_free == lane.pool.num_blocks - (1 if lane.graphs is not None else 0)
    return [outs[i] for i in range(len(ps))], eng.stats


def plain(target, ps):
    from nanoserve_amd.engine import LLMEngine
    eng = LLMEngine(target, [], max_seq_len=256, max_num_seqs=1, batch_wait_s=0.0, kv_cache_tokens=4096)
    outs = []
    for p in ps:
        sid = eng.add_request(p, MAX_NEW, ignore_eos=True)
        got = []
        while eng.has_unfinished():
            got += [o.token for o in eng.step() if o.seq_id == sid]
        outs.append(got)
    return outs


def test_fp32_self_speculation_is_identical_and_accepts_almost_everything(hiplib):
    m = model(TARGET, 0, torch.float32)
    ps = prompts(3, 1)
    out, st = spec(m, m, ps)
    print(f"self-speculation fp32: acceptance {st['acceptance_rate']:.3f}, verify graph steps "
          f"{st['graph_verify_steps']}, draft graph steps {st['graph_draft_steps']}")
    assert st["graph_verify_steps"] > 0 and st["graph_draft_steps"] > 0
    assert st["acceptance_rate"] >= 0.95
    assert out == plain(m, ps)


def test_fp32_draft_to_target_equals_plain_greedy_and_the_oracle(hiplib):
    sd = random_state_dict(TARGET, seed=2, dtype=torch.float32)
    target = Qwen2Model(TARGET, {k: v.cuda() for k, v in sd.items()})
    draft = model(DRAFT, 3, torch.float32)
    ps = prompts(4, 4)
    out, st = spec(target, draft, ps, k=3)
    print(f"draft -> target fp32: acceptance {st['acceptance_rate']:.3f}, "
          f"{st['tokens_per_target_forward']:.2f} tokens per verification")
    ref = plain(target, ps)
    assert out == ref
    orc = OracleModel(TARGET, sd)
    assert ref == [orc.generate_greedy([p], MAX_NEW)[0] for p in ps]


def test_batched_speculation_equals_one_request_at_a_time(hiplib):
    target, draft = model(TARGET, 5, torch.float32), model(DRAFT, 6, torch.float32)
    ps = prompts(5, 7)
    alone, _ = spec(target, draft, ps, max_num_seqs=1)
    together, st = spec(target, draft, ps, max_num_seqs=8)
    assert st["peak_running"] > 1
    assert together == alone


def test_bf16_speculation_follows_the_oracle(hiplib):
    sd = random_state_dict(TARGET128, seed=8, dtype=torch.bfloat16)
    target = Qwen2Model(TARGET128, {k: v.cuda() for k, v in sd.items()})
    ps = prompts(4, 9)
    out, st = spec(target, target, ps, max_num_seqs=4)
    print(f"bf16 self-speculation: acceptance {st['acceptance_rate']:.3f}")
    assert st["acceptance_rate"] >= 0.8
    orc = OracleModel(TARGET128, sd, dtype=torch.float32)
    # the verify steps' logits are not exposed: a disagreement passes only within 2x the shape's bound
    check_streams("bf16 self-speculation", ps, out, orc, delta_max=DELTA_SMALL128, min_identical=len(ps) - 1,
                  min_agree=0.98)

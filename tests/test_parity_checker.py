"""The bf16 stream checker of the GPU tests (tests/parity.py), pinned on the CPU.

The candidate here is the oracle itself run in bf16 (the reference algorithm at the GPU path's precision),
with and without mistakes planted in it; the checker compares it with the fp32 oracle exactly as the GPU
tests compare the HIP engine:
  * each per-shape bound stays within 1.5-3x of the reference algorithm's own bf16 error at that shape,
    re-measured here, and the correct bf16 candidate passes;
  * a wrong GQA head map in one layer fails (max |dlogit| far above the bound);
  * a token that is not the oracle's argmax fails unless the oracle's gap is within 2x the logit error, and
    a token that is not a maximum of the run's own logits fails;
  * too few agreeing positions or identical streams fail;
  * a dropped bf16 rounding inside RoPE stays below the model-level bound (it is smaller than the rounding
    differences between two correct bf16 implementations) and is caught by the op-level bitwise gate that
    tests/test_fused_ops.py applies to the RoPE kernel.
"""
import dataclasses

import pytest
import torch

from nanoserve_amd.model import QWEN25_1_5B, ModelConfig, random_state_dict
from oracle import ops
from oracle.model import OracleModel
from tests.parity import DELTA_1P5B_2L, DELTA_SMALL, DELTA_SMALL128, ParityFailure, check_streams

SMALL = ModelConfig(vocab_size=2048, hidden_size=256, n_layers=2, n_heads=4, n_kv_heads=2, head_dim=64,
                    intermediate_size=512, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
SMALL128 = ModelConfig(vocab_size=2048, hidden_size=768, n_layers=2, n_heads=6, n_kv_heads=2, head_dim=128,
                       intermediate_size=1024, rope_theta=1e6, rms_norm_eps=1e-6, tie_word_embeddings=True)
C3_2L = dataclasses.replace(QWEN25_1_5B, n_layers=2)


class WrongGQAMap(OracleModel):
    """Layer 1 pairs query head h with KV head h mod n_kv instead of h // (n_heads / n_kv)."""

    def attend(self, layer, q, ks, vs, ctx_len):
        if layer != 1:
            return super().attend(layer, q, ks, vs, ctx_len)
        g = q.shape[1] // ks.shape[1]
        return super().attend(layer, q, ks.repeat(1, g, 1), vs.repeat(1, g, 1), ctx_len)


def rope_unrounded(x, cos, sin):
    """RoPE with the three bf16 roundings of nanoserve/kernels/fused.py:87-104 dropped (fp32, one rounding)."""
    return (x.float() * cos.float()[:, None] + ops.rotate_half(x).float() * sin.float()[:, None]).to(x.dtype)


class DroppedRopeRounding(OracleModel):
    def rope(self, layer, x, cos, sin):
        return rope_unrounded(x, cos, sin) if layer == 0 else super().rope(layer, x, cos, sin)


def prompts(n, lo, hi, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, vocab, (int(torch.randint(lo, hi, (1,), generator=g)),), generator=g).tolist()
            for _ in range(n)]


def bf16_run(cls, cfg, sd, ps, n_new):
    """Greedy streams and their logits of the candidate (cls in bf16), like the engine's LogitsRecorder."""
    streams, logits = cls(cfg, sd, torch.bfloat16).generate_greedy(ps, n_new, return_logits=True)
    return streams, logits


@pytest.fixture(scope="module")
def small():
    sd = random_state_dict(SMALL, seed=3, dtype=torch.bfloat16)
    ps = prompts(6, 40, 160, SMALL.vocab_size, seed=4)
    ours, lg = bf16_run(OracleModel, SMALL, sd, ps, 12)
    orc = OracleModel(SMALL, sd, torch.float32)
    return sd, ps, ours, lg, orc, orc.teacher_forced(ps, ours)


@pytest.mark.parametrize("cfg,bound,plen,n", [(SMALL, DELTA_SMALL, (60, 200), 6), (SMALL128, DELTA_SMALL128, (20, 90), 6),
                                            (C3_2L, DELTA_1P5B_2L, (128, 129), 3)],
                         ids=["small", "small128", "1.5b-2-layers"])
def test_bounds_track_the_reference_algorithms_bf16_error(cfg, bound, plen, n):
    torch.manual_seed(0)
    sd = random_state_dict(cfg, seed=3, dtype=torch.bfloat16)
    ps = prompts(n, plen[0], plen[1], cfg.vocab_size, seed=4)
    ours, lg = bf16_run(OracleModel, cfg, sd, ps, 8)
    rec = check_streams(f"reference algorithm in bf16 ({cfg.hidden_size})", ps, ours,
                        OracleModel(cfg, sd, torch.float32), delta_max=bound, min_identical=0, min_agree=0.9,
                        ours_logits=lg)
    assert 1.5 <= bound / rec["delta_max"] <= 3.0, f"bound {bound} vs measured {rec['delta_max']}"


def test_wrong_gqa_head_map_in_one_layer_fails(small):
    sd, ps, _, _, orc, _ = small
    ours, lg = bf16_run(WrongGQAMap, SMALL, sd, ps, 12)
    with pytest.raises(ParityFailure, match="exceeds the bound"):
        check_streams("planted: GQA map", ps, ours, orc, delta_max=DELTA_SMALL, min_identical=0, min_agree=0.0,
                      ours_logits=lg)


def test_a_token_far_from_the_argmax_fails(small):
    sd, ps, ours, lg, orc, ref = small
    rec = check_streams("correct bf16", ps, ours, orc, delta_max=DELTA_SMALL, min_identical=len(ps) - 1,
                        min_agree=0.95, ours_logits=lg, ref_logits=ref)
    assert all(d["gap"] <= 2 * d["delta"] for d in rec["disagreements"])   # genuine near-ties only
    # position 5 of stream 2 takes the oracle's 10th-best token: its gap is far above 2x the logit error
    bad = [list(s) for s in ours]
    tenth = int(ref[2][5].float().topk(10).indices[-1])
    bad[2][5] = tenth
    with pytest.raises(ParityFailure, match="oracle gap"):
        check_streams("planted: wrong token", ps, bad, orc, delta_max=DELTA_SMALL, min_identical=0, min_agree=0.0)
    # the same token with the run's logits: it is not a maximum of them either
    with pytest.raises(ParityFailure, match="not a maximum of the run's own logits"):
        check_streams("planted: wrong token", ps, bad, orc, delta_max=DELTA_SMALL, min_identical=0, min_agree=0.0,
                      ours_logits=lg)


def test_agreement_floors_fail_when_too_few_positions_agree(small):
    sd, ps, ours, lg, orc, ref = small
    with pytest.raises(ParityFailure, match="streams identical"):
        check_streams("floors", ps, ours, orc, delta_max=DELTA_SMALL, min_identical=len(ps) + 1, min_agree=1.0,
                      ours_logits=lg, ref_logits=ref)
    # a run that takes the oracle's second choice at every position of stream 0 (within the gap rule only if
    # the gap is small): the agreement floor catches it even where the gap rule alone would not
    bad = [list(s) for s in ours]
    bad[0] = [int(ref[0][j].float().topk(2).indices[1]) for j in range(len(bad[0]))]
    with pytest.raises(ParityFailure, match="positions agree"):
        check_streams("floors", ps, bad, orc, delta_max=10.0, min_identical=0, min_agree=0.9, ref_logits=ref)


def test_dropped_rope_rounding_is_below_the_model_gate_and_fails_the_op_gate(small):
    sd, ps, _, _, orc, _ = small
    ours, lg = bf16_run(DroppedRopeRounding, SMALL, sd, ps, 12)
    rec = check_streams("planted: RoPE rounding", ps, ours, orc, delta_max=DELTA_SMALL, min_identical=0,
                        min_agree=0.9, ours_logits=lg)
    assert rec["delta_max"] <= DELTA_SMALL
    # the op-level gate: RoPE outputs are compared bitwise with the oracle's rope_qkv
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(32, 8 * 64, generator=g).to(torch.bfloat16)
    cos, sin = ops.rope_tables(torch.arange(100, 132), 64, 1e6, torch.bfloat16)
    q, k, _ = ops.rope_qkv(qkv, cos, sin, 4, 2, 64)
    q_bad = rope_unrounded(qkv[:, :256].reshape(32, 4, 64), cos, sin)
    assert not torch.equal(q_bad, q)
    assert (q_bad != q).float().mean().item() > 0.05

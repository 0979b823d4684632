"""The CPU oracle against the reference's own output: BASELINE config 1 (Qwen2.5-0.5B architecture,
random_state_dict(seed=0), fp32, 4 prompts of 128 tokens, 32 greedy steps) as nanoserve's LLMEngine produced
it on its fp32 CPU path (tests/golden/config1_fp32_streams.json, written by tests/golden/make_golden.py).
The oracle's greedy streams must be identical token for token; the GPU engine's are checked against the same
fixture in tests/test_model_engine_gpu.py."""
import json
from pathlib import Path

import torch

from nanoserve_amd.model import QWEN25_0_5B, random_state_dict
from oracle.model import OracleModel

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "config1_fp32_streams.json").read_text())


def test_fixture_prompts_are_the_seeded_config1_prompts():
    g = torch.Generator().manual_seed(1)
    assert GOLDEN["prompts"] == [torch.randint(0, 151936, (128,), generator=g).tolist() for _ in range(4)]
    assert [len(s) for s in GOLDEN["streams"]] == [32] * 4


def test_oracle_greedy_streams_equal_the_reference_engine():
    orc = OracleModel(QWEN25_0_5B, random_state_dict(QWEN25_0_5B, seed=0, dtype=torch.float32))
    assert orc.generate_greedy(GOLDEN["prompts"], 32) == GOLDEN["streams"]

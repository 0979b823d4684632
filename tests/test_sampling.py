"""Token selection: HIP argmax vs torch.argmax (first maximal index, NaN highest; the `logits.argmax(-1)`
of nanoserve/engine.py:239), the splitmix64 seed mixer and parameter validation (CPU), and the seeded
sampler's statistics on the GPU (the reference's tests/test_sampling.py:22-80 procedure: empirical
frequencies over many draws vs softmax(logits / T), top-k / top-p support, per-request reproducibility)."""
import pytest
import torch

from nanoserve_amd.sampling import SamplingParams, mix_seed
from tests.conftest import cpu_gen


def test_mix_seed_known_answers():
    # splitmix64 finaliser (Steele, Lea & Flood 2014) of seed * golden + step + 1, top bit cleared
    def ref(seed, step):
        m = (1 << 64) - 1
        z = (seed * 0x9E3779B97F4A7C15 + step + 1) & m
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        return (z ^ (z >> 31)) & ((1 << 63) - 1)
    # the public splitmix64 generator seeded with 0 first finalises the golden gamma itself, giving
    # 0xE220A8397B1DCDAF; mix_seed finalises seed * gamma + step + 1, i.e. the gamma at seed 1, step -1
    assert mix_seed(1, -1) == 0xE220A8397B1DCDAF & ((1 << 63) - 1)
    for seed, step in ((0, 0), (1, 5), (123456789, 42), (2 ** 61, 7)):
        assert mix_seed(seed, step) == ref(seed, step)
    assert len({mix_seed(7, n) for n in range(1000)}) == 1000


def test_sampling_params_validation():
    assert SamplingParams().greedy and SamplingParams(temperature=1.0, top_k=1).greedy
    assert not SamplingParams(temperature=0.7).greedy
    for bad in ({"temperature": -1.0}, {"top_p": 0.0}, {"top_p": 1.5}, {"top_k": -1}):
        with pytest.raises(ValueError):
            SamplingParams(**bad)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("V", [151936, 1000, 7, 8])
def test_argmax_rows_matches_torch(hiplib, dtype, V):
    from nanoserve_amd.kernels.sampling import argmax_rows
    g = cpu_gen(0)
    x = torch.randn(37, V, generator=g).to(dtype)
    x[3, :] = 1.0                                  # all equal: first index
    x[4, V // 2] = x[4].max() + 1
    x[4, V - 1] = x[4, V // 2]                     # tie between two maxima: the first
    x[5, min(2, V - 1)] = float("nan")             # NaN wins
    x[6, :] = float("-inf")
    ref = x.argmax(-1)
    assert torch.equal(argmax_rows(x.cuda()).cpu(), ref)
    assert torch.equal(argmax_rows(x.cuda()).cpu(), ref)     # the split path's counters are back at zero


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_argmax_rows_split_boundaries(hiplib, dtype):
    """Row splits: maxima placed on every split boundary, ties across splits (the first index wins), NaN in
    the last split, a row of one value, and the same call without a workspace (one workgroup per row)."""
    from nanoserve_amd import _lib
    from nanoserve_amd.kernels.sampling import argmax_rows
    g = cpu_gen(5)
    R, V = 32, 151936
    x = torch.randn(R, V, generator=g).to(dtype)
    vec = 8 if dtype == torch.bfloat16 else 4
    splits = min(512 // R, V // 2048, 64)
    bounds = [((k * (V // vec)) // splits) * vec for k in range(1, splits)]
    for r, bnd in enumerate(bounds[: R // 2]):
        x[r, bnd - 1] = 10.0 + r                  # last element of split k-1 ...
        x[r, bnd] = 10.0 + r                      # ... ties with the first of split k: the earlier wins
    x[20, -1] = float("nan")
    x[21, :] = 3.0
    x[22, 5] = 50.0
    x[22, V - 5] = 50.0
    ref = x.argmax(-1)
    xd = x.cuda()
    assert torch.equal(argmax_rows(xd).cpu(), ref)
    out = torch.empty(R, dtype=torch.int64, device="cuda")
    assert _lib.lib().ns_argmax_rows(xd.data_ptr(), xd.stride(0), R, V, _lib.dtype_code(xd), out.data_ptr(), None, 0,
                                     _lib.stream_of(xd)) == 0
    assert torch.equal(out.cpu(), ref)


@pytest.mark.gpu
def test_sampling_statistics_and_reproducibility(hiplib):
    from nanoserve_amd.sampling import sample
    logits = torch.tensor([2.0, 1.0, 0.5, 0.0, -1.0, -3.0]).cuda()
    R = 20000
    batch = logits[None].expand(R, -1).contiguous()
    for params, support in ((SamplingParams(temperature=0.8), range(6)),
                            (SamplingParams(temperature=1.0, top_k=3), range(3)),
                            (SamplingParams(temperature=1.0, top_p=0.7), range(2))):
        toks = sample(batch, [params] * R, list(range(R)), [0] * R)
        counts = torch.bincount(torch.tensor(toks), minlength=6).float() / R
        assert set(t for t in toks) <= set(support)
        p = torch.softmax(logits.cpu() / params.temperature, -1)
        if params.top_k:
            p = torch.where(torch.arange(6) < params.top_k, p, torch.zeros(()))
        if params.top_p < 1:
            p = torch.where(torch.arange(6) < len(support), p, torch.zeros(()))
        p = p / p.sum()
        assert (counts - p).abs().max().item() < 0.02, (params, counts, p)
    a = sample(batch[:50], [SamplingParams(temperature=1.0)] * 50, list(range(50)), [3] * 50)
    b = sample(batch[:50], [SamplingParams(temperature=1.0)] * 50, list(range(50)), [3] * 50)
    assert a == b                                     # same (seed, step) -> same draw
    greedy = sample(batch[:4], [None, SamplingParams(), None, None], [0] * 4, [0] * 4)
    assert greedy == [0, 0, 0, 0]

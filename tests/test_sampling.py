"""Greedy token selection: HIP argmax vs torch.argmax (first maximal index, NaN highest; the
`logits.argmax(-1)` of nanoserve/engine.py:239), split boundaries and ties, the kernel without a workspace,
and a workspace that grows after a graph captured the old one."""
import pytest
import torch

from tests.conftest import cpu_gen


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
def test_argmax_graph_survives_workspace_growth(hiplib):
    """A graph captured with the split argmax records its workspace address. An eager call over more rows
    than that workspace covers makes the wrapper allocate a larger one; the captured graph must still read
    and write memory that is its own, so replays keep matching torch.argmax."""
    from nanoserve_amd.kernels import sampling as smp
    from nanoserve_amd.kernels.sampling import argmax_rows
    V = 151936
    g = cpu_gen(9)
    x8 = torch.randn(8, V, generator=g).to(torch.bfloat16).cuda()
    out8 = torch.empty(8, dtype=torch.int64, device="cuda")
    argmax_rows(x8, out8)                                       # eager warm-up sizes the workspace
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        argmax_rows(x8, out8)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        argmax_rows(x8, out8)
    before = smp._WS[torch.cuda.current_device()].data_ptr()
    big = torch.randn(2048, V // 8, generator=g).to(torch.bfloat16).cuda()
    assert torch.equal(argmax_rows(big).cpu(), big.cpu().argmax(-1))   # grows the workspace
    grown = smp._WS[torch.cuda.current_device()].data_ptr() != before
    junk = torch.full((1 << 22,), -1, dtype=torch.int32, device="cuda")  # reuses freed memory, if any
    for rep in range(3):
        x8.copy_(torch.randn(8, V, generator=g).to(torch.bfloat16))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out8.cpu(), x8.cpu().argmax(-1)), f"replay {rep}"
    print(f"argmax workspace grown: {grown}")
    del junk


@pytest.mark.gpu
def test_argmax_one_workspace_serves_every_row_count(hiplib):
    """The wrapper's one workspace serves calls of 8, 128, 96, 8 and 256 rows in turn (the decode graph's
    buckets): the row counters live in a fixed region that no call's partials overlap."""
    from nanoserve_amd.kernels.sampling import argmax_rows
    g = cpu_gen(12)
    for R in (8, 128, 96, 8, 256, 32):
        x = torch.randn(R, 151936, generator=g).to(torch.bfloat16)
        assert torch.equal(argmax_rows(x.cuda()).cpu(), x.argmax(-1)), f"{R} rows"

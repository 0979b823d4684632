"""The binding INTEGRATION.md shows a nanoserve maintainer, executed as written (only the library path is
filled in): at BASELINE config 2's shape it must equal this package's wrapper bitwise and the oracle's
gather + SDPA within the bf16 gate, so the documented snippet cannot drift from the C ABI."""
import re
from pathlib import Path

import pytest
import torch

from nanoserve_amd import _lib
from oracle.ops import paged_attention_reference
from tests.conftest import cpu_gen

DOC = Path(__file__).resolve().parent.parent / "INTEGRATION.md"


def snippet() -> str:
    blocks = re.findall(r"```python\n(.*?)```", DOC.read_text(), flags=re.S)
    assert len(blocks) == 1, "INTEGRATION.md should hold exactly one python binding block"
    return blocks[0].replace("/path/to/libnanoserve_hip.so", str(_lib.LIB_PATH))


def test_snippet_declares_the_exported_signature():
    """CPU: the snippet's argtypes for ns_paged_attn_decode match the library's declaration."""
    ns: dict = {}
    exec(compile(snippet(), str(DOC), "exec"), ns)
    ours = _lib.SIGNATURES["ns_paged_attn_decode"][1]
    theirs = ns["_lib"].ns_paged_attn_decode.argtypes
    assert [t.__name__ for t in theirs] == [t.__name__ for t in ours]


@pytest.mark.gpu
def test_snippet_runs_at_config2(hiplib):
    from nanoserve_amd.kernels.paged_attention import paged_attention_decode
    ns: dict = {}
    exec(compile(snippet(), str(DOC), "exec"), ns)
    g = cpu_gen(2)
    B, nh, nkv, hd, NB, W = 32, 14, 2, 64, 65536, 256
    ctx = torch.randint(512, 4097, (B,), generator=g)
    perm = torch.randperm(NB, generator=g)
    tables = torch.zeros(B, W, dtype=torch.int32)
    used = 0
    for b in range(B):
        n = -(-int(ctx[b]) // 16)
        tables[b, :n] = perm[used:used + n].int()
        used += n
    k = torch.randn(NB, 16, nkv, hd, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(NB, 16, nkv, hd, generator=g).to(torch.bfloat16).cuda()
    q = torch.randn(B, nh, hd, generator=g).to(torch.bfloat16).cuda()
    dt, dl = tables.cuda(), ctx.int().cuda()
    doc_out = ns["paged_attention_decode"](q, k, v, dt, dl, 0.125)
    doc_again = ns["paged_attention_decode"](q, k, v, dt, dl, 0.125)
    ours = paged_attention_decode(q, k, v, dt, dl, 0.125)
    assert torch.equal(doc_out, ours) and torch.equal(doc_again, ours)
    ref = paged_attention_reference(q.float().cpu(), k.float().cpu(), v.float().cpu(), tables, ctx.int(), 0.125)
    assert (doc_out.float().cpu() - ref).abs().max().item() <= 1e-2

"""Greedy token selection on the GPU: row-wise argmax through the HIP kernel (csrc/sampling.hip), the
`logits.argmax(-1)` of nanoserve/engine.py:239 (first maximal index, NaN ranks highest)."""
from __future__ import annotations

import torch

from nanoserve_amd import _lib


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """logits [R, V] (last dim contiguous) -> int64 [R]."""
    assert logits.dim() == 2 and logits.stride(1) == 1
    _lib.require_gpu(logits)
    R, V = logits.shape
    if out is None:
        out = torch.empty(R, dtype=torch.int64, device=logits.device)
    assert out.dtype == torch.int64 and out.shape == (R,) and out.is_contiguous()
    _lib.check(_lib.lib().ns_argmax_rows(logits.data_ptr(), logits.stride(0), R, V, _lib.dtype_code(logits),
                                         out.data_ptr(), _lib.stream_of(logits)), "argmax_rows")
    return out

"""Greedy token selection on the GPU: row-wise argmax through the HIP kernel (csrc/sampling.hip), the
`logits.argmax(-1)` of nanoserve/engine.py:239 (first maximal index, NaN ranks highest)."""
from __future__ import annotations

import torch

from nanoserve_amd import _lib


_WS: dict[int, torch.Tensor] = {}
# Superseded workspaces stay alive: a captured graph keeps the address it was recorded with, and replays
# must not write counters into memory the caching allocator has handed to someone else.
_WS_RETIRED: list[torch.Tensor] = []
_WS_MIN_ROWS = 256      # the first buffer already covers every decode-graph bucket (at most 128 rows)


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A zero-filled workspace per device, grown (never shrunk) outside graph capture; the split kernel leaves
    its counters at zero, so one buffer serves every call. None when capture would need a larger one (the
    single-workgroup-per-row path needs none)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _WS.get(idx)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            return None
        floor = _lib.lib().ns_argmax_workspace_bytes(_WS_MIN_ROWS, 1 << 20)
        if ws is not None:
            _WS_RETIRED.append(ws)
        ws = torch.zeros(max(nbytes, floor, 1 << 16), dtype=torch.uint8, device=device)
        _WS[idx] = ws
    return ws


def argmax_workspace(device: torch.device) -> torch.Tensor | None:
    """The argmax workspace of `device` (at least the counter region the LM head with the argmax fused keeps
    its arrival counter and keys in); None inside a capture that would have to allocate it."""
    return _workspace(device, _lib.lib().ns_argmax_workspace_bytes(_WS_MIN_ROWS, 1 << 20))


def argmax_rows(logits: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """logits [R, V] (last dim contiguous) -> int64 [R]. `out` may be pinned host memory (the kernel writes
    it over the bus; read it after synchronising the stream)."""
    assert logits.dim() == 2 and logits.stride(1) == 1
    _lib.require_gpu(logits)
    R, V = logits.shape
    if out is None:
        out = torch.empty(R, dtype=torch.int64, device=logits.device)
    assert out.dtype == torch.int64 and out.shape == (R,) and out.is_contiguous()
    ws = _workspace(logits.device, _lib.lib().ns_argmax_workspace_bytes(R, V)) if R > 0 else None
    _lib.check(_lib.lib().ns_argmax_rows(logits.data_ptr(), logits.stride(0), R, V, _lib.dtype_code(logits),
                                         out.data_ptr(), _lib.ptr(ws), 0 if ws is None else ws.numel(),
                                         _lib.stream_of(logits)), "argmax_rows")
    return out

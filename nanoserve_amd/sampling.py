"""Token selection: greedy argmax, or temperature / top-k / top-p sampling by the Gumbel-max trick with a
per-request splitmix64 stream (semantics of nanoserve/sampling.py:26-90; draw n of request r uses a
generator seeded with mix_seed(seed_r, n), so results do not depend on batch composition). Greedy rows use
the HIP argmax kernel; the non-greedy rows' masking and Gumbel draw run as torch ops on the GPU (sampling
kernels are not part of the decode-loop hot path).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

_MASK64 = (1 << 64) - 1


@dataclass(frozen=True)
class SamplingParams:
    temperature: float = 0.0       # 0 = greedy
    top_p: float = 1.0             # 1 = off
    top_k: int = 0                 # 0 = off
    seed: int | None = None

    def __post_init__(self):
        if not self.temperature >= 0:
            raise ValueError(f"temperature must be >= 0, got {self.temperature}")
        if not 0 < self.top_p <= 1:
            raise ValueError(f"top_p must be in (0, 1], got {self.top_p}")
        if self.top_k < 0:
            raise ValueError(f"top_k must be >= 0, got {self.top_k}")

    @property
    def greedy(self) -> bool:
        return self.temperature == 0 or self.top_k == 1


def mix_seed(seed: int, step: int) -> int:
    """splitmix64 finaliser of (seed, step) (Steele, Lea & Flood 2014), 63 bits."""
    z = (seed * 0x9E3779B97F4A7C15 + step + 1) & _MASK64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _MASK64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _MASK64
    return (z ^ (z >> 31)) & ((1 << 63) - 1)


def sample(logits: torch.Tensor, params: list, seeds: list[int], steps: list[int]) -> list[int]:
    """logits [B, V] -> one token per row; row i uses params[i] (None = greedy) and stream (seeds[i], steps[i])."""
    from nanoserve_amd.kernels.sampling import argmax_rows
    greedy = [p is None or p.greedy for p in params]
    out = argmax_rows(logits)
    if all(greedy):
        return out.tolist()
    rows = [i for i, g in enumerate(greedy) if not g]
    x = logits[rows].float()
    R, V = x.shape
    dev = x.device
    x = x / torch.tensor([params[i].temperature for i in rows], device=dev)[:, None]
    ks = [params[i].top_k if params[i].top_k > 0 else V for i in rows]
    if min(ks) < V:
        kth = x.topk(max(ks), dim=-1).values.gather(1, torch.tensor([k - 1 for k in ks], device=dev)[:, None])
        x = x.masked_fill(x < kth, float("-inf"))
    ps = torch.tensor([params[i].top_p for i in rows], device=dev)
    if (ps < 1).any():
        sx, idx = x.sort(dim=-1, descending=True)
        probs = sx.softmax(-1)
        above = probs.cumsum(-1) - probs             # mass ranked strictly above each token
        sx = sx.masked_fill(above >= ps[:, None], float("-inf"))
        x = torch.full_like(x, float("-inf")).scatter(1, idx, sx)
    u = torch.empty(R, V, device=dev)
    for r, i in enumerate(rows):
        g = torch.Generator(device=dev)
        g.manual_seed(mix_seed(seeds[i], steps[i]))
        u[r].uniform_(generator=g)
    gumbel = -torch.log(-torch.log(u.clamp_(min=1e-20, max=1 - 1e-7)))
    out[rows] = (x + gumbel).argmax(-1)
    return out.tolist()

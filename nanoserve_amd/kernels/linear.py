"""Projection GEMMs of the decode loop: y = x @ W^T (+ b), x [M, K], W [N, K] row-major.

One indirection point for every projection of the model (QKV, O, gate/up, down, LM head;
nanoserve/model.py:231,256-257,362). Large-M (prefill) products go to the vendor GEMM through torch
(hipBLASLt on ROCm).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def linear(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor | None = None) -> torch.Tensor:
    return F.linear(x, w, b)

"""Unfused CPU restatements of the decode-loop ops (torch on the CPU, same op order as the reference).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """nanoserve/model.py:140-146 (HF order): fp32 statistics, cast back BEFORE the weight multiply."""
    dtype = x.dtype
    xf = x.to(torch.float32)
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * xf.to(dtype)


def rms_norm_residual(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor):
    """The fused kernel's contract (nanoserve/kernels/fused.py:45-59) in unfused ops: r = residual + x in the
    model dtype, then (rms_norm(r), r). Same as nanoserve/model.py:258-259."""
    r = residual + x
    return rms_norm(r, weight, eps), r


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """nanoserve/model.py:149-151."""
    h = x.shape[-1] // 2
    return torch.cat((-x[..., h:], x[..., :h]), dim=-1)


def inv_freq(head_dim: int, theta: float) -> torch.Tensor:
    """nanoserve/model.py:168: fp32 on the CPU, exactly like HF."""
    return 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))


def rope_tables(positions: torch.Tensor, head_dim: int, theta: float, dtype: torch.dtype):
    """nanoserve/model.py:212-217 without the leading batch dim: cos/sin [T, head_dim] in `dtype`."""
    freqs = positions[:, None].to(torch.float32) * inv_freq(head_dim, theta)
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """nanoserve/model.py:242-244: x [T, heads, hd], cos/sin [T, hd] broadcast over heads."""
    c, s = cos[:, None, :], sin[:, None, :]
    return x * c + rotate_half(x) * s


def silu_mul(x: torch.Tensor) -> torch.Tensor:
    """nanoserve/model.py:260 on the merged [gate | up] layout of nanoserve/kernels/fused.py:75-83."""
    n = x.shape[-1] // 2
    return F.silu(x[..., :n]) * x[..., n:]


def rope_qkv(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_heads: int, n_kv_heads: int,
             head_dim: int, k_cache=None, v_cache=None, slots=None):
    """Contract of nanoserve/kernels/fused.py:156-175 in unfused ops: split the merged projection
    (model.py:239-241 layout), rotate q and k (model.py:242-244), store k and v at `slots` with one indexed
    copy each (kv_cache.py:274-279)."""
    N = qkv.shape[0]
    q = qkv[:, :n_heads * head_dim].reshape(N, n_heads, head_dim)
    k = qkv[:, n_heads * head_dim:(n_heads + n_kv_heads) * head_dim].reshape(N, n_kv_heads, head_dim)
    v = qkv[:, (n_heads + n_kv_heads) * head_dim:].reshape(N, n_kv_heads, head_dim).clone()
    q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    if k_cache is not None:
        k_cache.view(-1, n_kv_heads, head_dim).index_copy_(0, slots, k)
        v_cache.view(-1, n_kv_heads, head_dim).index_copy_(0, slots, v)
    return q, k, v


def paged_attention_reference(q, k_pool, v_pool, block_tables, context_lens, scale):
    """nanoserve/kernels/paged_attention.py:108-121: gather each row's blocks, then SDPA with GQA."""
    outs = []
    block_size, n_kv_heads, head_dim = k_pool.shape[1:]
    lens = context_lens.tolist()
    for b in range(q.shape[0]):
        L = lens[b]
        nb = -(-L // block_size)
        blocks = block_tables[b, :nb].long()
        k = k_pool[blocks].reshape(-1, n_kv_heads, head_dim)[:L].transpose(0, 1)[None]
        v = v_pool[blocks].reshape(-1, n_kv_heads, head_dim)[:L].transpose(0, 1)[None]
        o = F.scaled_dot_product_attention(q[b][None, :, None, :], k, v, scale=scale, enable_gqa=True)
        outs.append(o[0, :, 0, :])
    return torch.stack(outs)


def paged_attention_fp64(q, k_pool, v_pool, block_tables, context_lens, scale) -> np.ndarray:
    """Independent check of the paged-decode contract: plain fp64 loops over tokens, explicit slot
    arithmetic (token t of row b at block table[b, t // bs], offset t % bs), max-subtracted softmax.
    Slow; for small shapes."""
    qn = q.double().numpy()
    kn, vn = k_pool.double().numpy(), v_pool.double().numpy()
    bt = block_tables.numpy()
    B, H, D = qn.shape
    bs, nkv = kn.shape[1], kn.shape[2]
    G = H // nkv
    out = np.zeros((B, H, D))
    for b in range(B):
        L = int(context_lens[b])
        ks = np.stack([kn[bt[b, t // bs], t % bs] for t in range(L)])   # [L, nkv, D]
        vs = np.stack([vn[bt[b, t // bs], t % bs] for t in range(L)])
        for h in range(H):
            g = h // G
            s = ks[:, g, :] @ qn[b, h] * scale
            p = np.exp(s - s.max())
            out[b, h] = (p[:, None] * vs[:, g, :]).sum(0) / p.sum()
    return out


def causal_offset_attention(q, k, v, ctx_len: int, scale: float):
    """Several new tokens on top of a cached context, nanoserve/model.py:292-309: query j (absolute
    position ctx_len + j) sees keys 0 .. ctx_len + j. q [T, H, D]; k, v [ctx_len + T, KVH, D]. The explicit
    mask + repeat_interleave + SDPA path of the reference; returns [T, H, D]."""
    T, H, D = q.shape
    L = k.shape[0]
    rep = H // k.shape[1]
    qs = q.transpose(0, 1)[None]
    ks = k.transpose(0, 1)[None].repeat_interleave(rep, dim=1)
    vs = v.transpose(0, 1)[None].repeat_interleave(rep, dim=1)
    if ctx_len == 0:
        o = F.scaled_dot_product_attention(qs, ks, vs, is_causal=T > 1, scale=scale)
    else:
        mask = torch.arange(L)[None, :] <= (ctx_len + torch.arange(T))[:, None]
        o = F.scaled_dot_product_attention(qs, ks, vs, attn_mask=mask, scale=scale)
    return o[0].transpose(0, 1)


def bf16_ulp_close(out: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    """(fraction bitwise identical, max |diff| / max(|ref|, tiny) in bf16 ulps) — the reference's `check`
    (tests/test_fused_ops.py:29-36) reports the first and bounds the second by 1 ulp."""
    same = (out == ref).float().mean().item()
    o, r = out.float(), ref.float()
    ulp = torch.where(r == 0, torch.full_like(r, 2.0 ** -133), r.abs() * 2.0 ** -7)
    return same, ((o - r).abs() / ulp).max().item() if o.numel() else 0.0


def kv_bytes_per_token(n_layers: int, n_kv_heads: int, head_dim: int, dtype_bytes: int) -> int:
    """nanoserve/model.py:54-56."""
    return n_layers * 2 * n_kv_heads * head_dim * dtype_bytes


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


__all__ = [n for n in dir() if not n.startswith("_") and n not in ("np", "torch", "F", "math", "annotations")]

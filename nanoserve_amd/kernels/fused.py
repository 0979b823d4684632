"""Fused token-wise ops on the GPU through the HIP kernels (csrc/fused.hip).

Same entry points, argument meaning and return values as nanoserve/kernels/fused.py:

    rms_norm(x, weight, eps, residual=None) -> out | (out, residual_out)      (fused.py:45-59)
    silu_mul(x) -> out                                                        (fused.py:75-83)
    rope_qkv(qkv, cos, sin, n_heads, n_kv_heads, head_dim,
             k_cache=None, v_cache=None, slots=None) -> (q, k, v)             (fused.py:156-175)

and the step's first ops in one launch (F.embedding + Qwen2Model.rope, nanoserve/model.py:341,212-217):

    embed_rope(token_ids, positions, embed, inv_freq, head_dim, row_stats=False) -> (x, cos, sin, sumsq)

Each kernel rounds to the model dtype where PyTorch's unfused ops round, so bf16 results equal the
unfused ops bit for bit except for RMSNorm's fp32 summation order (then at most 1 bf16 ulp apart).
Outputs are allocated here with torch (inside a graph capture they come from the graph's pool).
"""
from __future__ import annotations

import torch

from nanoserve_amd import _lib


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, residual: torch.Tensor | None = None):
    """RMSNorm over the last dim in one kernel. With `residual`: r = residual + x first (rounded to the
    dtype), returns (rms_norm(r), r)."""
    N = x.shape[-1]
    x2 = x.reshape(-1, N)
    assert x2.is_contiguous() and weight.is_contiguous() and weight.shape == (N,) and weight.dtype == x.dtype
    _lib.require_gpu(x, weight, residual)
    out = torch.empty_like(x2)
    res = None
    res_out = None
    if residual is not None:
        res = residual.reshape(-1, N)
        assert res.is_contiguous() and res.dtype == x.dtype and res.shape == x2.shape
        res_out = torch.empty_like(x2)
    _lib.check(_lib.lib().ns_rms_norm(x2.data_ptr(), _lib.ptr(res), weight.data_ptr(), out.data_ptr(),
                                      _lib.ptr(res_out), x2.shape[0], N, float(eps), _lib.dtype_code(x),
                                      _lib.stream_of(x)), "rms_norm")
    if residual is None:
        return out.view(x.shape)
    return out.view(x.shape), res_out.view(x.shape)


def silu_mul(x: torch.Tensor) -> torch.Tensor:
    """x = [..., 2N] holding [gate | up] (the merged gate/up projection) -> silu(gate) * up, [..., N]."""
    N = x.shape[-1] // 2
    x2 = x.reshape(-1, 2 * N)
    assert x2.is_contiguous() and x.shape[-1] == 2 * N
    _lib.require_gpu(x)
    out = torch.empty(x2.shape[0], N, device=x.device, dtype=x.dtype)
    _lib.check(_lib.lib().ns_silu_mul(x2.data_ptr(), out.data_ptr(), x2.shape[0], N, _lib.dtype_code(x),
                                      _lib.stream_of(x)), "silu_mul")
    return out.view(*x.shape[:-1], N)


def rope_qkv(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_heads: int, n_kv_heads: int,
             head_dim: int, k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
             slots: torch.Tensor | None = None):
    """qkv: [N, (n_heads + 2*n_kv_heads) * head_dim], the merged Q/K/V projection output (bias included).
    cos/sin: [N, head_dim]. Returns rotated q [N, n_heads, hd], rotated k and plain v [N, n_kv_heads, hd]; with
    a paged cache layer (k_cache/v_cache [blocks, block_size, n_kv_heads, hd]) and int64 slots [N], also stores
    k and v at those slots."""
    N = qkv.shape[0]
    assert qkv.is_contiguous() and cos.is_contiguous() and sin.is_contiguous()
    assert qkv.dtype in (torch.bfloat16, torch.float32), "rounding is emulated for bf16 / exact for fp32"
    assert qkv.shape[1] == (n_heads + 2 * n_kv_heads) * head_dim
    assert cos.shape == (N, head_dim) and sin.shape == (N, head_dim)
    assert cos.dtype == sin.dtype == qkv.dtype
    write = k_cache is not None
    if write:
        assert v_cache is not None and slots is not None
        assert k_cache.is_contiguous() and v_cache.is_contiguous() and k_cache.shape == v_cache.shape
        assert k_cache.shape[-2:] == (n_kv_heads, head_dim) and k_cache.dtype == qkv.dtype
        assert slots.dtype == torch.int64 and slots.shape == (N,) and slots.is_contiguous()
    _lib.require_gpu(qkv, cos, sin, k_cache, v_cache, slots)
    q = torch.empty(N, n_heads, head_dim, device=qkv.device, dtype=qkv.dtype)
    k = torch.empty(N, n_kv_heads, head_dim, device=qkv.device, dtype=qkv.dtype)
    v = torch.empty_like(k)
    _lib.check(_lib.lib().ns_rope_qkv(
        qkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(),
        _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(slots) if write else None,
        N, n_heads, n_kv_heads, head_dim, _lib.dtype_code(qkv), _lib.stream_of(qkv)), "rope_qkv")
    return q, k, v


def embed_rope(token_ids: torch.Tensor, positions: torch.Tensor, embed: torch.Tensor, inv_freq: torch.Tensor,
               head_dim: int, row_stats: bool = False):
    """x = embed[token_ids] [N, H]; cos/sin [N, head_dim] (cat(f, f).cos()/.sin() in the embedding dtype,
    f = positions.float() * inv_freq); with row_stats (N <= NORM_ROWS) also the first RMSNorm's row statistics
    sumsq (fp32 [ceil(H / 16), NORM_ROWS]) for a NormedRows, else None."""
    N = token_ids.shape[0]
    V, H = embed.shape
    assert token_ids.dtype == torch.int64 and positions.dtype == torch.int64 and positions.shape == (N,)
    assert token_ids.is_contiguous() and positions.is_contiguous() and embed.is_contiguous()
    assert inv_freq.dtype == torch.float32 and inv_freq.shape == (head_dim // 2,) and inv_freq.is_contiguous()
    _lib.require_gpu(token_ids, positions, embed, inv_freq)
    dev, dt = embed.device, embed.dtype
    x = torch.empty(N, H, device=dev, dtype=dt)
    cos = torch.empty(N, head_dim, device=dev, dtype=dt)
    sin = torch.empty(N, head_dim, device=dev, dtype=dt)
    from nanoserve_amd.kernels.linear import NORM_ROWS
    sumsq = torch.empty(-(-H // 16), NORM_ROWS, device=dev, dtype=torch.float32) if row_stats else None
    _lib.check(_lib.lib().ns_embed_rope(token_ids.data_ptr(), positions.data_ptr(), N, embed.data_ptr(), V, H,
                                        inv_freq.data_ptr(), head_dim, x.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                        _lib.ptr(sumsq), _lib.dtype_code(embed), _lib.stream_of(embed)), "embed_rope")
    return x, cos, sin, sumsq


def gather_rows(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """x[idx] for a 2-D x with contiguous rows (row bytes a multiple of 16) and int64 indices on its device, by
    the HIP row gather (the LM head's row selection, nanoserve/model.py:353-356); other shapes index with torch."""
    assert x.dim() == 2 and idx.dim() == 1
    row_bytes = x.shape[1] * x.element_size()
    if (x.stride(1) != 1 or row_bytes % 16 or (x.stride(0) * x.element_size()) % 16 or x.data_ptr() % 16
            or idx.dtype != torch.int64 or idx.device != x.device or not idx.is_contiguous()):
        return x[idx]
    _lib.require_gpu(x, idx)
    out = torch.empty(idx.shape[0], x.shape[1], device=x.device, dtype=x.dtype)
    _lib.check(_lib.lib().ns_gather_rows(x.data_ptr(), x.stride(0) * x.element_size(), x.shape[0], idx.data_ptr(),
                                         idx.shape[0], row_bytes, out.data_ptr(), row_bytes, _lib.stream_of(x)),
               "gather_rows")
    return out

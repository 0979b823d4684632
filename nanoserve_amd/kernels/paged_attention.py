"""Paged attention on the GPU through the HIP kernels: decode (csrc/paged_attention.hip) and chunked
prefill (csrc/prefill_attention.hip).

Same entry point and argument meaning as nanoserve/kernels/paged_attention.py:85-105:

    paged_attention_decode(q, k_pool, v_pool, block_tables, context_lens, scale) -> out

q: [B, n_heads, head_dim] (last dim contiguous); k_pool / v_pool: ONE layer's pool
[num_blocks, block_size, n_kv_heads, head_dim] with identical strides; block_tables: int32 [B, max_blocks]
(padding entries never read); context_lens: int32 [B], including the new token whose K/V must already be
written. Returns out = torch.empty_like(q) filled with the attention output.

The bf16 kernel splits long contexts across workgroups; the last partition of a row to finish merges the
partial softmax states (one launch). That needs a small device workspace; one per (device, B, n_kv_heads,
head_dim, max_blocks) is allocated zero-filled on first use (outside any graph capture: the graph runners warm
up eagerly first) and reused by every later call and graph replay. Calls on one stream never overlap, so
sharing it is safe.

    paged_attention_prefill(q, k_pool, v_pool, block_tables, seq_info, max_new, max_kv, scale, out=None)

The new tokens of several sequences at once (nanoserve/model.py:283-318, the per-sequence SDPA branch):
q [N, n_heads, head_dim] holds the step's tokens; seq_info int32 [S, 4] (device) holds per sequence
(q_start, n_new, ctx_len, 0); block_tables int32 [S, W]; max_new / max_kv = the largest n_new and
ctx_len + n_new (host ints: they size the grid). Token j of sequence s attends to keys 0 .. ctx_len + j of
its pages, which must already hold the new tokens' K/V. Rows of `out` outside every sequence are left
untouched. bf16 only; `prefill_seq_info` builds seq_info from host lists. Long tiles are split over
several workgroups whose partial states meet in a zero-filled workspace, kept per (device, shape) like
the decode one (the prefill path runs eagerly, so it is never first allocated inside a capture).
"""
from __future__ import annotations

import torch

from nanoserve_amd import _lib

_WORKSPACES: dict[tuple, torch.Tensor] = {}


def decode_workspace(device: torch.device, B: int, n_kv_heads: int, head_dim: int, max_blocks: int,
                     dtype: torch.dtype) -> torch.Tensor | None:
    """The split-K workspace for this launch shape, or None if the launch needs none."""
    nbytes = _lib.lib().ns_decode_workspace_bytes(B, n_kv_heads, head_dim, max_blocks, _lib.dtype_code_of(dtype))
    if nbytes == 0:
        return None
    key = (device.index if device.index is not None else torch.cuda.current_device(), B, n_kv_heads, head_dim,
           max_blocks, dtype)
    ws = _WORKSPACES.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("paged_attention_decode: first call for this shape happened inside a graph capture; "
                               "run one eager call (warm-up) before capturing")
        # zero-filled once: the kernel's per-row arrival counters start at zero and every call leaves them there
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def paged_attention_decode(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                           block_tables: torch.Tensor, context_lens: torch.Tensor, scale: float,
                           products: str = "mfma", pairs: torch.Tensor | None = None) -> torch.Tensor:
    """products="valu" runs the same kernel with the QK^T and P.V products on the vector ALUs
    (ns_paged_attn_decode_valu: bf16 whole-row shapes only), for measuring the matrix-core design choice.
    pairs (int32 [B], device; see pair_rows) lets rows that share a block table run together
    (ns_paged_attn_decode_pairs): the same result, each page read once per pair."""
    if products not in ("mfma", "valu"):
        raise ValueError(f"products must be 'mfma' or 'valu', got {products!r}")
    B, n_heads, head_dim = q.shape
    num_blocks, block_size, n_kv_heads, hd2 = k_pool.shape
    assert hd2 == head_dim and q.dtype == k_pool.dtype == v_pool.dtype
    assert q.stride(-1) == 1 and k_pool.stride(-1) == 1 and v_pool.stride() == k_pool.stride()
    assert v_pool.shape == k_pool.shape
    assert block_tables.dtype == torch.int32 and block_tables.dim() == 2 and block_tables.shape[0] == B
    assert block_tables.stride(1) == 1 or block_tables.shape[1] == 1
    assert context_lens.dtype == torch.int32 and context_lens.shape == (B,) and context_lens.is_contiguous()
    _lib.require_gpu(q, k_pool, v_pool, block_tables, context_lens)
    out = torch.empty_like(q)
    if B == 0:
        return out
    max_blocks = block_tables.shape[1]
    ws = decode_workspace(q.device, B, n_kv_heads, head_dim, max_blocks, q.dtype)
    L = _lib.lib()
    if pairs is not None and products == "mfma":
        assert pairs.dtype == torch.int32 and pairs.shape == (B,) and pairs.is_contiguous()
        fn, extra = L.ns_paged_attn_decode_pairs, (pairs.data_ptr(),)
    else:
        fn, extra = (L.ns_paged_attn_decode if products == "mfma" else L.ns_paged_attn_decode_valu), ()
    _lib.check(fn(
        q.data_ptr(), q.stride(0), q.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(), *extra,
        out.data_ptr(), out.stride(0), out.stride(1),
        B, n_heads, n_kv_heads, head_dim, block_size, max_blocks, num_blocks, float(scale), _lib.dtype_code(q),
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _lib.stream_of(q)),
        "paged_attention_decode")
    return out


def paged_attention_decode_rows(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                                block_tables: torch.Tensor, context_lens: torch.Tensor, rows: torch.Tensor,
                                scale: float, out: torch.Tensor) -> torch.Tensor:
    """paged_attention_decode for entries whose query rows sit at `rows` (int64 [B], device) of q [N, nh, hd];
    each entry's output goes to the same row of `out` [N, nh, hd] (other rows untouched). Replaces the gather
    q[0][decode_meta.token_idx] and the index_copy_ of nanoserve/model.py:277-281."""
    N, n_heads, head_dim = q.shape
    B = rows.shape[0]
    num_blocks, block_size, n_kv_heads, hd2 = k_pool.shape
    assert hd2 == head_dim and q.dtype == k_pool.dtype == v_pool.dtype == out.dtype and out.shape == q.shape
    assert q.stride(-1) == 1 and out.stride(-1) == 1 and k_pool.stride(-1) == 1 and v_pool.stride() == k_pool.stride()
    assert v_pool.shape == k_pool.shape and rows.dtype == torch.int64 and rows.is_contiguous()
    assert block_tables.dtype == torch.int32 and block_tables.dim() == 2 and block_tables.shape[0] == B
    assert block_tables.stride(1) == 1 or block_tables.shape[1] == 1
    assert context_lens.dtype == torch.int32 and context_lens.shape == (B,) and context_lens.is_contiguous()
    _lib.require_gpu(q, k_pool, v_pool, block_tables, context_lens, rows, out)
    if B == 0:
        return out
    max_blocks = block_tables.shape[1]
    ws = decode_workspace(q.device, B, n_kv_heads, head_dim, max_blocks, q.dtype)
    _lib.check(_lib.lib().ns_paged_attn_decode_rows(
        q.data_ptr(), q.stride(0), q.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        block_tables.data_ptr(), block_tables.stride(0), context_lens.data_ptr(), rows.data_ptr(),
        out.data_ptr(), out.stride(0), out.stride(1),
        B, n_heads, n_kv_heads, head_dim, block_size, max_blocks, num_blocks, float(scale), _lib.dtype_code(q),
        None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _lib.stream_of(q)),
        "paged_attention_decode_rows")
    return out


def paged_attention_mixed(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, pf_tables: torch.Tensor,
                          seq_info: torch.Tensor, max_new: int, max_kv: int, dec_tables: torch.Tensor,
                          context_lens: torch.Tensor, rows: torch.Tensor, scale: float, out: torch.Tensor) -> torch.Tensor:
    """A mixed step's attention in one launch: paged_attention_prefill(q, ..., pf_tables, seq_info, max_new, max_kv,
    out=out) for the chunks' rows and paged_attention_decode_rows(q, ..., dec_tables, context_lens, rows, out=out)
    for the decode rows (model.py:277-318), their workgroups in one grid so the decode rows run beside the
    prefill instead of after it. bf16; the same arguments, workspaces and results as the two calls."""
    N, n_heads, head_dim = q.shape
    num_blocks, block_size, n_kv_heads, hd2 = k_pool.shape
    assert hd2 == head_dim and q.dtype == k_pool.dtype == v_pool.dtype == out.dtype == torch.bfloat16
    assert out.shape == q.shape and q.stride(-1) == 1 and out.stride(-1) == 1 and k_pool.stride(-1) == 1
    assert v_pool.shape == k_pool.shape and v_pool.stride() == k_pool.stride()
    S, B = seq_info.shape[0], rows.shape[0]
    assert seq_info.dtype == torch.int32 and seq_info.shape == (S, 4) and seq_info.is_contiguous()
    assert pf_tables.dtype == torch.int32 and pf_tables.dim() == 2 and pf_tables.shape[0] == S
    assert pf_tables.stride(1) == 1 or pf_tables.shape[1] == 1
    assert rows.dtype == torch.int64 and rows.is_contiguous()
    assert dec_tables.dtype == torch.int32 and dec_tables.dim() == 2 and dec_tables.shape[0] == B
    assert dec_tables.stride(1) == 1 or dec_tables.shape[1] == 1
    assert context_lens.dtype == torch.int32 and context_lens.shape == (B,) and context_lens.is_contiguous()
    _lib.require_gpu(q, k_pool, v_pool, pf_tables, seq_info, dec_tables, context_lens, rows, out)
    L = _lib.lib()
    pws = prefill_workspace(q.device, L.ns_prefill_workspace_bytes(S, n_heads, head_dim, int(max_new), int(max_kv))) \
        if S > 0 and max_new > 0 else None
    dws = decode_workspace(q.device, B, n_kv_heads, head_dim, dec_tables.shape[1], q.dtype) if B > 0 else None
    _lib.check(L.ns_paged_attn_mixed(
        q.data_ptr(), q.stride(0), q.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        pf_tables.data_ptr(), pf_tables.stride(0), seq_info.data_ptr(), S, int(max_new), int(max_kv),
        pf_tables.shape[1], None if pws is None else pws.data_ptr(), 0 if pws is None else pws.numel(),
        dec_tables.data_ptr(), dec_tables.stride(0), context_lens.data_ptr(), rows.data_ptr(), B, dec_tables.shape[1],
        None if dws is None else dws.data_ptr(), 0 if dws is None else dws.numel(),
        out.data_ptr(), out.stride(0), out.stride(1),
        n_heads, n_kv_heads, head_dim, block_size, num_blocks, float(scale), _lib.dtype_code(q), _lib.stream_of(q)),
        "paged_attention_mixed")
    return out


def prefill_seq_info(q_starts: list[int], n_new: list[int], ctx_lens: list[int], device) -> torch.Tensor:
    """int32 [S, 4] (q_start, n_new, ctx_len, 0) on `device`, from host lists."""
    rows = [[a, b, c, 0] for a, b, c in zip(q_starts, n_new, ctx_lens)]
    return torch.tensor(rows, dtype=torch.int32).reshape(-1, 4).to(device)


_PREFILL_WS: dict[int, torch.Tensor] = {}
_PREFILL_WS_RETIRED: list[torch.Tensor] = []   # superseded buffers stay alive: captured graphs may point at them


def prefill_workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    """A zero-filled workspace of at least nbytes on `device` (grown, never shrunk), or None for 0 bytes."""
    if nbytes == 0:
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _PREFILL_WS.get(idx)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("paged_attention_prefill: workspace must be sized by an eager call before capture")
        if ws is not None:
            _PREFILL_WS_RETIRED.append(ws)
        # zero-filled: the kernel's arrival counters start at zero and every call leaves them there
        ws = torch.zeros(nbytes, dtype=torch.uint8, device=device)
        _PREFILL_WS[idx] = ws
    return ws


def paged_attention_prefill(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, block_tables: torch.Tensor,
                            seq_info: torch.Tensor, max_new: int, max_kv: int, scale: float,
                            out: torch.Tensor | None = None) -> torch.Tensor:
    N, n_heads, head_dim = q.shape
    num_blocks, block_size, n_kv_heads, hd2 = k_pool.shape
    assert hd2 == head_dim and q.dtype == k_pool.dtype == v_pool.dtype
    assert q.stride(-1) == 1 and k_pool.stride(-1) == 1 and v_pool.stride() == k_pool.stride()
    assert v_pool.shape == k_pool.shape
    S = seq_info.shape[0]
    assert seq_info.dtype == torch.int32 and seq_info.shape == (S, 4) and seq_info.is_contiguous()
    assert block_tables.dtype == torch.int32 and block_tables.dim() == 2 and block_tables.shape[0] == S
    assert block_tables.stride(1) == 1 or block_tables.shape[1] == 1
    if out is None:
        out = torch.empty_like(q)
    assert out.shape == q.shape and out.dtype == q.dtype and out.stride(-1) == 1
    _lib.require_gpu(q, k_pool, v_pool, block_tables, seq_info, out)
    if S == 0 or max_new == 0:
        return out
    L = _lib.lib()
    ws = None
    if head_dim in (64, 128):
        ws = prefill_workspace(q.device, L.ns_prefill_workspace_bytes(S, n_heads, head_dim, int(max_new), int(max_kv)))
    _lib.check(L.ns_paged_attn_prefill(
        q.data_ptr(), q.stride(0), q.stride(1),
        k_pool.data_ptr(), v_pool.data_ptr(), k_pool.stride(0), k_pool.stride(1), k_pool.stride(2),
        block_tables.data_ptr(), block_tables.stride(0), seq_info.data_ptr(), S, int(max_new), int(max_kv),
        out.data_ptr(), out.stride(0), out.stride(1),
        n_heads, n_kv_heads, head_dim, block_size, block_tables.shape[1], num_blocks, float(scale),
        _lib.dtype_code(q), None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(),
        _lib.stream_of(q)), "paged_attention_prefill")
    return out


def pair_rows(tables: list, out) -> None:
    """Fill `out` (int32 array-like, len >= len(tables)) with the row pairing of ns_paged_attn_decode_pairs:
    consecutive rows whose block tables are the same list (or equal) are paired left to right (1 for the
    first of a pair, -1 for the second), every other row 0."""
    n, i = len(tables), 0
    while i < n:
        if i + 1 < n and (tables[i + 1] is tables[i] or tables[i + 1] == tables[i]):
            out[i], out[i + 1] = 1, -1
            i += 2
        else:
            out[i] = 0
            i += 1

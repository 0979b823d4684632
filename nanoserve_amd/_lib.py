"""Loader for libnanoserve_hip.so (the gfx950 kernels) and the glue every wrapper shares.

The library is a plain C ABI (include/nanoserve_hip.h) opened with ctypes. torch is imported first so
the process already holds torch's HIP runtime; the library's `libamdhip64.so.7` dependency then binds to
that same runtime, and stream handles and device pointers from torch are valid inside it.

There is no fallback: when the library is missing or cannot be opened, or a tensor is not on a GPU,
the call raises. A nonzero status from a kernel entry point raises RuntimeError with the library's own
message (the engine's step-failure handling expects RuntimeError, as in nanoserve/async_engine.py:119-127).
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_NAME = "libnanoserve_hip.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1}

_c_int, _c_i64, _c_f32, _c_vp, _c_sz = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# Argument types of every exported entry point (must match include/nanoserve_hip.h).
SIGNATURES: dict[str, tuple[object, list]] = {
    "ns_last_error": (ctypes.c_char_p, []),
    "ns_version": (ctypes.c_char_p, []),
    "ns_paged_attn_decode": (_c_int, [
        _c_vp, _c_i64, _c_i64,                  # q, q_sb, q_sh
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,   # k_pool, v_pool, kv_sblk, kv_spos, kv_sh
        _c_vp, _c_i64, _c_vp,                   # block_tables, bt_sb, context_lens
        _c_vp, _c_i64, _c_i64,                  # out, o_sb, o_sh
        _c_int, _c_int, _c_int, _c_int, _c_int,  # B, n_heads, n_kv_heads, head_dim, block_size
        _c_int, _c_int, _c_f32, _c_int,         # max_blocks, num_blocks, scale, dtype
        _c_vp, _c_sz, _c_vp]),                  # workspace, workspace_bytes, stream
    "ns_paged_attn_decode_pairs": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_vp, _c_i64,
        _c_i64, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_f32, _c_int, _c_vp, _c_sz, _c_vp]),
    "ns_paged_attn_decode_valu": (_c_int, [
        _c_vp, _c_i64, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp, _c_vp, _c_i64, _c_i64,
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_f32, _c_int, _c_vp, _c_sz, _c_vp]),
    "ns_paged_attn_decode_rows": (_c_int, [
        _c_vp, _c_i64, _c_i64,                  # q, q_sb, q_sh
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,   # k_pool, v_pool, kv_sblk, kv_spos, kv_sh
        _c_vp, _c_i64, _c_vp, _c_vp,            # block_tables, bt_sb, context_lens, q_rows
        _c_vp, _c_i64, _c_i64,                  # out, o_sb, o_sh
        _c_int, _c_int, _c_int, _c_int, _c_int,  # B, n_heads, n_kv_heads, head_dim, block_size
        _c_int, _c_int, _c_f32, _c_int,         # max_blocks, num_blocks, scale, dtype
        _c_vp, _c_sz, _c_vp]),                  # workspace, workspace_bytes, stream
    "ns_decode_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "ns_paged_attn_decode_noalloc": (_c_int, [
        _c_vp, _c_i64, _c_i64,                  # q, q_sb, q_sh
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,   # k_pool, v_pool, kv_sblk, kv_spos, kv_sh
        _c_vp, _c_i64, _c_vp,                   # block_tables, bt_sb, context_lens
        _c_vp, _c_i64, _c_i64,                  # out, o_sb, o_sh
        _c_int, _c_int, _c_int, _c_int, _c_int,  # B, n_heads, n_kv_heads, head_dim, block_size
        _c_int, _c_int, _c_f32, _c_int,         # max_blocks, num_blocks, scale, dtype
        _c_vp]),                                # stream
    "ns_paged_attn_prefill": (_c_int, [
        _c_vp, _c_i64, _c_i64,                  # q, q_st, q_sh
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,   # k_pool, v_pool, kv_sblk, kv_spos, kv_sh
        _c_vp, _c_i64, _c_vp, _c_int, _c_int, _c_int,   # block_tables, bt_sb, seq_info, n_seqs, max_new, max_kv
        _c_vp, _c_i64, _c_i64,                  # out, o_st, o_sh
        _c_int, _c_int, _c_int, _c_int,         # n_heads, n_kv_heads, head_dim, block_size
        _c_int, _c_int, _c_f32, _c_int,         # max_blocks, num_blocks, scale, dtype
        _c_vp, _c_sz, _c_vp]),                  # workspace, workspace_bytes, stream
    "ns_prefill_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "ns_paged_attn_mixed": (_c_int, [
        _c_vp, _c_i64, _c_i64,                  # q, q_sb, q_sh
        _c_vp, _c_vp, _c_i64, _c_i64, _c_i64,   # k_pool, v_pool, kv_sblk, kv_spos, kv_sh
        _c_vp, _c_i64, _c_vp, _c_int, _c_int, _c_int,   # pf_block_tables, pf_bt_sb, seq_info, n_seqs, max_new, max_kv
        _c_int, _c_vp, _c_sz,                   # pf_max_blocks, pf_workspace, pf_workspace_bytes
        _c_vp, _c_i64, _c_vp, _c_vp, _c_int, _c_int,   # dec_block_tables, dec_bt_sb, context_lens, q_rows, B, dec_max_blocks
        _c_vp, _c_sz,                           # dec_workspace, dec_workspace_bytes
        _c_vp, _c_i64, _c_i64,                  # out, o_sb, o_sh
        _c_int, _c_int, _c_int, _c_int, _c_int, _c_f32, _c_int,   # n_heads n_kv head_dim block_size num_blocks scale dtype
        _c_vp]),                                # stream
    "ns_rms_norm": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_int, _c_f32, _c_int, _c_vp]),
    "ns_silu_mul": (_c_int, [_c_vp, _c_vp, _c_i64, _c_int, _c_int, _c_vp]),
    "ns_rope_qkv": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                             _c_i64, _c_int, _c_int, _c_int, _c_int, _c_vp]),
    "ns_argmax_workspace_bytes": (_c_sz, [_c_i64, _c_int]),
    "ns_argmax_rows": (_c_int, [_c_vp, _c_i64, _c_i64, _c_int, _c_int, _c_vp, _c_vp, _c_sz, _c_vp]),
    "ns_embed_rope": (_c_int, [_c_vp, _c_vp, _c_i64, _c_vp, _c_i64, _c_int, _c_vp, _c_int,   # ids pos n embed V H inv hd
                               _c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_vp]),                 # x cos sin sumsq dtype stream
    "ns_gemm_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int]),
    "ns_gemm": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,   # x w bias y M N K dtype
                         _c_vp, _c_vp, _c_f32,                                      # x_sumsq x_norm_w x_eps
                         _c_vp, _c_sz, _c_vp]),                                     # ws ws_bytes stream
    "ns_gemm_argmax_fused": (_c_int, [_c_int, _c_int, _c_int]),
    "ns_gemm_argmax": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,   # x w y M N K dtype
                                _c_vp, _c_vp, _c_f32, _c_vp,                       # x_sumsq x_norm_w x_eps tokens
                                _c_vp, _c_sz, _c_vp]),                             # argmax ws, bytes, stream
    "ns_gemm_silu_mul": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
                                  _c_vp, _c_vp, _c_f32, _c_vp, _c_sz, _c_vp]),
    "ns_gemm_residual_norm_stats": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp,      # x w residual res_out sumsq
                                             _c_int, _c_int, _c_int, _c_int, _c_vp, _c_sz, _c_vp]),
    "ns_rms_norm_apply": (_c_int, [_c_vp, _c_vp, _c_vp, _c_f32, _c_vp, _c_i64, _c_int, _c_int, _c_vp]),
    "ns_gather_rows": (_c_int, [_c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_i64, _c_vp, _c_i64, _c_vp]),
    "ns_gemm_rope_qkv_fits": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "ns_gemm_rope_qkv": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                  _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                  _c_vp, _c_vp, _c_f32, _c_vp, _c_sz, _c_vp]),
    # fragment-packed weights (decode-sized products)
    "ns_packed_weight_bytes": (_c_sz, [_c_int, _c_int, _c_int, _c_int]),             # N K order head_dim
    "ns_pack_weight": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_vp]),   # w packed N K order hd stream
    "ns_gemm_packed_workspace_bytes": (_c_sz, [_c_int, _c_int, _c_int, _c_int, _c_int]),   # M N K order hd
    "ns_gemm_packed_sliced": (_c_int, [_c_int, _c_int, _c_int, _c_int, _c_int]),
    "ns_gemm_packed": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,   # x wp bias y M N K dtype
                                _c_vp, _c_vp, _c_f32, _c_vp, _c_sz, _c_vp]),
    "ns_gemm_argmax_packed_fits": (_c_int, [_c_int, _c_int, _c_int]),
    "ns_gemm_argmax_packed": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,   # x wp y M N K dtype
                                       _c_vp, _c_vp, _c_f32, _c_vp, _c_vp, _c_sz, _c_vp]),
    "ns_gemm_silu_mul_packed": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
                                         _c_vp, _c_vp, _c_f32, _c_vp, _c_sz, _c_vp]),
    "ns_gemm_residual_norm_stats_packed": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                                    _c_int, _c_int, _c_int, _c_int, _c_vp, _c_sz, _c_vp]),
    "ns_gemm_rope_qkv_packed": (_c_int, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                         _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                         _c_vp, _c_vp, _c_f32, _c_vp, _c_sz, _c_vp]),
}

_lib: ctypes.CDLL | None = None


def load_library(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Open the library once (no GPU needed just to open it) and declare every signature."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')")
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load_library()


def check(status: int, what: str) -> None:
    if status != 0:
        msg = lib().ns_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def dtype_code_of(dtype: torch.dtype) -> int:
    code = DTYPE_CODES.get(dtype)
    if code is None:
        raise ValueError(f"dtype {dtype} not supported by the HIP kernels (float32, bfloat16)")
    return code


def dtype_code(t: torch.Tensor) -> int:
    return dtype_code_of(t.dtype)


def require_gpu(*tensors: torch.Tensor) -> None:
    for t in tensors:
        if t is not None and t.device.type != "cuda":
            raise ValueError(f"the HIP kernels run on the GPU; got a tensor on {t.device}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream

"""The C-ABI library loads without a GPU and exports every entry point include/nanoserve_hip.h declares;
argument validation (pure host code) rejects unsupported launches with a message, before any GPU work."""
import ctypes
import re
from pathlib import Path

import pytest

from nanoserve_amd import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "nanoserve_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(ns_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load_library()
    names = declared_functions()
    assert len(names) >= 7
    for n in names:
        assert hasattr(lib, n), f"{n} declared in the header but not exported"
        assert n in _lib.SIGNATURES, f"{n} has no ctypes signature"


def test_version_and_error_slot():
    lib = _lib.load_library()
    assert lib.ns_version().startswith(b"nanoserve_hip")
    assert isinstance(lib.ns_last_error(), bytes)


def test_workspace_sizing():
    lib = _lib.load_library()
    # one partition covers 16 pages (hd 64) / 8 pages (hd 128): short tables need no workspace
    assert lib.ns_decode_workspace_bytes(32, 2, 64, 16, 1) == 0
    assert lib.ns_decode_workspace_bytes(32, 2, 128, 8, 1) == 0
    assert lib.ns_decode_workspace_bytes(32, 2, 64, 256, 0) == 0          # fp32 path never splits
    n = lib.ns_decode_workspace_bytes(32, 2, 64, 256, 1)
    slots = 32 * 2 * 16
    assert n >= slots * 16 * (64 + 2) * 4


def test_gemm_routes_on_the_host():
    """Host-only queries of the GEMM entry points (no GPU call): which merged-QKV shapes the fused RoPE
    epilogue takes, and which plans need a K-slice workspace."""
    lib = _lib.load_library()
    fits = lib.ns_gemm_rope_qkv_fits
    for M in (1, 64, 65, 192, 193, 1552, 8192):   # a plain input: any M (skinny, tile-16, tiled epilogue)
        assert fits(M, 1536, 12, 2, 128, 0) == 1 and fits(M, 896, 14, 2, 64, 0) == 1
    assert fits(128, 1536, 12, 2, 128, 1) == 1 and fits(129, 1536, 12, 2, 128, 1) == 0   # normalised: <= 128
    assert fits(1552, 1536, 12, 2, 96, 0) == 0 and fits(1552, 1000, 12, 2, 128, 0) == 0  # head_dim, K % 32
    # K = 1536 products never split K; the 1552-row down projection (K = 8960) runs K slices
    assert lib.ns_gemm_workspace_bytes(1552, 1536, 1536) == 0
    assert lib.ns_gemm_workspace_bytes(1552, 2048, 1536) == 0
    assert lib.ns_gemm_workspace_bytes(1552, 1536, 8960) > 0


def test_invalid_arguments_are_rejected_on_the_host():
    lib = _lib.load_library()
    args = [None, 0, 0, None, None, 0, 0, 0, None, 0, None, None, 0, 0,
            4, 12, 2, 96, 16, 8, 100, 0.1, 1, None, 0, None]   # head_dim 96: unsupported
    st = lib.ns_paged_attn_decode(*args)
    assert st == 1 and b"head_dim" in lib.ns_last_error()
    args[17], args[18] = 128, 8                                  # block size 8: unsupported
    assert lib.ns_paged_attn_decode(*args) == 1 and b"block_size" in lib.ns_last_error()
    assert lib.ns_rms_norm(None, None, None, None, None, 4, 100000, 1e-6, 1, None) == 1
    assert lib.ns_silu_mul(None, None, 4, 8, 7, None) == 1
    assert lib.ns_rope_qkv(None, None, None, None, None, None, None, None, None, 4, 12, 2, 127, 1, None) == 1
    # hidden not a multiple of 16; row statistics for more than NS_NORM_ROWS (128) tokens
    assert lib.ns_embed_rope(None, None, 4, None, 10, 100, None, 64, None, None, None, None, 1, None) == 1
    assert b"hidden" in lib.ns_last_error()
    sq = ctypes.c_float()
    assert lib.ns_embed_rope(None, None, 129, None, 10, 128, None, 64, None, None, None, ctypes.byref(sq), 1, None) == 1
    assert b"128 tokens" in lib.ns_last_error()


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="missing"):
        _lib.load_library(tmp_path / "nope.so")

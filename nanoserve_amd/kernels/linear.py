"""Projection GEMMs of the decode loop: y = x @ W^T (+ b), x [M, K], W [N, K] row-major.

The one indirection point for every projection of the model (QKV, O, gate/up, down, LM head;
nanoserve/model.py:231,256-257,362). Every bf16 product runs a HIP GEMM of csrc/gemm.hip: decode-sized ones
(M <= 64) the skinny kernels, which stream each weight once and fold the neighbouring token-wise ops into
their epilogues; larger ones (prefill chunks, mixed steps, speculative verify batches) the tiled MFMA
kernel, with the SiLU epilogue fused and the residual/RMSNorm and RoPE steps in the standalone HIP
token-wise kernels. fp32 (the correctness paths) goes through torch. Every route rounds where the unfused
PyTorch ops round, so they differ only in the fp32 summation order of the products.

RMSNorm between projections is not a pass of its own on the skinny route: the projection that produces
the residual stream also writes per-16-column row sums of its square, and the projection that consumes
rms_norm(residual) normalises its input fragments as it loads them ("norm on load"). Such an input is a
NormedRows (r, row_sumsq, weight, eps); NormedRows.tensor() materialises h with the same arithmetic.

Decode-sized products (M <= 64) run on fragment-packed weights where the caller hands a PackedWeight: the
weight stored once more, at load, in the order the MFMA consumes it (csrc/packed_gemm.hip), which streams
at a far higher rate than the row-major skinny kernels. A PackedWeight keeps the row-major tensor too, for
the larger products.

Fused entry points (each with the unfused composition it equals):
  linear(x, w, b)                                   F.linear(x, w, b)
  linear_silu_mul(x, w_gate_up)                     silu_mul(F.linear(x, w_gate_up))
  linear_residual_rms_norm(x, w, residual, nw, eps) rms_norm(F.linear(x, w), nw, eps, residual=residual)
                                                    -> (h, residual + F.linear(x, w)); nw=None -> (None, sum)
  linear_rope_qkv(x, w, b, cos, sin, ...)           rope_qkv(F.linear(x, w, b), cos, sin, ...)
where x may be a tensor or a NormedRows, and h comes back as a NormedRows on the skinny route.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from nanoserve_amd import _lib
from nanoserve_amd.kernels.fused import rms_norm, rope_qkv, silu_mul

SKINNY_MAX_M = 64
TILED_MIN_M = 193   # above 192 rows every plain product runs the tiled kernel (csrc/gemm.hip T16_LARGE_M)
NORM_COLS = 16   # columns per row-sum partial of a NormedRows
NORM_ROWS = 128  # rows the row-sum buffer holds (NS_NORM_ROWS: decode batches and verify batches)

_WS: dict[int, torch.Tensor] = {}
_WS_RETIRED: list[torch.Tensor] = []   # superseded buffers stay alive: captured graphs may point at them


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _WS.get(idx)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("skinny GEMM workspace must be sized by an eager call before graph capture")
        if ws is not None:
            _WS_RETIRED.append(ws)
        # zero-filled once: the kernels' tile counters start at zero and every call leaves them there
        ws = torch.zeros(max(nbytes, 1 << 22), dtype=torch.uint8, device=device)
        _WS[idx] = ws
    return ws


class NormedRows:
    """rms_norm(r) held as r (bf16 [M, K]) plus the row statistics of r: sumsq (fp32 [ceil(K/16), NORM_ROWS],
    column m = row m, each entry the sum of r^2 over 16 columns), the norm weight [K] and eps."""

    def __init__(self, r: torch.Tensor, sumsq: torch.Tensor, weight: torch.Tensor, eps: float):
        self.r, self.sumsq, self.weight, self.eps = r, sumsq, weight, float(eps)
        self._h: torch.Tensor | None = None

    @property
    def shape(self):
        return self.r.shape

    @property
    def dtype(self):
        return self.r.dtype

    @property
    def device(self):
        return self.r.device

    def tensor(self) -> torch.Tensor:
        """h = rms_norm(r), bitwise what the GEMMs compute on load."""
        if self._h is None:
            M, K = self.r.shape
            h = torch.empty_like(self.r)
            _lib.check(_lib.lib().ns_rms_norm_apply(self.r.data_ptr(), self.sumsq.data_ptr(), self.weight.data_ptr(),
                                                    self.eps, h.data_ptr(), M, K, 1, _lib.stream_of(self.r)),
                       "rms_norm_apply")
            self._h = h
        return self._h

    def rows(self, idx: torch.Tensor) -> "NormedRows":
        """The rows idx (in that order) as a NormedRows."""
        n = idx.shape[0]
        sq = torch.zeros(self.sumsq.shape[0], NORM_ROWS, dtype=self.sumsq.dtype, device=self.sumsq.device)
        sq[:, :n] = self.sumsq[:, idx]
        from nanoserve_amd.kernels.fused import gather_rows
        return NormedRows(gather_rows(self.r, idx), sq, self.weight, self.eps)


PACK_ROWS, PACK_GATE_UP, PACK_ROPE = 0, 1, 2   # tile row orders of csrc/packed_gemm.hip


class PackedWeight:
    """A bf16 weight W [N, K] (row-major, `w`) with its fragment-packed copy (`p`, uint8) for decode-sized
    products. order: PACK_ROWS (plain, residual and LM-head projections), PACK_GATE_UP (a merged [gate; up]
    weight), PACK_ROPE (a merged QKV weight of head_dim-wide heads)."""

    def __init__(self, w: torch.Tensor, order: int = PACK_ROWS, head_dim: int = 0):
        assert w.dtype == torch.bfloat16 and w.dim() == 2 and w.is_cuda and w.is_contiguous()
        N, K = w.shape
        self.w, self.order, self.head_dim = w, order, head_dim
        nbytes = _lib.lib().ns_packed_weight_bytes(N, K, order, head_dim)
        if nbytes == 0:
            raise ValueError(f"weight {tuple(w.shape)} cannot be packed (K must be a multiple of 32)")
        self.p = torch.empty(nbytes, dtype=torch.uint8, device=w.device)
        _lib.check(_lib.lib().ns_pack_weight(w.data_ptr(), self.p.data_ptr(), N, K, order, head_dim,
                                             _lib.stream_of(w)), "pack_weight")

    @property
    def shape(self):
        return self.w.shape


_SLICED_OK = [False]   # tests switch this on to exercise the packed K-sliced plans (packed_sliced_plans())


class packed_sliced_plans:
    """Within this context, decode-sized products on a PackedWeight take the packed kernels even where
    their plan slices K (by default those go to the row-major kernels, which are faster there)."""

    def __enter__(self):
        _SLICED_OK[0] = True

    def __exit__(self, *exc):
        _SLICED_OK[0] = False


def _split(w, M: int | None = None):
    """(row-major tensor, PackedWeight or None) of a weight argument; with M, the packed copy only where its
    plan keeps K whole (a sliced plan's merge costs more than the row-major kernels' streaming)."""
    if not isinstance(w, PackedWeight):
        return w, None
    if M is not None and 1 <= M <= SKINNY_MAX_M and not _SLICED_OK[0]:
        N, K = w.w.shape
        if _lib.lib().ns_gemm_packed_sliced(M, N, K, w.order, w.head_dim) == 1:
            return w.w, None
    return w.w, w


def _pk_ws(x, pw: PackedWeight):
    M, K = x.shape
    N = pw.w.shape[0]
    ws = _workspace(x.device, _lib.lib().ns_gemm_packed_workspace_bytes(M, N, K, pw.order, pw.head_dim))
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel())


def _dense(x) -> torch.Tensor:
    return x.tensor() if isinstance(x, NormedRows) else x


def hip_ok(x, w: torch.Tensor) -> bool:
    """A product the HIP GEMMs take: bf16 on the GPU, K a multiple of 32, contiguous 16-byte aligned operands."""
    t = x.r if isinstance(x, NormedRows) else x
    M, K = t.shape
    return (t.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and t.device.type == "cuda" and M >= 1
            and K % 32 == 0 and t.is_contiguous() and w.is_contiguous() and t.data_ptr() % 16 == 0
            and w.data_ptr() % 16 == 0)


def skinny_ok(x, w: torch.Tensor) -> bool:
    """A decode-sized product (M <= 64): the skinny kernels, with norm on load and the fused epilogues."""
    return hip_ok(x, w) and x.shape[0] <= SKINNY_MAX_M


def _tiled_input(x) -> torch.Tensor:
    """The tiled kernel reads a plain tensor: a NormedRows input is materialised first."""
    x = _dense(x)
    if not (x.is_contiguous() and x.data_ptr() % 16 == 0):
        x = x.contiguous()
    return x


def _x_args(x):
    """(x pointer, x_sumsq, x_norm_w, x_eps) of a tensor or NormedRows input."""
    if isinstance(x, NormedRows):
        return x.r.data_ptr(), x.sumsq.data_ptr(), x.weight.data_ptr(), x.eps
    return x.data_ptr(), None, None, 0.0


def _ws_args(x, N: int):
    M, K = x.shape
    ws = _workspace(x.device, _lib.lib().ns_gemm_workspace_bytes(M, N, K))
    return (None, 0) if ws is None else (ws.data_ptr(), ws.numel())


def linear(x, w, b: torch.Tensor | None = None) -> torch.Tensor:
    w, pw = _split(w, x.shape[0])
    if pw is not None and skinny_ok(x, w) and w.shape[0] % 8 == 0 and (b is None or b.data_ptr() % 16 == 0):
        M, K = x.shape
        N = w.shape[0]
        y = torch.empty(M, N, device=x.device, dtype=x.dtype)
        wsp, wsn = _pk_ws(x, pw)
        xp, sq, nw, eps = _x_args(x)
        _lib.check(_lib.lib().ns_gemm_packed(xp, pw.p.data_ptr(), _lib.ptr(b), y.data_ptr(), M, N, K, 1, sq, nw, eps,
                                             wsp, wsn, _lib.stream_of(w)), "linear (packed)")
        return y
    if not hip_ok(x, w):
        return F.linear(_dense(x), w, b)
    if not skinny_ok(x, w):
        x = _tiled_input(x)
    M, K = x.shape
    N = w.shape[0]
    y = torch.empty(M, N, device=x.device, dtype=x.dtype)
    wsp, wsn = _ws_args(x, N)
    xp, sq, nw, eps = _x_args(x)
    _lib.check(_lib.lib().ns_gemm(xp, w.data_ptr(), _lib.ptr(b), y.data_ptr(), M, N, K, 1, sq, nw, eps, wsp, wsn,
                                  _lib.stream_of(w)), "linear")
    return y


def linear_argmax(x, w, tokens: torch.Tensor) -> torch.Tensor:
    """LM head with the greedy choice: returns x W^T (the logits of `linear`) and writes their row-wise argmax
    (first maximal index, NaN highest) into `tokens` (int64 [M], device or pinned host memory). One launch
    where the persistent LM-head kernel takes the shape (ns_gemm_argmax_fused), else linear + argmax_rows."""
    from nanoserve_amd.kernels.sampling import argmax_rows, argmax_workspace
    w, pw = _split(w)
    t = x.r if isinstance(x, NormedRows) else x
    M, K = t.shape
    N = w.shape[0]
    assert tokens.dtype == torch.int64 and tokens.shape == (M,) and tokens.is_contiguous()
    if pw is not None and skinny_ok(x, w) and N % 8 == 0:
        # the packed product, with the argmax fused where the plan keeps K whole; otherwise the same packed
        # product (bitwise what `linear` returns for it) and the argmax kernel after it
        ws = argmax_workspace(w.device)
        if ws is not None and _lib.lib().ns_gemm_argmax_packed_fits(M, N, K) == 1:
            y = torch.empty(M, N, device=t.device, dtype=t.dtype)
            xp, sq, nw, eps = _x_args(x)
            _lib.check(_lib.lib().ns_gemm_argmax_packed(xp, pw.p.data_ptr(), y.data_ptr(), M, N, K, 1, sq, nw, eps,
                                                        tokens.data_ptr(), ws.data_ptr(), ws.numel(),
                                                        _lib.stream_of(w)), "linear_argmax (packed)")
            return y
        y = linear(x, pw)
        argmax_rows(y, tokens)
        return y
    if hip_ok(x, w) and _lib.lib().ns_gemm_argmax_fused(M, N, K) == 1:
        ws = argmax_workspace(w.device)
        if ws is not None:
            y = torch.empty(M, N, device=t.device, dtype=t.dtype)
            xp, sq, nw, eps = _x_args(x)
            _lib.check(_lib.lib().ns_gemm_argmax(xp, w.data_ptr(), y.data_ptr(), M, N, K, 1, sq, nw, eps,
                                                 tokens.data_ptr(), ws.data_ptr(), ws.numel(), _lib.stream_of(w)),
                       "linear_argmax")
            return y
    y = linear(x, w)
    argmax_rows(y, tokens)
    return y


def linear_silu_mul(x, w_gate_up) -> torch.Tensor:
    w_gate_up, pw = _split(w_gate_up, x.shape[0])
    if pw is not None and skinny_ok(x, w_gate_up):
        M, K = x.shape
        N2 = w_gate_up.shape[0]
        out = torch.empty(M, N2 // 2, device=x.device, dtype=x.dtype)
        wsp, wsn = _pk_ws(x, pw)
        xp, sq, nw, eps = _x_args(x)
        _lib.check(_lib.lib().ns_gemm_silu_mul_packed(xp, pw.p.data_ptr(), out.data_ptr(), M, N2, K, 1, sq, nw, eps,
                                                      wsp, wsn, _lib.stream_of(w_gate_up)), "linear_silu_mul (packed)")
        return out
    if not hip_ok(x, w_gate_up):
        return silu_mul(F.linear(_dense(x), w_gate_up))
    if not skinny_ok(x, w_gate_up):
        x = _tiled_input(x)
    M, K = x.shape
    N2 = w_gate_up.shape[0]
    out = torch.empty(M, N2 // 2, device=x.device, dtype=x.dtype)
    wsp, wsn = _ws_args(x, N2)
    xp, sq, nw, eps = _x_args(x)
    _lib.check(_lib.lib().ns_gemm_silu_mul(xp, w_gate_up.data_ptr(), out.data_ptr(), M, N2, K, 1, sq, nw, eps, wsp, wsn,
                                           _lib.stream_of(w_gate_up)), "linear_silu_mul")
    return out


def linear_residual_rms_norm(x: torch.Tensor, w, residual: torch.Tensor, norm_w: torch.Tensor | None,
                             eps: float):
    """(rms_norm(residual + x W^T), residual + x W^T) with the sum rounded to the dtype; norm_w None -> (None, sum).
    x [M, K], residual [M, N]. On the skinny route the first element is a NormedRows."""
    w, pw = _split(w, x.shape[0])
    if (pw is not None and skinny_ok(x, w) and residual.is_contiguous() and w.shape[0] % 8 == 0
            and residual.data_ptr() % 16 == 0):
        M, K = x.shape
        N = w.shape[0]
        res_out = torch.empty(M, N, device=x.device, dtype=x.dtype)
        sumsq = (torch.empty(-(-N // NORM_COLS), NORM_ROWS, device=x.device, dtype=torch.float32)
                 if norm_w is not None else None)
        wsp, wsn = _pk_ws(x, pw)
        _lib.check(_lib.lib().ns_gemm_residual_norm_stats_packed(
            x.data_ptr(), pw.p.data_ptr(), residual.data_ptr(), res_out.data_ptr(), _lib.ptr(sumsq), M, N, K, 1, wsp, wsn,
            _lib.stream_of(x)), "linear_residual_rms_norm (packed)")
        if norm_w is None:
            return None, res_out
        return NormedRows(res_out, sumsq, norm_w, eps), res_out
    # above 64 rows the plain product and the RMSNorm kernel: the GEMMs' residual epilogue plus a consumer that
    # normalises on load (or the materialised norm) measured slower on verify batches than the separate pass.
    # Above 192 rows (the tiled kernel) the product's epilogue adds the residual and the norm kernel reads only
    # the sum (half the norm pass's traffic).
    if (x.shape[0] >= TILED_MIN_M and hip_ok(x, w) and residual.is_contiguous() and w.shape[0] % 8 == 0
            and residual.data_ptr() % 16 == 0 and residual.dtype == w.dtype and residual.shape == (x.shape[0], w.shape[0])):
        x = _tiled_input(x)
        M, K = x.shape
        N = w.shape[0]
        res_out = torch.empty(M, N, device=x.device, dtype=x.dtype)
        wsp, wsn = _ws_args(x, N)
        _lib.check(_lib.lib().ns_gemm_residual_norm_stats(
            x.data_ptr(), w.data_ptr(), residual.data_ptr(), res_out.data_ptr(), None, M, N, K, 1, wsp, wsn,
            _lib.stream_of(x)), "linear_residual_rms_norm (tiled)")
        if norm_w is None:
            return None, res_out
        return rms_norm(res_out, norm_w, eps), res_out
    if not skinny_ok(x, w) or not residual.is_contiguous() or w.shape[0] % 8 != 0:
        y = linear(x, w)
        if norm_w is None:
            return None, residual + y
        return rms_norm(y, norm_w, eps, residual=residual)
    M, K = x.shape
    N = w.shape[0]
    res_out = torch.empty(M, N, device=x.device, dtype=x.dtype)
    sumsq = torch.empty(-(-N // NORM_COLS), NORM_ROWS, device=x.device, dtype=torch.float32) if norm_w is not None else None
    wsp, wsn = _ws_args(x, N)
    _lib.check(_lib.lib().ns_gemm_residual_norm_stats(
        x.data_ptr(), w.data_ptr(), residual.data_ptr(), res_out.data_ptr(), _lib.ptr(sumsq), M, N, K, 1, wsp, wsn,
        _lib.stream_of(x)), "linear_residual_rms_norm")
    if norm_w is None:
        return None, res_out
    return NormedRows(res_out, sumsq, norm_w, eps), res_out


def linear_rope_qkv(x, w, b: torch.Tensor | None, cos: torch.Tensor, sin: torch.Tensor,
                    n_heads: int, n_kv_heads: int, head_dim: int, k_cache=None, v_cache=None, slots=None):
    w, pw = _split(w, x.shape[0])
    if (pw is not None and skinny_ok(x, w) and head_dim in (64, 128) and cos.is_contiguous() and sin.is_contiguous()
            and all(t is None or t.data_ptr() % 16 == 0 for t in (b, cos, sin, k_cache, v_cache))):
        M, K = x.shape
        N = w.shape[0]
        assert N == (n_heads + 2 * n_kv_heads) * head_dim and cos.shape == (M, head_dim) and sin.shape == (M, head_dim)
        if k_cache is not None:
            assert k_cache.is_contiguous() and v_cache.is_contiguous() and slots.dtype == torch.int64
            assert slots.shape == (M,) and slots.is_contiguous()
        q = torch.empty(M, n_heads, head_dim, device=x.device, dtype=x.dtype)
        k = torch.empty(M, n_kv_heads, head_dim, device=x.device, dtype=x.dtype)
        v = torch.empty_like(k)
        wsp, wsn = _pk_ws(x, pw)
        xp, sq, nw, eps = _x_args(x)
        _lib.check(_lib.lib().ns_gemm_rope_qkv_packed(
            xp, pw.p.data_ptr(), _lib.ptr(b), cos.data_ptr(), sin.data_ptr(), q.data_ptr(), k.data_ptr(),
            v.data_ptr(), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(slots) if k_cache is not None else None,
            M, K, n_heads, n_kv_heads, head_dim, 1, sq, nw, eps, wsp, wsn, _lib.stream_of(w)), "linear_rope_qkv (packed)")
        return q, k, v
    if isinstance(x, NormedRows) and x.shape[0] > SKINNY_MAX_M:
        x = _dense(x)   # 16-row token blocks would each normalise their rows again: materialise once
    fits = (hip_ok(x, w) and head_dim in (64, 128) and cos.is_contiguous() and sin.is_contiguous()
            and _lib.lib().ns_gemm_rope_qkv_fits(x.shape[0], x.shape[1], n_heads, n_kv_heads, head_dim,
                                                 int(isinstance(x, NormedRows))) == 1)
    if not fits:
        return rope_qkv(linear(x, w, b), cos, sin, n_heads, n_kv_heads, head_dim, k_cache, v_cache, slots)
    M, K = x.shape
    N = w.shape[0]
    assert N == (n_heads + 2 * n_kv_heads) * head_dim and cos.shape == (M, head_dim) and sin.shape == (M, head_dim)
    if k_cache is not None:
        assert k_cache.is_contiguous() and v_cache.is_contiguous() and slots.dtype == torch.int64
        assert slots.shape == (M,) and slots.is_contiguous()
    q = torch.empty(M, n_heads, head_dim, device=x.device, dtype=x.dtype)
    k = torch.empty(M, n_kv_heads, head_dim, device=x.device, dtype=x.dtype)
    v = torch.empty_like(k)
    wsp, wsn = _ws_args(x, N)
    xp, sq, nw, eps = _x_args(x)
    _lib.check(_lib.lib().ns_gemm_rope_qkv(
        xp, w.data_ptr(), _lib.ptr(b), cos.data_ptr(), sin.data_ptr(), q.data_ptr(), k.data_ptr(),
        v.data_ptr(), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(slots) if k_cache is not None else None,
        M, K, n_heads, n_kv_heads, head_dim, 1, sq, nw, eps, wsp, wsn, _lib.stream_of(w)), "linear_rope_qkv")
    return q, k, v
